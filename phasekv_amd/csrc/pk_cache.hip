// Decode-side lifecycle of one layer's FP16 hot window (gfx950): append the new
// token's K/V, and the lazy cooling step that moves the oldest hot tokens into
// a cold segment.
//
// Semantics follow src/phasekv/phasekv_cache.py of the reference:
//   append_hot / _append_token   phasekv_cache.py:292-301, 405-422
//   _cool_aged_tokens            phasekv_cache.py:322-340
//   _gather_kv                   phasekv_cache.py:110-114
// The cooled tokens are packed afterwards by pk_quantize_pack (the cache's
// _pack_kv, phasekv_cache.py:101-107).
#include "pk_common.h"
#include "pk_quant.h"

#include <algorithm>

#pragma clang fp contract(off)

namespace {

constexpr int kCoolThreads = 256;
constexpr int kCoolWaves = kCoolThreads / 64;
constexpr size_t kCoolStagedLds = 64 * 1024;   // dynamic LDS of the staged cooling kernel

struct HotView {
  int64_t bs, hs, ts;   // element strides of batch, kv head, token; head_dim is contiguous
};

// ---------------------------------------------------------------------------
// append: hot[b, h, position + t, :] = src[b, h, t, :] for K and V, t < count
// ---------------------------------------------------------------------------
struct SrcView {
  int64_t bs, hs, ts;   // element strides of batch, kv head, token; head_dim is contiguous
};

__global__ void __launch_bounds__(kCoolThreads)
append_hot_kernel(const uint16_t* __restrict__ ks, const uint16_t* __restrict__ vs, SrcView kv,
                  SrcView vv, uint16_t* hk, uint16_t* hv, HotView hot, int Hkv, int hd,
                  int64_t position, int64_t count, int64_t total) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / hd;
    const int c = (int)(i - row * hd);
    const int64_t bh = row / count, t = row - bh * count;
    const int64_t b = bh / Hkv, h = bh - b * Hkv;
    const int64_t dst = b * hot.bs + h * hot.hs + (position + t) * hot.ts + c;
    hk[dst] = ks[b * kv.bs + h * kv.hs + t * kv.ts + c];
    hv[dst] = vs[b * vv.bs + h * vv.hs + t * vv.ts + c];
  }
}

// One decode token's rotary embedding, fused with the window append: thread
// (row, d) with d < hd/2 rotates the pair (d, d + hd/2) of one q head or one
// kv head.  The arithmetic is the sequence of rotate_half RoPE on tensors of
// the model's dtype T (fp16 or bf16), x * cos + rotate_half(x) * sin: each
// product and the sum computed in float and rounded to T.  The results are
// then rounded to fp16 (exact for fp16; for bf16 the cast `.to(float16)` that
// feeds the fp16 cache).  q heads go to q_out [B, Hq, hd] fp16; k heads are
// rotated into the window at `position`, v heads converted and copied there.
template <bool BF16>
__device__ __forceinline__ float rope_load(uint16_t h) { return BF16 ? pk_bf2f(h) : pk_h2f(h); }

// float -> bf16, round to nearest even; NaN becomes the quiet NaN 0x7FC0, as
// torch's conversion does
__device__ __forceinline__ float round_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return __uint_as_float(0x7FC00000u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return __uint_as_float(u & 0xFFFF0000u);
}

template <bool BF16>
__device__ __forceinline__ float rope_round(float f) {
  return BF16 ? round_bf16(f) : pk_h2f(pk_f2h(f));
}

template <bool BF16>
__device__ __forceinline__ uint16_t rope_half(float x, float c, float r, float sn) {
  const float a = rope_round<BF16>(x * c);
  const float b = rope_round<BF16>(r * sn);
  return pk_f2h(rope_round<BF16>(a + b));
}

template <bool BF16>
__global__ void __launch_bounds__(256)
rope_append_kernel(const uint16_t* __restrict__ q, int64_t qsb, const uint16_t* __restrict__ k,
                   const uint16_t* __restrict__ v, int64_t kvsb, const uint16_t* __restrict__ cs,
                   const uint16_t* __restrict__ sn, int64_t csb, uint16_t* __restrict__ q_out,
                   uint16_t* hk, uint16_t* hv, HotView hot, int Hq, int Hkv, int hd,
                   int64_t position, int64_t total) {
  const int half = hd / 2;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / half;
    const int d = (int)(i - row * half);
    const int64_t b = row / (Hq + Hkv);
    const int h = (int)(row - b * (Hq + Hkv));
    const uint16_t* cr = cs + b * csb;
    const uint16_t* sr = sn + b * csb;
    const float c1 = rope_load<BF16>(cr[d]), c2 = rope_load<BF16>(cr[d + half]);
    const float s1 = rope_load<BF16>(sr[d]), s2 = rope_load<BF16>(sr[d + half]);
    if (h < Hq) {
      const uint16_t* x = q + b * qsb + (int64_t)h * hd;
      const float x1 = rope_load<BF16>(x[d]), x2 = rope_load<BF16>(x[d + half]);
      uint16_t* o = q_out + (b * Hq + h) * (int64_t)hd;
      o[d] = rope_half<BF16>(x1, c1, -x2, s1);
      o[d + half] = rope_half<BF16>(x2, c2, x1, s2);
    } else {
      const int hk_ = h - Hq;
      const int64_t src = b * kvsb + (int64_t)hk_ * hd;
      const float x1 = rope_load<BF16>(k[src + d]), x2 = rope_load<BF16>(k[src + d + half]);
      const int64_t dst = b * hot.bs + hk_ * hot.hs + position * hot.ts;
      hk[dst + d] = rope_half<BF16>(x1, c1, -x2, s1);
      hk[dst + d + half] = rope_half<BF16>(x2, c2, x1, s2);
      hv[dst + d] = BF16 ? pk_f2h(pk_bf2f(v[src + d])) : v[src + d];
      hv[dst + d + half] = BF16 ? pk_f2h(pk_bf2f(v[src + d + half])) : v[src + d + half];
    }
  }
}

// ---------------------------------------------------------------------------
// cooling: one workgroup per (b, kv head)
// ---------------------------------------------------------------------------
// The importance of hot token t is the L2 norm of its fp16 V row in float32:
// lane l of a wave sums the exact squares of channels l, l + 64, ... in that
// order, the 64 lane sums are added by the butterfly o = 32, 16, ..., 1 (every
// lane ends with the same sum), and the norm is the correctly rounded sqrt.
// A token is kept when fewer than `keep` tokens rank above it: u ranks above t
// when norm_u > norm_t, or the norms are equal and u < t (NaN ranks above every
// number, equal NaNs by position).  Kept tokens are written in position order.
__device__ __forceinline__ bool ranks_above(float nu, int u, float nt, int t) {
  const bool un = nu != nu, tn = nt != nt;
  if (un != tn) return un;
  if (un || nu == nt) return u < t;
  return nu > nt;
}

__global__ void __launch_bounds__(kCoolThreads)
cool_hot_kernel(uint16_t* hk, uint16_t* hv, HotView hot, int Hkv, int hd, int hot_len, int aged,
                int keep, uint16_t* __restrict__ ok, uint16_t* __restrict__ ov,
                int64_t* __restrict__ oidx) {
  extern __shared__ float lds_f[];
  float* norm = lds_f;                                   // [aged]
  int* sel = reinterpret_cast<int*>(norm + aged);        // [aged]: 1 if kept
  int* pos = sel + aged;                                 // [aged]: output row or -1
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t b = blockIdx.x / Hkv, h = blockIdx.x - b * Hkv;
  uint16_t* krow0 = hk + b * hot.bs + h * hot.hs;
  uint16_t* vrow0 = hv + b * hot.bs + h * hot.hs;
  if (keep < aged) {
    for (int t = wave; t < aged; t += kCoolWaves) {
      const uint16_t* v = vrow0 + t * hot.ts;
      float s = 0.f;
      for (int c = lane; c < hd; c += 64) {
        const float x = pk_h2f(v[c]);
        s = __fadd_rn(s, __fmul_rn(x, x));   // x * x is exact for an fp16 x
      }
      for (int o = 32; o >= 1; o >>= 1) s = __fadd_rn(s, __shfl_xor(s, o));
      if (lane == 0) norm[t] = __fsqrt_rn(s);
    }
    __syncthreads();
    for (int t = tid; t < aged; t += kCoolThreads) {
      const float nt = norm[t];
      int rank = 0;
      for (int u = 0; u < aged; ++u) rank += ranks_above(norm[u], u, nt, t) ? 1 : 0;
      sel[t] = rank < keep ? 1 : 0;
    }
    __syncthreads();
    // output row of a kept token: the kept tokens before it
    for (int t = tid; t < aged; t += kCoolThreads) {
      int before = 0;
      for (int u = 0; u < t; ++u) before += sel[u];
      pos[t] = sel[t] ? before : -1;
    }
  } else {
    for (int t = tid; t < aged; t += kCoolThreads) pos[t] = t;
  }
  __syncthreads();
  // gather the kept rows
  const int64_t obase = ((int64_t)b * Hkv + h) * keep;
  for (int i = tid; i < aged * hd; i += kCoolThreads) {
    const int t = i / hd, c = i - t * hd;
    const int j = pos[t];
    if (j < 0) continue;
    ok[(obase + j) * hd + c] = krow0[t * hot.ts + c];
    ov[(obase + j) * hd + c] = vrow0[t * hot.ts + c];
    if (oidx && c == 0) oidx[obase + j] = t;
  }
  __syncthreads();
  // tail shift: rows [aged, hot_len) -> [0, hot_len - aged), `aged` rows at a
  // time, so each step reads only rows that no earlier step wrote and writes
  // only rows that earlier steps have finished reading
  const int remaining = hot_len - aged;
  for (int r0 = 0; r0 < remaining; r0 += aged) {
    const int n = min(aged, remaining - r0);
    for (int i = tid; i < n * hd; i += kCoolThreads) {
      const int r = r0 + i / hd, c = i % hd;
      krow0[r * hot.ts + c] = krow0[(r + aged) * hot.ts + c];
      vrow0[r * hot.ts + c] = vrow0[(r + aged) * hot.ts + c];
    }
    __syncthreads();
  }
}

// The same cooling step with the whole window of the row staged in LDS first:
// every global read is issued at once (16-byte pieces), the norms, the ranking,
// the gather and the shift then work from LDS, and the shift has no overlap
// hazard (its sources are in LDS).  Needs head_dim, the token stride and both
// bases in whole 16-byte pieces; LDS holds 4 * hot_len * head_dim bytes plus
// 8 bytes per aged token (plus the packing statistics of the fused variant).
struct Staged {
  uint4* sk;      // [hot_len][hd / 8]
  uint4* sv;
  int* pos;       // [aged]: output row of a kept token, -1 otherwise
  char* tail;     // first free byte
};

__device__ __forceinline__ Staged stage_and_select(const uint16_t* krow0, const uint16_t* vrow0,
                                                   int64_t ts, int hd, int hot_len, int aged,
                                                   int keep, char* lds) {
  const int pr = hd / 8;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  Staged st;
  st.sk = reinterpret_cast<uint4*>(lds);
  st.sv = st.sk + hot_len * pr;
  float* norm = reinterpret_cast<float*>(st.sv + hot_len * pr);
  st.pos = reinterpret_cast<int*>(norm + aged);
  st.tail = reinterpret_cast<char*>(st.pos + aged);
  for (int i = tid; i < hot_len * pr; i += kCoolThreads) {
    const int t = i / pr, c = i - t * pr;
    st.sk[i] = *reinterpret_cast<const uint4*>(krow0 + t * ts + 8 * c);
    st.sv[i] = *reinterpret_cast<const uint4*>(vrow0 + t * ts + 8 * c);
  }
  __syncthreads();
  const uint16_t* svh = reinterpret_cast<const uint16_t*>(st.sv);
  if (keep < aged) {
    // norms: each wave takes 4 tokens at a time, their butterflies interleaved
    // (the same per-token order as the one-token loop)
    for (int t0 = wave; t0 < aged; t0 += 4 * kCoolWaves) {
      float s[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = min(t0 + j * kCoolWaves, aged - 1);
        const uint16_t* v = svh + t * hd;
        s[j] = 0.f;
        for (int c = lane; c < hd; c += 64) {
          const float x = pk_h2f(v[c]);
          s[j] = __fadd_rn(s[j], __fmul_rn(x, x));
        }
      }
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1)
#pragma unroll
        for (int j = 0; j < 4; ++j) s[j] = __fadd_rn(s[j], __shfl_xor(s[j], o));
      if (lane == 0) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (t0 + j * kCoolWaves < aged) norm[t0 + j * kCoolWaves] = __fsqrt_rn(s[j]);
      }
    }
    __syncthreads();
    // wave 0 ranks 64 tokens at a time; output rows by ballot prefix counts
    if (wave == 0) {
      int count = 0;
      for (int base = 0; base < aged; base += 64) {
        const int t = base + lane;
        bool kept = false;
        if (t < aged) {
          const float nt = norm[t];
          int rank = 0;
          for (int u = 0; u < aged; ++u) rank += ranks_above(norm[u], u, nt, t) ? 1 : 0;
          kept = rank < keep;
        }
        const uint64_t mask = __ballot(kept);
        if (t < aged) st.pos[t] = kept ? count + __popcll(mask & ((1ull << lane) - 1ull)) : -1;
        count += __popcll(mask);
      }
    }
  } else {
    for (int t = tid; t < aged; t += kCoolThreads) st.pos[t] = t;
  }
  __syncthreads();
  return st;
}

// rows [aged, hot_len) of the staged window back to rows [0, hot_len - aged)
__device__ __forceinline__ void shift_from_lds(const Staged& st, uint16_t* krow0, uint16_t* vrow0,
                                               int64_t ts, int hd, int hot_len, int aged) {
  const int pr = hd / 8;
  const int remaining = hot_len - aged;
  for (int i = threadIdx.x; i < remaining * pr; i += kCoolThreads) {
    const int r = i / pr, c = i - r * pr;
    *reinterpret_cast<uint4*>(krow0 + r * ts + 8 * c) = st.sk[i + aged * pr];
    *reinterpret_cast<uint4*>(vrow0 + r * ts + 8 * c) = st.sv[i + aged * pr];
  }
}

__global__ void __launch_bounds__(kCoolThreads)
cool_hot_staged_kernel(uint16_t* hk, uint16_t* hv, HotView hot, int Hkv, int hd, int hot_len,
                       int aged, int keep, uint16_t* __restrict__ ok, uint16_t* __restrict__ ov,
                       int64_t* __restrict__ oidx) {
  extern __shared__ __attribute__((aligned(16))) char lds_c[];
  const int64_t b = blockIdx.x / Hkv, h = blockIdx.x - b * Hkv;
  uint16_t* krow0 = hk + b * hot.bs + h * hot.hs;
  uint16_t* vrow0 = hv + b * hot.bs + h * hot.hs;
  const Staged st = stage_and_select(krow0, vrow0, hot.ts, hd, hot_len, aged, keep, lds_c);
  const int pr = hd / 8;
  const int64_t obase = ((int64_t)b * Hkv + h) * keep;
  uint4* okq = reinterpret_cast<uint4*>(ok);
  uint4* ovq = reinterpret_cast<uint4*>(ov);
  for (int i = threadIdx.x; i < aged * pr; i += kCoolThreads) {
    const int t = i / pr, c = i - t * pr;
    const int j = st.pos[t];
    if (j < 0) continue;
    okq[(obase + j) * pr + c] = st.sk[i];
    ovq[(obase + j) * pr + c] = st.sv[i];
    if (oidx && c == 0) oidx[obase + j] = t;
  }
  shift_from_lds(st, krow0, vrow0, hot.ts, hd, hot_len, aged);
}

// Outputs of the fused cooling + packing step, in the storage quantize_pack
// gives the cache's segments (phasekv_cache.py:101-107): K grouped along the
// kept tokens, codes [B*Hkv][nbk][hd] and scale / min [B*Hkv][ngk][hd] (token
// bytes and groups outermost); V grouped along head_dim, codes
// [B*Hkv*keep][nbv] and scale / min [B*Hkv*keep][ngv].
struct PackOut {
  uint8_t* kp;
  uint16_t* ks;
  uint16_t* km;
  uint8_t* vp;
  uint16_t* vs;
  uint16_t* vm;
  int bits, gsk, ngk, nbk, gsv, ngv, nbv;
};

__global__ void __launch_bounds__(kCoolThreads)
cool_pack_staged_kernel(uint16_t* hk, uint16_t* hv, HotView hot, int Hkv, int hd, int hot_len,
                        int aged, int keep, PackOut po, int64_t* __restrict__ oidx) {
  extern __shared__ __attribute__((aligned(16))) char lds_c[];
  const int tid = threadIdx.x;
  const int64_t b = blockIdx.x / Hkv, h = blockIdx.x - b * Hkv;
  const int64_t bh = (int64_t)b * Hkv + h;
  uint16_t* krow0 = hk + b * hot.bs + h * hot.hs;
  uint16_t* vrow0 = hv + b * hot.bs + h * hot.hs;
  const Staged st = stage_and_select(krow0, vrow0, hot.ts, hd, hot_len, aged, keep, lds_c);
  int* kidx = reinterpret_cast<int*>(st.tail);                      // [keep]: token of kept row
  pk::GroupStats* kst = reinterpret_cast<pk::GroupStats*>(kidx + keep + (keep & 1));  // [ngk][hd]
  pk::GroupStats* vst = kst + po.ngk * hd;                            // [keep][ngv]
  // the kept rows, dense and in output order: kk[j][c], vv[j][c]
  const int pr = hd / 8;
  uint4* kkq = reinterpret_cast<uint4*>(((reinterpret_cast<uintptr_t>(vst + keep * po.ngv)) + 15) &
                                        ~uintptr_t(15));
  uint4* vvq = kkq + keep * pr;
  for (int t = tid; t < aged; t += kCoolThreads)
    if (st.pos[t] >= 0) kidx[st.pos[t]] = t;
  __syncthreads();
  for (int i = tid; i < keep * pr; i += kCoolThreads) {
    const int j = i / pr, c = i - j * pr;
    kkq[i] = st.sk[kidx[j] * pr + c];
    vvq[i] = st.sv[kidx[j] * pr + c];
  }
  __syncthreads();
  const uint16_t* kk = reinterpret_cast<const uint16_t*>(kkq);
  const uint16_t* vv = reinterpret_cast<const uint16_t*>(vvq);
  // group statistics and the fp16 scale / min: K items (g, c) on the first threads,
  // V items (j, g) after them, in one pass
  const int nks = po.ngk * hd, nvs = keep * po.ngv;
  for (int i = tid; i < nks + nvs; i += kCoolThreads) {
    float mn, mx;
    if (i < nks) {
      const int g = i / hd, c = i - g * hd;
      const int j0 = g * po.gsk, j1 = min(j0 + po.gsk, keep);
      mn = mx = pk_h2f(kk[j0 * hd + c]);
      for (int j = j0 + 1; j < j1; ++j) {
        const float x = pk_h2f(kk[j * hd + c]);
        mn = pk::nan_min(mn, x);
        mx = pk::nan_max(mx, x);
      }
      const pk::GroupStats s = pk::group_stats_from(mn, mx, po.bits);
      kst[i] = s;
      po.ks[(bh * po.ngk + g) * hd + c] = pk_f2h(s.scale);
      po.km[(bh * po.ngk + g) * hd + c] = pk_f2h(s.mn);
    } else {
      const int iv = i - nks;
      const int j = iv / po.ngv, g = iv - j * po.ngv;
      const uint16_t* row = vv + j * hd;
      const int c0 = g * po.gsv, c1 = min(c0 + po.gsv, hd);
      mn = mx = pk_h2f(row[c0]);
      for (int c = c0 + 1; c < c1; ++c) {
        const float x = pk_h2f(row[c]);
        mn = pk::nan_min(mn, x);
        mx = pk::nan_max(mx, x);
      }
      const pk::GroupStats s = pk::group_stats_from(mn, mx, po.bits);
      vst[iv] = s;
      po.vs[(bh * keep + j) * po.ngv + g] = pk_f2h(s.scale);
      po.vm[(bh * keep + j) * po.ngv + g] = pk_f2h(s.mn);
    }
  }
  __syncthreads();
  // code bytes, LSB first, zero codes past the end of the axis: K bytes, then V bytes
  const int vpb = 8 / po.bits;
  const int nkb = po.nbk * hd, nvb = keep * po.nbv;
  for (int i = tid; i < nkb + nvb; i += kCoolThreads) {
    uint32_t x = 0;
    if (i < nkb) {
      const int byte = i / hd, c = i - byte * hd;
      for (int k = 0; k < vpb; ++k) {
        const int j = byte * vpb + k;
        if (j < keep)
          x |= pk::quant_code(pk_h2f(kk[j * hd + c]), kst[(j / po.gsk) * hd + c], po.bits)
               << (k * po.bits);
      }
      po.kp[(bh * po.nbk + byte) * hd + c] = static_cast<uint8_t>(x);
    } else {
      const int iv = i - nkb;
      const int j = iv / po.nbv, byte = iv - j * po.nbv;
      const uint16_t* row = vv + j * hd;
      for (int k = 0; k < vpb; ++k) {
        const int c = byte * vpb + k;
        if (c < hd)
          x |= pk::quant_code(pk_h2f(row[c]), vst[j * po.ngv + c / po.gsv], po.bits) << (k * po.bits);
      }
      po.vp[(bh * keep + j) * po.nbv + byte] = static_cast<uint8_t>(x);
    }
  }
  if (oidx)
    for (int j = tid; j < keep; j += kCoolThreads) oidx[bh * keep + j] = kidx[j];
  shift_from_lds(st, krow0, vrow0, hot.ts, hd, hot_len, aged);
}

// LDS bytes of the staged kernels (0 if the row does not stage)
static size_t staged_lds(int64_t hot_len, int hd, int64_t aged, int64_t keep, bool pack,
                         int64_t ngk, int64_t ngv) {
  if (hd % 8) return 0;
  size_t bytes = (size_t)4 * hot_len * hd + (size_t)8 * aged;
  if (pack)
    bytes += (size_t)4 * (keep + (keep & 1)) + sizeof(pk::GroupStats) * (ngk * hd + keep * ngv) +
             15 + (size_t)4 * keep * hd;   // kept rows, dense, 16-byte aligned
  return bytes <= kCoolStagedLds ? bytes : 0;
}

}  // namespace

// 16-byte pieces of the hot rows
static bool hot_vectors(const uint16_t* hk, const uint16_t* hv, int hd, int64_t bs, int64_t hs,
                        int64_t ts) {
  return hd % 8 == 0 && ts % 8 == 0 && bs % 8 == 0 && hs % 8 == 0 &&
         reinterpret_cast<uintptr_t>(hk) % 16 == 0 && reinterpret_cast<uintptr_t>(hv) % 16 == 0;
}

static int check_hot(const uint16_t* hk, const uint16_t* hv, int batch, int hkv, int hd,
                     int64_t hbs, int64_t hhs, int64_t hts) {
  if (!hk || !hv) return pk::fail("null hot buffer");
  if (batch <= 0 || hkv <= 0 || hd <= 0) return pk::fail("batch, num_kv_heads and head_dim must be positive");
  if (hbs < 0 || hhs < 0 || hts < hd) return pk::fail("hot strides must be non-negative with token stride >= head_dim");
  return PK_OK;
}

extern "C" int pk_append_hot(const uint16_t* k_src, const uint16_t* v_src, int64_t k_bstride,
                             int64_t k_hstride, int64_t v_bstride, int64_t v_hstride,
                             uint16_t* hot_k, uint16_t* hot_v, int64_t hot_bstride,
                             int64_t hot_hstride, int64_t hot_tstride, int batch,
                             int num_kv_heads, int head_dim, int64_t position, int64_t capacity,
                             void* stream) {
  return pk::guarded("pk_append_hot", [&]() -> int {
    pk::clear_error();
    if (int rc = check_hot(hot_k, hot_v, batch, num_kv_heads, head_dim, hot_bstride, hot_hstride,
                           hot_tstride))
      return rc;
    if (!k_src || !v_src) return pk::fail("null K/V source");
    if (position < 0 || position >= capacity) return pk::fail("hot window is full");
    const int64_t total = (int64_t)batch * num_kv_heads * head_dim;
    const int grid = (int)std::min<int64_t>(pk::cdiv(total, kCoolThreads), 4096);
    hipLaunchKernelGGL(append_hot_kernel, dim3(grid), dim3(kCoolThreads), 0,
                       static_cast<hipStream_t>(stream), k_src, v_src,
                       SrcView{k_bstride, k_hstride, 0}, SrcView{v_bstride, v_hstride, 0}, hot_k,
                       hot_v, HotView{hot_bstride, hot_hstride, hot_tstride}, num_kv_heads,
                       head_dim, position, (int64_t)1, total);
    return pk::check_launch("append_hot");
  });
}

extern "C" int pk_append_hot_rows(const uint16_t* k_src, const uint16_t* v_src, int64_t k_bstride,
                                  int64_t k_hstride, int64_t k_tstride, int64_t v_bstride,
                                  int64_t v_hstride, int64_t v_tstride, uint16_t* hot_k,
                                  uint16_t* hot_v, int64_t hot_bstride, int64_t hot_hstride,
                                  int64_t hot_tstride, int batch, int num_kv_heads, int head_dim,
                                  int64_t position, int64_t count, int64_t capacity,
                                  void* stream) {
  return pk::guarded("pk_append_hot_rows", [&]() -> int {
    pk::clear_error();
    if (int rc = check_hot(hot_k, hot_v, batch, num_kv_heads, head_dim, hot_bstride, hot_hstride,
                           hot_tstride))
      return rc;
    if (!k_src || !v_src) return pk::fail("null K/V source");
    if (count <= 0) return pk::fail("count must be positive");
    if (position < 0 || position > capacity - count)
      return pk::fail("the rows do not fit in the hot window");
    const int64_t total = (int64_t)batch * num_kv_heads * count * head_dim;
    const int grid = (int)std::min<int64_t>(pk::cdiv(total, kCoolThreads), 4096);
    hipLaunchKernelGGL(append_hot_kernel, dim3(grid), dim3(kCoolThreads), 0,
                       static_cast<hipStream_t>(stream), k_src, v_src,
                       SrcView{k_bstride, k_hstride, k_tstride},
                       SrcView{v_bstride, v_hstride, v_tstride}, hot_k, hot_v,
                       HotView{hot_bstride, hot_hstride, hot_tstride}, num_kv_heads, head_dim,
                       position, count, total);
    return pk::check_launch("append_hot_rows");
  });
}

extern "C" int pk_rope_append_hot(const uint16_t* q, int64_t q_bstride, const uint16_t* k,
                                  const uint16_t* v, int64_t kv_bstride, const uint16_t* cos,
                                  const uint16_t* sin, int64_t cs_bstride, int dtype,
                                  uint16_t* q_out,
                                  uint16_t* hot_k, uint16_t* hot_v, int64_t hot_bstride,
                                  int64_t hot_hstride, int64_t hot_tstride, int batch,
                                  int num_q_heads, int num_kv_heads, int head_dim,
                                  int64_t position, int64_t capacity, void* stream) {
  return pk::guarded("pk_rope_append_hot", [&]() -> int {
    pk::clear_error();
    if (int rc = check_hot(hot_k, hot_v, batch, num_kv_heads, head_dim, hot_bstride, hot_hstride,
                           hot_tstride))
      return rc;
    if (!q || !k || !v || !cos || !sin || !q_out) return pk::fail("null q / K / V / cos / sin / q_out");
    if (num_q_heads <= 0 || num_q_heads % num_kv_heads)
      return pk::fail("num_q_heads must be a positive multiple of num_kv_heads");
    if (head_dim % 2) return pk::fail("head_dim must be even for the rotary embedding");
    if (dtype != PK_DTYPE_F16 && dtype != PK_DTYPE_BF16)
      return pk::fail("q / K / V / cos / sin must be float16 or bfloat16");
    if (q_bstride < (int64_t)num_q_heads * head_dim || kv_bstride < (int64_t)num_kv_heads * head_dim ||
        cs_bstride < 0)
      return pk::fail("q / K / V batch strides must cover their heads; cos / sin stride >= 0");
    if (position < 0 || position >= capacity) return pk::fail("hot window is full");
    const int64_t total = (int64_t)batch * (num_q_heads + num_kv_heads) * (head_dim / 2);
    const int grid = (int)std::min<int64_t>(pk::cdiv(total, 256), 4096);
    if (dtype == PK_DTYPE_BF16)
      hipLaunchKernelGGL(rope_append_kernel<true>, dim3(grid), dim3(256), 0,
                         static_cast<hipStream_t>(stream), q, q_bstride, k, v, kv_bstride, cos, sin,
                         cs_bstride, q_out, hot_k, hot_v,
                         HotView{hot_bstride, hot_hstride, hot_tstride}, num_q_heads, num_kv_heads,
                         head_dim, position, total);
    else
      hipLaunchKernelGGL(rope_append_kernel<false>, dim3(grid), dim3(256), 0,
                         static_cast<hipStream_t>(stream), q, q_bstride, k, v, kv_bstride, cos, sin,
                         cs_bstride, q_out, hot_k, hot_v,
                         HotView{hot_bstride, hot_hstride, hot_tstride}, num_q_heads, num_kv_heads,
                         head_dim, position, total);
    return pk::check_launch("rope_append_hot");
  });
}

extern "C" int pk_cool_hot(uint16_t* hot_k, uint16_t* hot_v, int64_t hot_bstride,
                           int64_t hot_hstride, int64_t hot_tstride, int batch, int num_kv_heads,
                           int head_dim, int64_t hot_len, int64_t aged, int64_t keep,
                           uint16_t* out_k, uint16_t* out_v, int64_t* out_index, void* stream) {
  return pk::guarded("pk_cool_hot", [&]() -> int {
    pk::clear_error();
    if (int rc = check_hot(hot_k, hot_v, batch, num_kv_heads, head_dim, hot_bstride, hot_hstride,
                           hot_tstride))
      return rc;
    if (aged <= 0 || aged > hot_len) return pk::fail("aged must be in [1, hot_len]");
    if (aged > PK_COOL_MAX_AGED) return pk::fail("aged above PK_COOL_MAX_AGED");
    if (keep <= 0 || keep > aged) return pk::fail("keep must be in [1, aged]");
    if (!out_k || !out_v) return pk::fail("null output buffer");
    const size_t meta = (size_t)aged * (sizeof(float) + 2 * sizeof(int));
    const size_t staged = staged_lds(hot_len, head_dim, aged, keep, false, 0, 0);
    const bool vec = hot_vectors(hot_k, hot_v, head_dim, hot_bstride, hot_hstride, hot_tstride) &&
                     reinterpret_cast<uintptr_t>(out_k) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(out_v) % 16 == 0;
    if (vec && staged) {
      hipLaunchKernelGGL(cool_hot_staged_kernel, dim3(batch * num_kv_heads), dim3(kCoolThreads),
                         staged, static_cast<hipStream_t>(stream), hot_k, hot_v,
                         HotView{hot_bstride, hot_hstride, hot_tstride}, num_kv_heads, head_dim,
                         (int)hot_len, (int)aged, (int)keep, out_k, out_v, out_index);
      return pk::check_launch("cool_hot");
    }
    const size_t lds = meta;
    hipLaunchKernelGGL(cool_hot_kernel, dim3(batch * num_kv_heads), dim3(kCoolThreads), lds,
                       static_cast<hipStream_t>(stream), hot_k, hot_v,
                       HotView{hot_bstride, hot_hstride, hot_tstride}, num_kv_heads, head_dim,
                       (int)hot_len, (int)aged, (int)keep, out_k, out_v, out_index);
    return pk::check_launch("cool_hot");
  });
}

extern "C" int pk_cool_pack_supported(int64_t hot_len, int head_dim, int64_t aged, int64_t keep,
                                      int group_size) {
  return pk::guarded("pk_cool_pack_supported", [&]() -> int {
    if (hot_len <= 0 || head_dim <= 0 || aged <= 0 || aged > hot_len || keep <= 0 || keep > aged ||
        group_size <= 0)
      return 0;
    const int64_t ngk = pk::cdiv(keep, std::min<int64_t>(group_size, keep));
    const int64_t ngv = pk::cdiv(head_dim, std::min<int64_t>(group_size, head_dim));
    return staged_lds(hot_len, head_dim, aged, keep, true, ngk, ngv) ? 1 : 0;
  });
}

extern "C" int pk_cool_pack_hot(uint16_t* hot_k, uint16_t* hot_v, int64_t hot_bstride,
                                int64_t hot_hstride, int64_t hot_tstride, int batch,
                                int num_kv_heads, int head_dim, int64_t hot_len, int64_t aged,
                                int64_t keep, int bits, int group_size, uint8_t* k_packed,
                                uint16_t* k_scale, uint16_t* k_mins, uint8_t* v_packed,
                                uint16_t* v_scale, uint16_t* v_mins, int64_t* out_index,
                                void* stream) {
  return pk::guarded("pk_cool_pack_hot", [&]() -> int {
    pk::clear_error();
    if (int rc = check_hot(hot_k, hot_v, batch, num_kv_heads, head_dim, hot_bstride, hot_hstride,
                           hot_tstride))
      return rc;
    if (aged <= 0 || aged > hot_len) return pk::fail("aged must be in [1, hot_len]");
    if (keep <= 0 || keep > aged) return pk::fail("keep must be in [1, aged]");
    if (!pk::valid_bits(bits)) return pk::fail("bits must be one of (2, 4, 8)");
    if (group_size <= 0) return pk::fail("group_size must be positive");
    if (!k_packed || !k_scale || !k_mins || !v_packed || !v_scale || !v_mins)
      return pk::fail("null output buffer");
    if (!pk_cool_pack_supported(hot_len, head_dim, aged, keep, group_size) ||
        !hot_vectors(hot_k, hot_v, head_dim, hot_bstride, hot_hstride, hot_tstride))
      return pk::fail("this window does not fit the fused cooling step "
                      "(use pk_cool_hot and pk_quantize_pack)");
    PackOut po;
    po.kp = k_packed; po.ks = k_scale; po.km = k_mins;
    po.vp = v_packed; po.vs = v_scale; po.vm = v_mins;
    po.bits = bits;
    const int vpb = 8 / bits;
    po.gsk = (int)std::min<int64_t>(group_size, keep);
    po.ngk = (int)pk::cdiv(keep, po.gsk);
    po.nbk = (int)pk::cdiv(keep, vpb);
    po.gsv = std::min(group_size, head_dim);
    po.ngv = (int)pk::cdiv(head_dim, po.gsv);
    po.nbv = (int)pk::cdiv(head_dim, vpb);
    const size_t lds = staged_lds(hot_len, head_dim, aged, keep, true, po.ngk, po.ngv);
    hipLaunchKernelGGL(cool_pack_staged_kernel, dim3(batch * num_kv_heads), dim3(kCoolThreads),
                       lds, static_cast<hipStream_t>(stream), hot_k, hot_v,
                       HotView{hot_bstride, hot_hstride, hot_tstride}, num_kv_heads, head_dim,
                       (int)hot_len, (int)aged, (int)keep, po, out_index);
    return pk::check_launch("cool_pack_hot");
  });
}
