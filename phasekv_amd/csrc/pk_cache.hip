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

#include <algorithm>

#pragma clang fp contract(off)

namespace {

constexpr int kCoolThreads = 256;
constexpr int kCoolWaves = kCoolThreads / 64;

struct HotView {
  int64_t bs, hs, ts;   // element strides of batch, kv head, token; head_dim is contiguous
};

// ---------------------------------------------------------------------------
// append: hot[b, h, position, :] = src[b, h, 0, :] for K and V
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(kCoolThreads)
append_hot_kernel(const uint16_t* __restrict__ ks, const uint16_t* __restrict__ vs,
                  int64_t ksb, int64_t ksh, int64_t vsb, int64_t vsh, uint16_t* hk, uint16_t* hv,
                  HotView hot, int Hkv, int hd, int64_t position, int64_t total) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i / hd;
    const int c = (int)(i - row * hd);
    const int64_t b = row / Hkv, h = row - b * Hkv;
    const int64_t dst = b * hot.bs + h * hot.hs + position * hot.ts + c;
    hk[dst] = ks[b * ksb + h * ksh + c];
    hv[dst] = vs[b * vsb + h * vsh + c];
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

}  // namespace

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
  pk::clear_error();
  if (int rc = check_hot(hot_k, hot_v, batch, num_kv_heads, head_dim, hot_bstride, hot_hstride,
                         hot_tstride))
    return rc;
  if (!k_src || !v_src) return pk::fail("null K/V source");
  if (position < 0 || position >= capacity) return pk::fail("hot window is full");
  const int64_t total = (int64_t)batch * num_kv_heads * head_dim;
  const int grid = (int)std::min<int64_t>(pk::cdiv(total, kCoolThreads), 4096);
  hipLaunchKernelGGL(append_hot_kernel, dim3(grid), dim3(kCoolThreads), 0,
                     static_cast<hipStream_t>(stream), k_src, v_src, k_bstride, k_hstride,
                     v_bstride, v_hstride, hot_k, hot_v,
                     HotView{hot_bstride, hot_hstride, hot_tstride}, num_kv_heads, head_dim,
                     position, total);
  return pk::check_launch("append_hot");
}

extern "C" int pk_cool_hot(uint16_t* hot_k, uint16_t* hot_v, int64_t hot_bstride,
                           int64_t hot_hstride, int64_t hot_tstride, int batch, int num_kv_heads,
                           int head_dim, int64_t hot_len, int64_t aged, int64_t keep,
                           uint16_t* out_k, uint16_t* out_v, int64_t* out_index, void* stream) {
  pk::clear_error();
  if (int rc = check_hot(hot_k, hot_v, batch, num_kv_heads, head_dim, hot_bstride, hot_hstride,
                         hot_tstride))
    return rc;
  if (aged <= 0 || aged > hot_len) return pk::fail("aged must be in [1, hot_len]");
  if (aged > PK_COOL_MAX_AGED) return pk::fail("aged above PK_COOL_MAX_AGED");
  if (keep <= 0 || keep > aged) return pk::fail("keep must be in [1, aged]");
  if (!out_k || !out_v) return pk::fail("null output buffer");
  const size_t lds = (size_t)aged * (sizeof(float) + 2 * sizeof(int));
  hipLaunchKernelGGL(cool_hot_kernel, dim3(batch * num_kv_heads), dim3(kCoolThreads), lds,
                     static_cast<hipStream_t>(stream), hot_k, hot_v,
                     HotView{hot_bstride, hot_hstride, hot_tstride}, num_kv_heads, head_dim,
                     (int)hot_len, (int)aged, (int)keep, out_k, out_v, out_index);
  return pk::check_launch("cool_hot");
}
