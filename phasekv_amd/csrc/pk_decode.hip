// Split-K mixed-precision decode attention over the PhaseKV tiers (gfx950).
//
// One launch covers a list of segments (packed KIVI prompt / prompt-extension /
// cold segments, legacy per-token packed segments and the FP16 hot window).
// Each workgroup owns one (batch row, kv head, head slab, token chunk) and
// computes the softmax partial (m, l, acc) of every query head of its GQA group
// from a single read of the chunk's K/V bytes.  A log-sum-exp combine merges the
// partials of all chunks of all segments.
//
// Reference semantics (paths relative to the reference checkout):
//   per-segment kernel    src/phasekv/kernels/attention_triton.py:514-596
//   split reduce / merge  src/phasekv/kernels/attention_triton.py:257-266, 300-307
//   FP16 hot partial      src/phasekv/kernels/attention_triton.py:285-297
//   legacy per-token K/V  src/phasekv/kernels/attention_triton.py:24-92, 145-213
//   entry point           src/phasekv/kernels/attention_triton.py:643-669
#include "pk_common.h"
#include "pk_decode.h"

#include <math.h>

#include <stdlib.h>

#include <algorithm>
#include <mutex>
#include <vector>

namespace pk {

// ---------------------------------------------------------------------------
// tile loaders of the generic kernel: dequantize one (token, channel) element
// ---------------------------------------------------------------------------
__device__ __forceinline__ float kivi_k_elem(const SegDev& s, int64_t kd_off, int64_t km_off,
                                             int tok, int d) {
  const int vpb = 8 / s.kbits;
  const int64_t row_bytes = (s.length + vpb - 1) / vpb;
  const int64_t row_groups = (s.length + s.kgs - 1) / s.kgs;
  const uint32_t byte = s.kd[kd_off + (s.kdata_tm ? (int64_t)(tok / vpb) * s.hd_meta + d
                                                 : d * row_bytes + tok / vpb)];
  const uint32_t code = (byte >> ((tok % vpb) * s.kbits)) & ((1u << s.kbits) - 1u);
  const int64_t g = s.kmeta_gm ? (int64_t)(tok / s.kgs) * s.hd_meta + d : d * row_groups + tok / s.kgs;
  return static_cast<float>(code) * pk_h2f(s.ks[km_off + g]) + pk_h2f(s.km[km_off + g]);
}

// Per-token packed element (V of every packed segment, K of legacy segments).
__device__ __forceinline__ float token_elem(const uint8_t* data, const uint16_t* sc,
                                            const uint16_t* mn, int bits, int gs, int hd,
                                            int64_t d_off, int64_t m_off, int tok, int d) {
  const int vpb = 8 / bits;
  const int row_bytes = (hd + vpb - 1) / vpb;
  const int row_groups = (hd + gs - 1) / gs;
  const uint32_t byte = data[d_off + (int64_t)tok * row_bytes + d / vpb];
  const uint32_t code = (byte >> ((d % vpb) * bits)) & ((1u << bits) - 1u);
  const int64_t g = (int64_t)tok * row_groups + d / gs;
  return static_cast<float>(code) * pk_h2f(sc[m_off + g]) + pk_h2f(mn[m_off + g]);
}

// ---------------------------------------------------------------------------
// generic partial kernel (any power-of-two hd <= 256, any bits / group sizes)
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(kThreads)
decode_partials_generic(const DecodeParams p) {
  extern __shared__ float lds[];
  const int tid = threadIdx.x;
  const int hd = p.hd;
  const int T = p.tile;
  const int HS = p.HS;
  float* q_s = lds;                       // [HS][hd]
  float* acc_s = q_s + HS * hd;           // [HS][hd]
  float* k_s = acc_s + HS * hd;           // [T][hd+1]
  float* v_s = k_s + T * (hd + 1);        // [T][hd+1]
  float* p_s = v_s + T * (hd + 1);        // [HS][T]
  float* m_s = p_s + HS * T;              // [HS]
  float* l_s = m_s + HS;                  // [HS]
  float* a_s = l_s + HS;                  // [HS]

  const Block3 blk = xcd_block();
  const int b = blk.z;
  const int kvh = blk.y / p.nslab;
  const int slab = blk.y - kvh * p.nslab;
  const int h0 = kvh * p.G + slab * HS;
  const int nh = min(HS, p.G - slab * HS);

  int si = 0;
  while (si + 1 < p.nseg && blk.x >= p.seg[si + 1].lbegin) ++si;
  const SegDev& s = p.seg[si];
  const int local = blk.x - s.lbegin;
  const int cg = s.gbegin + local;
  int len_b = s.length;
  if (s.seq_lens) len_b = min(len_b, s.seq_lens[b]);
  const int t_begin = local * s.chunk_len;
  const int t_end = min(t_begin + s.chunk_len, len_b);

  for (int i = tid; i < nh * hd; i += kThreads) {
    const int h = i / hd, d = i - h * hd;
    q_s[i] = pk_h2f(p.q[b * p.q_bs + (int64_t)(h0 + h) * p.q_hs + d]);
    acc_s[i] = 0.f;
  }
  for (int h = tid; h < nh; h += kThreads) { m_s[h] = -INFINITY; l_s[h] = 0.f; }

  const int64_t kd_off = b * s.kd_bs + kvh * s.kd_hs;
  const int64_t km_off = b * s.km_bs + kvh * s.km_hs;
  const int64_t vd_off = b * s.vd_bs + kvh * s.vd_hs;
  const int64_t vm_off = b * s.vm_bs + kvh * s.vm_hs;
  __syncthreads();

  for (int t0 = t_begin; t0 < t_end; t0 += T) {
    const int nt = min(T, t_end - t0);
    // ---- dequantize the K/V tile into LDS (fp32) ----
    if (s.kind == PK_SEG_KIVI) {
      for (int i = tid; i < T * hd; i += kThreads) {
        const int d = i / T, t = i - d * T;          // tokens fastest: one channel row
        k_s[t * (hd + 1) + d] = (t < nt) ? kivi_k_elem(s, kd_off, km_off, t0 + t, d) : 0.f;
      }
    } else if (s.kind == PK_SEG_TOKEN) {
      for (int i = tid; i < T * hd; i += kThreads) {
        const int t = i / hd, d = i - t * hd;
        k_s[t * (hd + 1) + d] = (t < nt) ? token_elem(s.kd, s.ks, s.km, s.kbits, s.kgs, hd, kd_off,
                                                      km_off, t0 + t, d) : 0.f;
      }
    } else {
      const uint16_t* kh = reinterpret_cast<const uint16_t*>(s.kd);
      for (int i = tid; i < T * hd; i += kThreads) {
        const int t = i / hd, d = i - t * hd;
        k_s[t * (hd + 1) + d] = (t < nt) ? pk_h2f(kh[kd_off + (int64_t)(t0 + t) * s.tok_stride + d]) : 0.f;
      }
    }
    if (s.kind == PK_SEG_FP16) {
      const uint16_t* vh = reinterpret_cast<const uint16_t*>(s.vd);
      for (int i = tid; i < T * hd; i += kThreads) {
        const int t = i / hd, d = i - t * hd;
        v_s[t * (hd + 1) + d] = (t < nt) ? pk_h2f(vh[vd_off + (int64_t)(t0 + t) * s.tok_stride + d]) : 0.f;
      }
    } else {
      for (int i = tid; i < T * hd; i += kThreads) {
        const int t = i / hd, d = i - t * hd;
        v_s[t * (hd + 1) + d] = (t < nt) ? token_elem(s.vd, s.vs, s.vm, s.vbits, s.vgs, hd, vd_off,
                                                      vm_off, t0 + t, d) : 0.f;
      }
    }
    __syncthreads();
    // ---- scores ----
    for (int i = tid; i < nh * T; i += kThreads) {
      const int h = i / T, t = i - h * T;
      float sc = -INFINITY;
      if (t < nt) {
        const float* qr = q_s + h * hd;
        const float* kr = k_s + t * (hd + 1);
        float dot = 0.f;
        for (int d = 0; d < hd; ++d) dot += qr[d] * kr[d];
        sc = dot * p.scale;
      }
      p_s[i] = sc;
    }
    __syncthreads();
    // ---- online softmax (one thread per head) ----
    for (int h = tid; h < nh; h += kThreads) {
      float* pr = p_s + h * T;
      float mt = -INFINITY;
      for (int t = 0; t < nt; ++t) mt = fmaxf(mt, pr[t]);
      const float m_old = m_s[h];
      const float m_new = fmaxf(m_old, mt);
      const float alpha = (m_old == -INFINITY) ? 0.f : __expf(m_old - m_new);
      float sum = 0.f;
      for (int t = 0; t < T; ++t) {
        const float e = (t < nt) ? __expf(pr[t] - m_new) : 0.f;
        pr[t] = e;
        sum += e;
      }
      l_s[h] = l_s[h] * alpha + sum;
      m_s[h] = m_new;
      a_s[h] = alpha;
    }
    __syncthreads();
    // ---- P V ----
    for (int i = tid; i < nh * hd; i += kThreads) {
      const int h = i / hd, d = i - h * hd;
      const float* pr = p_s + h * T;
      float a = acc_s[i] * a_s[h];
      for (int t = 0; t < nt; ++t) a += pr[t] * v_s[t * (hd + 1) + d];
      acc_s[i] = a;
    }
    __syncthreads();
  }

  // ---- write the partial of every head of the slab ----
  for (int i = tid; i < nh * hd; i += kThreads) {
    const int h = i / hd, d = i - h * hd;
    const int64_t row = (int64_t)b * p.Hq + h0 + h;
    p.ws_acc[(row * p.C + cg) * hd + d] = acc_s[i];
  }
  for (int h = tid; h < nh; h += kThreads) {
    const int64_t row = (int64_t)b * p.Hq + h0 + h;
    p.ws_m[row * p.C + cg] = m_s[h];
    p.ws_l[row * p.C + cg] = l_s[h];
  }
}

// Log-sum-exp merge of the C partials of each output row
// (attention_triton.py:257-266, 300-307).  Three kernels share the contract; the
// host picks by C and the row count (combine_rows_kernel for C <= 8 over many rows,
// combine_wave_kernel for the other C <= 128, this one for longer rows, head_dims
// below 16 and buffers not 16-byte aligned).
// A workgroup owns one row and a slice of hs channels (16 <= hs <= 64, chosen by
// the host from C: many partials per row give narrow slices, so a batch-1 decode
// still spreads over rows * hd / 16 workgroups).  Thread (cs, d) owns channel d of partials cs, cs + ncs, ...
// (ncs = 256 / hs): it loads m, l and acc of up to kCombineLoads of them at
// once, so a pass is one memory round trip.  The
// row maximum is a wave shuffle reduction plus one LDS exchange between the
// four waves; the sums over cs are the same, once, at the end.
__device__ inline float wave_max_over(float v, int from) {
  for (int o = from; o < 64; o <<= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}
__device__ inline float wave_sum_over(float v, int from) {
  for (int o = from; o < 64; o <<= 1) v += __shfl_xor(v, o);
  return v;
}

__global__ void __launch_bounds__(kThreads)
combine_kernel(const float* __restrict__ m, const float* __restrict__ l,
               const float* __restrict__ acc, int C, int hd, int hs, uint16_t* out, float* om,
               float* ol, float* oacc) {
  __shared__ float xch[kThreads / 64][65];   // [wave][channel], [wave][64] = l
  const int tid = threadIdx.x, wave = tid / 64;
  const int nsl = hd / hs;
  const int wg = xcd_block().x;               // slices of one row share cache lines
  const int64_t row = wg / nsl;
  const int d = (wg % nsl) * hs + tid % hs;
  const int ncs = kThreads / hs, cs = tid / hs;
  const float* mr = m + row * C;
  const float* lr = l + row * C;
  const float* ar = acc + row * (int64_t)C * hd + d;
  float M = -INFINITY, sum = 0.f, ls = 0.f;
  for (int base = 0; base < C; base += kCombineLoads * ncs) {
    float a[kCombineLoads], mk[kCombineLoads], lk[kCombineLoads];
#pragma unroll
    for (int k = 0; k < kCombineLoads; ++k) {
      const int c = base + cs + k * ncs;
      const bool ok = c < C;
      a[k] = ok ? ar[(int64_t)c * hd] : 0.f;
      mk[k] = ok ? mr[c] : -INFINITY;
      lk[k] = ok ? lr[c] : 0.f;
    }
    float mx = mk[0];
#pragma unroll
    for (int k = 1; k < kCombineLoads; ++k) mx = fmaxf(mx, mk[k]);
    mx = wave_max_over(mx, hs);
    if ((tid & 63) == 0) xch[wave][0] = mx;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) mx = fmaxf(mx, xch[w][0]);
    __syncthreads();
    const float Mn = fmaxf(M, mx);
    if (Mn != -INFINITY) {
      const float so = (M == -INFINITY) ? 0.f : expf(M - Mn);
      sum *= so;
      ls *= so;
#pragma unroll
      for (int k = 0; k < kCombineLoads; ++k) {
        const float w = (mk[k] == -INFINITY) ? 0.f : expf(mk[k] - Mn);
        sum += w * a[k];
        ls += w * lk[k];
      }
      M = Mn;
    }
  }
  // every lane of one cs holds the same ls: sum over cs lanes, then over waves
  sum = wave_sum_over(sum, hs);
  ls = wave_sum_over(ls, hs);
  if ((tid & 63) < hs) xch[wave][tid & 63] = sum;
  if ((tid & 63) == 0) xch[wave][64] = ls;
  __syncthreads();
  if (tid < hs) {
    float S = 0.f, L = 0.f;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) {
      S += xch[w][tid];
      L += xch[w][64];
    }
    if (out) out[row * hd + d] = pk_f2h(S / L);
    if (oacc) oacc[row * hd + d] = S;
    if (om && d == 0) {
      om[row] = M;
      ol[row] = L;
    }
  }
}

// The same merge for many rows with few partials (C <= kCombineLoads: the
// batched decodes, hundreds of rows of eight partials, and the input-chunk
// attention, thousands of rows of two to four).  There a workgroup per row slice is thousands of short
// workgroups, each a load, two barriers and a store, and the launch is bound by
// the rate at which waves start, not by the bytes.  Here one thread owns four
// channels of one row and holds every partial of the row in registers: one
// round trip, no barrier, one float4 load per partial.
__global__ void __launch_bounds__(kCombineRowsThreads)
combine_rows_kernel(const float* __restrict__ m, const float* __restrict__ l,
                    const float* __restrict__ acc, int64_t rows, int C, int hd,
                    uint16_t* out, float* om, float* ol, float* oacc) {
  const int quads = hd / 4;
  const int64_t t = (int64_t)blockIdx.x * kCombineRowsThreads + threadIdx.x;
  const int64_t row = t / quads;
  if (row >= rows) return;
  const int d = (int)(t % quads) * 4;
  const float* mr = m + row * C;
  const float* lr = l + row * C;
  const float* ar = acc + row * (int64_t)C * hd + d;
  float4 a[kCombineLoads];
  float mk[kCombineLoads], lk[kCombineLoads];
#pragma unroll
  for (int k = 0; k < kCombineLoads; ++k) {
    const bool ok = k < C;
    a[k] = ok ? *reinterpret_cast<const float4*>(ar + (int64_t)k * hd) : make_float4(0, 0, 0, 0);
    mk[k] = ok ? mr[k] : -INFINITY;
    lk[k] = ok ? lr[k] : 0.f;
  }
  float M = mk[0];
#pragma unroll
  for (int k = 1; k < kCombineLoads; ++k) M = fmaxf(M, mk[k]);
  float4 S = make_float4(0, 0, 0, 0);
  float L = 0.f;
  if (M != -INFINITY) {
#pragma unroll
    for (int k = 0; k < kCombineLoads; ++k) {
      const float w = (mk[k] == -INFINITY) ? 0.f : expf(mk[k] - M);
      S.x += w * a[k].x;
      S.y += w * a[k].y;
      S.z += w * a[k].z;
      S.w += w * a[k].w;
      L += w * lk[k];
    }
  }
  const int64_t o = row * hd + d;
  if (out) {
    out[o] = pk_f2h(S.x / L);
    out[o + 1] = pk_f2h(S.y / L);
    out[o + 2] = pk_f2h(S.z / L);
    out[o + 3] = pk_f2h(S.w / L);
  }
  if (oacc) *reinterpret_cast<float4*>(oacc + o) = S;
  if (om && d == 0) {
    om[row] = M;
    ol[row] = L;
  }
}

// Sum / maximum over the 16 lanes of a wave that share lane & 3, all in the VALU:
// DPP rotations by 8 and 4 within each 16-lane row, then permlane swaps across the
// four rows (no trip through the LDS crossbar).
__device__ __forceinline__ float dpp_ror(float v, int ctrl_sel) {
  return ctrl_sel == 8
             ? __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false))
             : __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xF, 0xF, false));
}
__device__ __forceinline__ float quad_column_sum(float v) {
  v += dpp_ror(v, 8);
  v += dpp_ror(v, 4);
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
__device__ __forceinline__ float quad_column_max(float v) {
  v = fmaxf(v, dpp_ror(v, 8));
  v = fmaxf(v, dpp_ror(v, 4));
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// The merge for few rows of more partials (8 < C <= 16 * NL: the batch-1 decodes,
// 28 rows of 35 partials at C2).  One wave per (row, 16 channels): lane (cs, q)
// holds channels 4q .. 4q + 3 of partials cs, cs + 16, ..., so the row maximum
// and the sums are two DPP rotations and two permlane swaps each, with no LDS and
// no barrier.
template <int NL>
__global__ void __launch_bounds__(64)
combine_wave_kernel(const float* __restrict__ m, const float* __restrict__ l,
                    const float* __restrict__ acc, int64_t rows, int C, int hd,
                    uint16_t* out, float* om, float* ol, float* oacc) {
  const int lane = threadIdx.x;
  const int nsl = hd / 16;
  const int bx = xcd_block().x;              // a row's slices share lines: one XCD's L2
  const int64_t row = bx / nsl;
  if (row >= rows) return;
  const int slice = bx % nsl;
  const int q = lane & 3, cs = lane >> 2;
  const int d = slice * 16 + q * 4;
  const float* mr = m + row * C;
  const float* lr = l + row * C;
  const float* ar = acc + row * (int64_t)C * hd + d;
  float4 a[NL];
  float mk[NL], lk[NL];
#pragma unroll
  for (int k = 0; k < NL; ++k) {
    const int c = cs + 16 * k;
    const bool ok = c < C;
    a[k] = ok ? *reinterpret_cast<const float4*>(ar + (int64_t)c * hd) : make_float4(0, 0, 0, 0);
    mk[k] = ok ? mr[c] : -INFINITY;
    lk[k] = ok ? lr[c] : 0.f;
  }
  float M = mk[0];
#pragma unroll
  for (int k = 1; k < NL; ++k) M = fmaxf(M, mk[k]);
  M = quad_column_max(M);
  float4 S = make_float4(0, 0, 0, 0);
  float L = 0.f;
  if (M != -INFINITY) {
#pragma unroll
    for (int k = 0; k < NL; ++k) {
      const float w = (mk[k] == -INFINITY) ? 0.f : expf(mk[k] - M);
      S.x += w * a[k].x;
      S.y += w * a[k].y;
      S.z += w * a[k].z;
      S.w += w * a[k].w;
      L += w * lk[k];
    }
  }
  S.x = quad_column_sum(S.x);
  S.y = quad_column_sum(S.y);
  S.z = quad_column_sum(S.z);
  S.w = quad_column_sum(S.w);
  L = quad_column_sum(L);
  if (cs != 0) return;
  const int64_t o = row * hd + d;
  if (out) {
    out[o] = pk_f2h(S.x / L);
    out[o + 1] = pk_f2h(S.y / L);
    out[o + 2] = pk_f2h(S.z / L);
    out[o + 3] = pk_f2h(S.w / L);
  }
  if (oacc) *reinterpret_cast<float4*>(oacc + o) = S;
  if (om && d == 0) {
    om[row] = M;
    ol[row] = L;
  }
}

// The merge over several sets of partials whose rows are numbered differently:
// output row (o, i) takes row o * so + i * si of every set.  One thread owns
// four channels of one output row and folds the partials in, kCombineLoads at a
// time, with the running maximum rescaled as in combine_kernel.
struct PartialSetDev {
  const float* m;
  const float* l;
  const float* acc;
  int64_t so, si;
  int n;
};
struct PartialSets {
  PartialSetDev s[PK_MAX_PARTIAL_SETS];
  int nsets;
};

__global__ void __launch_bounds__(kCombineRowsThreads)
combine_sets_kernel(const PartialSets ps, int64_t outer, int64_t inner, int hd, uint16_t* out,
                    float* om, float* ol, float* oacc) {
  const int quads = hd / 4;
  const int64_t t = (int64_t)blockIdx.x * kCombineRowsThreads + threadIdx.x;
  const int64_t row = t / quads;
  if (row >= outer * inner) return;
  const int d = (int)(t % quads) * 4;
  const int64_t o = row / inner, i = row - o * inner;
  float M = -INFINITY, L = 0.f;
  float4 S = make_float4(0, 0, 0, 0);
  for (int k = 0; k < ps.nsets; ++k) {
    const PartialSetDev& st = ps.s[k];
    const int64_t r = o * st.so + i * st.si;
    const float* mr = st.m + r * st.n;
    const float* lr = st.l + r * st.n;
    const float* ar = st.acc + r * (int64_t)st.n * hd + d;
    for (int base = 0; base < st.n; base += kCombineLoads) {
      float4 a[kCombineLoads];
      float mk[kCombineLoads], lk[kCombineLoads];
#pragma unroll
      for (int j = 0; j < kCombineLoads; ++j) {
        const int c = base + j;
        const bool ok = c < st.n;
        a[j] = ok ? *reinterpret_cast<const float4*>(ar + (int64_t)c * hd)
                  : make_float4(0, 0, 0, 0);
        mk[j] = ok ? mr[c] : -INFINITY;
        lk[j] = ok ? lr[c] : 0.f;
      }
      float mx = mk[0];
#pragma unroll
      for (int j = 1; j < kCombineLoads; ++j) mx = fmaxf(mx, mk[j]);
      const float Mn = fmaxf(M, mx);
      if (Mn == -INFINITY) continue;
      const float so = (M == -INFINITY) ? 0.f : expf(M - Mn);
      S.x *= so;
      S.y *= so;
      S.z *= so;
      S.w *= so;
      L *= so;
#pragma unroll
      for (int j = 0; j < kCombineLoads; ++j) {
        const float w = (mk[j] == -INFINITY) ? 0.f : expf(mk[j] - Mn);
        S.x += w * a[j].x;
        S.y += w * a[j].y;
        S.z += w * a[j].z;
        S.w += w * a[j].w;
        L += w * lk[j];
      }
      M = Mn;
    }
  }
  const int64_t off = row * hd + d;
  if (out) {
    out[off] = pk_f2h(S.x / L);
    out[off + 1] = pk_f2h(S.y / L);
    out[off + 2] = pk_f2h(S.z / L);
    out[off + 3] = pk_f2h(S.w / L);
  }
  if (oacc) *reinterpret_cast<float4*>(oacc + off) = S;
  if (om && d == 0) {
    om[row] = M;
    ol[row] = L;
  }
}

// ---------------------------------------------------------------------------
// host-side planning
// ---------------------------------------------------------------------------
// Query heads per workgroup: q and acc of the slab stay within 2048 floats of
// LDS each and at most 32 heads, so the generic kernel's LDS stays below 64 KB.
static int head_slab(int G, int hd) { return std::min(G, std::min(32, std::max(1, 2048 / hd))); }

static int validate_problem(const pk_decode_problem* p) {
  if (!p) return fail("null problem");
  if (p->batch <= 0 || p->num_q_heads <= 0 || p->num_kv_heads <= 0 || p->head_dim <= 0)
    return fail("batch, heads and head_dim must be positive");
  if (p->num_q_heads % p->num_kv_heads)
    return fail("num_q_heads must be a multiple of num_kv_heads");
  const int hd = p->head_dim;
  if (hd & (hd - 1)) return fail("head_dim must be a power of two");
  if (hd > kCombineMaxHd) return fail("head_dim above 256 is not supported");
  if (!p->q) return fail("null q");
  if (p->table_count < 0) return fail("table_count must be non-negative");
  if (p->table_count > 0) {
    if (!p->table) return fail("null segment table");
    if (p->table_bits != 2 && p->table_bits != 4) return fail("table_bits must be 2 or 4");
    if (hd != 64 && hd != 128) return fail("a segment table needs head_dim 64 or 128");
    if (p->flags & PK_FLAG_GENERIC_KERNEL)
      return fail("a segment table runs on the MFMA kernel only");
  }
  if (p->num_segments < 0 || (p->num_segments > 0 && !p->segments) ||
      (p->num_segments == 0 && p->table_count == 0))
    return fail("no segments to attend");
  for (int i = 0; i < p->num_segments; ++i) {
    const pk_segment& s = p->segments[i];
    if (s.length <= 0) return fail("segment " + std::to_string(i) + " is empty");
    if (!s.k_data || !s.v_data) return fail("segment " + std::to_string(i) + ": null K/V data");
    if (s.splits < 0 || s.split_len < 0) return fail("splits and split_len must be non-negative");
    if (s.split_len > 0 && (s.splits <= 0 || (int64_t)s.splits * s.split_len < s.length))
      return fail("split_len needs splits with splits * split_len >= length");
    if (s.kind == PK_SEG_FP16) {
      if (s.tok_stride < hd) return fail("FP16 segment token stride below head_dim");
      continue;
    }
    if (s.kind != PK_SEG_KIVI && s.kind != PK_SEG_TOKEN)
      return fail("unknown segment kind " + std::to_string(s.kind));
    if (!valid_bits(s.k_bits) || !valid_bits(s.v_bits)) return fail("bits must be one of (2, 4, 8)");
    if (s.k_group <= 0 || s.v_group <= 0) return fail("group sizes must be positive");
    if (!s.k_scale || !s.k_mins || !s.v_scale || !s.v_mins)
      return fail("segment " + std::to_string(i) + ": null scale/min");
    if (s.kind == PK_SEG_KIVI && s.k_group > s.length)
      return fail("K group size exceeds the segment length");
    if (s.k_meta_layout != PK_META_CHANNEL_MAJOR &&
        (s.k_meta_layout != PK_META_GROUP_MAJOR || s.kind != PK_SEG_KIVI))
      return fail("k_meta_layout must be channel major, or group major for a KIVI segment");
    if (s.k_data_layout != PK_CODES_CHANNEL_MAJOR &&
        (s.k_data_layout != PK_CODES_TOKEN_MAJOR || s.kind != PK_SEG_KIVI))
      return fail("k_data_layout must be channel major, or token major for a KIVI segment");
    if (s.v_group > hd) return fail("V group size exceeds head_dim");
    if (s.kind == PK_SEG_TOKEN && s.k_group > hd) return fail("K group size exceeds head_dim");
  }
  return PK_OK;
}

struct Plan {
  bool mfma;            // MFMA fast path (else the generic kernel)
  int tbl_items = 0;    // work items over the device segment table, per row
  int tbl_per_item = 0; // table entries per work item (kWaves per wave round)
  int tbl_gbegin = 0;   // partial column of the first table item
  int G, HS, nslab, tile;
  int C;
  int max_kbits, max_vbits;
  std::vector<int> n_chunks, chunk_len, gbegin;
  std::vector<int> seg_order;   // launch order of the segments (costliest chunks first)
  int order = 0;                // MFMA kernel workgroup order (DecodeParams::order)
  size_t off_m, off_l, off_acc, bytes;
};

static bool aligned(const void* ptr, int64_t a) { return (reinterpret_cast<uintptr_t>(ptr) % a) == 0; }

// The MFMA kernel covers head_dim 64 / 128, FP16 segments with 16-byte aligned
// rows, KIVI segments with 32-token K groups (or a single group) and 32-channel
// V groups, and per-token K segments with 32-channel K and V groups (not in the
// same launch as KIVI segments); explicit split lengths must be whole 32-token
// groups.
static bool mfma_eligible(const pk_decode_problem* p) {
  if (p->flags & PK_FLAG_GENERIC_KERNEL) return false;
  const int hd = p->head_dim;
  if (hd != 64 && hd != 128) return false;
  if (!aligned(p->q, 16) || p->q_hstride % 8 || p->q_bstride % 8) return false;
  bool has_kivi = p->table_count > 0, has_token = false;
  for (int i = 0; i < p->num_segments; ++i) {
    has_kivi = has_kivi || p->segments[i].kind == PK_SEG_KIVI;
    has_token = has_token || p->segments[i].kind == PK_SEG_TOKEN;
  }
  if (has_kivi && has_token) return false;
  const int ns = hd / 32;
  for (int i = 0; i < p->num_segments; ++i) {
    const pk_segment& s = p->segments[i];
    if (s.splits > 0) {
      const int64_t cl = s.split_len > 0 ? s.split_len
                                         : cdiv(s.length, std::min<int64_t>(s.length, s.splits));
      const int64_t nc = s.split_len > 0 ? s.splits : cdiv(s.length, cl);
      if (nc > 1 && cl % 32) return false;
    }
    if (s.kind == PK_SEG_FP16) {
      if (s.tok_stride % 8 || !aligned(s.k_data, 16) || !aligned(s.v_data, 16)) return false;
      if (s.k_data_bstride % 8 || s.k_data_hstride % 8 || s.v_data_bstride % 8 ||
          s.v_data_hstride % 8)
        return false;
      continue;
    }
    if (s.kind == PK_SEG_TOKEN) {
      // K code rows (hd * k_bits / 8 bytes) in 16-byte pieces, K metadata one token
      // (hd / 32 fp16) per load
      if (s.k_group != 32 || s.v_group != 32) return false;
      if (!aligned(s.k_data, 16) || s.k_data_bstride % 16 || s.k_data_hstride % 16) return false;
      if (!aligned(s.k_scale, 2 * ns) || !aligned(s.k_mins, 2 * ns) || s.k_meta_bstride % ns ||
          s.k_meta_hstride % ns)
        return false;
    } else if (s.kind != PK_SEG_KIVI) {
      return false;
    }
    // token-major K codes are read in 16-byte pieces of HD-byte rows
    if (s.k_data_layout == PK_CODES_TOKEN_MAJOR &&
        (!aligned(s.k_data, 16) || s.k_data_bstride % 16 || s.k_data_hstride % 16))
      return false;
    // K groups of 32 tokens, or one group for a segment of at most 32 tokens
    if (s.kind == PK_SEG_KIVI &&
        (!(s.k_group == 32 || (s.length <= 32 && s.k_group >= s.length)) || s.v_group != 32))
      return false;
    // K rows and K metadata are read at whatever alignment they have; V rows in
    // 16-byte pieces and V metadata one token (hd / 32 fp16) per load
    if (!aligned(s.v_data, 16) || s.v_data_bstride % 16 || s.v_data_hstride % 16) return false;
    const int vma = hd / 32;
    if (!aligned(s.v_scale, 2 * vma) || !aligned(s.v_mins, 2 * vma) || s.v_meta_bstride % vma ||
        s.v_meta_hstride % vma)
      return false;
  }
  return true;
}

static int64_t env_int(const char* name, int64_t dflt) {
  const char* v = getenv(name);
  if (!v || !*v) return dflt;
  return std::max<int64_t>(1, atoll(v));
}

static double env_double(const char* name, double dflt) {
  const char* v = getenv(name);
  if (!v || !*v) return dflt;
  const double x = atof(v);
  return x > 0 ? x : dflt;
}

// Relative cost of a 32-token group in the MFMA kernel (measured on MI355X at
// batch 8, hd 128): 2/2-bit 100, 4/4-bit 118, 2/8-bit 150, 8/8-bit 190, fp16 280.
static int group_weight(const pk_segment& s) {
  if (s.kind == PK_SEG_FP16) return 280;
  const int lo = std::min(s.k_bits, s.v_bits), hi = std::max(s.k_bits, s.v_bits);
  if (hi == 2) return 100;
  if (hi == 4) return lo == 2 ? 110 : 118;
  return lo == 2 ? 150 : lo == 4 ? 165 : 190;
}

static bool wave_path_only(const pk_decode_problem* p);

// Per-group factor of a chunk on an eight-wave workgroup (a wave's group chain shared
// with the SIMD's second wave), fitted on the legacy 16K / 32K rows: -0.5 µs per step.
constexpr double kPlanWave8Factor = 1.6;

// Automatic plan of the MFMA kernel: per-segment chunk lengths (whole 32-token
// groups, at least one per wave) sized by group weight, so every chunk costs about the same whatever its segment's bit
// widths, and the number of chunks per row chosen among a few candidates around
// one and two workgroups per CU by an estimate of the finishing time (fitted to
// MI355X measurements): chunk cost = 5 + groups per wave * weight * t, t = 1
// alone on a CU and 1.8 with a second workgroup; workgroups beyond two per CU run
// as the cheapest chunks (launch order), so they add about half a cheap chunk.  A plan
// of at most one workgroup per CU with chunks of 8 or more groups runs eight waves per
// workgroup where the segments allow it (launch_partials): groups per wave halve, at
// factor kPlanWave8Factor.

static void plan_weighted(const pk_decode_problem* p, int64_t per_bh, Plan& pl) {
  const int ns = p->num_segments;
  const bool wave8 = wave_path_only(p);
  std::vector<int64_t> G(ns), w(ns);
  int64_t row = 0;
  for (int i = 0; i < ns; ++i) {
    G[i] = cdiv(p->segments[i].length, 32);
    w[i] = group_weight(p->segments[i]);
    row += G[i] * w[i];
  }
  const int64_t cus = device_cu_count(), slots = 2 * cus;
  const double w8t = env_double("PK_PLAN_W8T", kPlanWave8Factor);
  std::vector<int64_t> g(ns), best_g(ns, 4);
  double best = 1e30;
  int64_t best_wgs = 0;
  auto evaluate = [&](int64_t U) -> int64_t {   // plan for chunk cost U; returns workgroups
    int64_t wgs = 0;
    for (int i = 0; i < ns; ++i) {
      g[i] = std::min(G[i], std::max<int64_t>(4, U / w[i]));
      wgs += cdiv(G[i], g[i]) * per_bh;
    }
    const double t = wgs <= cus ? 1.0 : 1.8;
    // eight waves per workgroup (launch_partials) when the launch fits one workgroup per CU
    // and its chunks hold 8 or more groups: the groups spread over twice the waves
    int64_t gmin = INT64_MAX;
    for (int i = 0; i < ns; ++i) gmin = std::min(gmin, g[i]);
    const bool w8 = w8t > 0 && wave8 && wgs <= cus && gmin >= 8;
    auto cost = [&](int64_t groups, int64_t wi) {
      if (w8) return 5.0 + std::ceil(groups / 8.0) * (double)wi / 100.0 * w8t;
      return 5.0 + std::ceil(groups / 4.0) * (double)wi / 100.0 * t;
    };
    double cmax = 0, cmin = 1e30, total = 0;
    for (int i = 0; i < ns; ++i) {
      const int64_t n = cdiv(G[i], g[i]);
      const double c = cost(g[i], w[i]);
      cmax = std::max(cmax, c);
      cmin = std::min(cmin, c);
      total += ((double)(n - 1) * c + cost(G[i] - (n - 1) * g[i], w[i])) * (double)per_bh;
    }
    const double est = wgs <= slots ? cmax : std::max(cmax, total / slots) + 0.5 * cmin;
    if (est < best - 1e-9 || (est < best + 1e-9 && wgs < best_wgs)) {
      best = est;
      best_wgs = wgs;
      best_g = g;
    }
    return wgs;
  };
  const int64_t forced = env_int("PK_PLAN_UNITS", 0);   // a fixed chunk cost, for experiments
  if (forced > 0) {
    best = 1e30;
    evaluate(forced);
    best = -1.0;   // keep it
  }
  // the smallest chunks that fit one, then two workgroups per CU
  for (int64_t cap : {cus, slots}) {
    int64_t U = std::max<int64_t>(400, cdiv(row * per_bh, cap));
    for (int it = 0; it < 64 && evaluate(U) > cap; ++it) U += std::max<int64_t>(1, U / 32);
  }
  // and a few with more workgroups than two per CU
  for (double f : {1.25, 1.5, 2.0, 3.0})
    evaluate(std::max<int64_t>(400, (int64_t)(row * per_bh / (f * slots))));
  std::vector<double> cost(ns);
  for (int i = 0; i < ns; ++i) {
    pl.chunk_len.push_back(static_cast<int>(std::min<int64_t>(32 * best_g[i], p->segments[i].length)));
    pl.n_chunks.push_back(static_cast<int>(cdiv(G[i], best_g[i])));
    pl.gbegin.push_back(pl.C);
    pl.C += pl.n_chunks.back();
    cost[i] = (double)best_g[i] * (double)w[i];
  }
  pl.seg_order.resize(ns);
  for (int i = 0; i < ns; ++i) pl.seg_order[i] = i;
  std::stable_sort(pl.seg_order.begin(), pl.seg_order.end(),
                   [&](int a, int b) { return cost[a] > cost[b]; });
  // chunk-major order unless a segment keeps the reference's channel-major K,
  // whose neighbouring chunks share lines (those go to one XCD's L2)
  pl.order = 1;
  for (int i = 0; i < ns; ++i) {
    const pk_segment& s = p->segments[i];
    if (s.kind == PK_SEG_KIVI &&
        (s.k_data_layout != PK_CODES_TOKEN_MAJOR || s.k_meta_layout != PK_META_GROUP_MAJOR))
      pl.order = 0;
  }
}

// Work items over the device segment table: one segment per wave, kWaves per item.
static constexpr int kHostWaves = kThreads / 64;
static void plan_table(const pk_decode_problem* p, int64_t per_bh, Plan& pl) {
  (void)per_bh;
  pl.tbl_per_item = kHostWaves;
  pl.tbl_items = static_cast<int>(cdiv(p->table_count, kHostWaves));
  pl.tbl_gbegin = pl.C;
  pl.C += pl.tbl_items;
  pl.max_kbits = std::max(pl.max_kbits, (int)p->table_bits);
  pl.max_vbits = std::max(pl.max_vbits, (int)p->table_bits);
}

static bool weighted_plan(const pk_decode_problem* p) {
  if (env_int("PK_CHUNK_TOKENS", 0) > 0 || env_int("PK_TARGET_WORKGROUPS", 0) > 0) return false;
  const char* v = getenv("PK_WEIGHTED_PLAN");
  if (v && v[0] == '0') return false;
  for (int i = 0; i < p->num_segments; ++i)
    if (p->segments[i].splits > 0) return false;
  return true;
}

static Plan make_plan(const pk_decode_problem* p) {
  Plan pl{};
  const int hd = p->head_dim;
  pl.mfma = mfma_eligible(p);
  pl.G = p->num_q_heads / p->num_kv_heads;
  pl.HS = pl.mfma ? std::min(pl.G, 16) : head_slab(pl.G, hd);
  pl.nslab = static_cast<int>(cdiv(pl.G, pl.HS));
  pl.tile = std::min(64, std::max(8, 4096 / hd));
  int64_t total_len = 0;
  pl.max_kbits = 2;
  pl.max_vbits = 2;
  for (int i = 0; i < p->num_segments; ++i) {
    const pk_segment& s = p->segments[i];
    total_len += s.length;
    if (s.kind != PK_SEG_FP16) {
      pl.max_kbits = std::max(pl.max_kbits, s.k_bits);
      pl.max_vbits = std::max(pl.max_vbits, s.v_bits);
    }
  }
  const int64_t per_bh = (int64_t)p->batch * p->num_kv_heads * pl.nslab;
  int64_t auto_len;
  if (pl.mfma) {
    // about two 4-wave workgroups per CU, chunks of whole 128-token rounds (one
    // 32-token group per wave), so few partials per row reach the combine
    const int64_t want = env_int("PK_TARGET_WORKGROUPS", 2LL * device_cu_count());
    auto_len = cdiv(cdiv(total_len * per_bh, want), 128) * 128;
    auto_len = env_int("PK_CHUNK_TOKENS", std::max<int64_t>(128, auto_len));
    auto_len = cdiv(auto_len, 32) * 32;
  } else {
    const int64_t want = 4LL * device_cu_count();
    const int64_t chunks_target = std::max<int64_t>(1, cdiv(want, per_bh));
    auto_len = cdiv(total_len, chunks_target);
    auto_len = std::max<int64_t>(kMinChunk, cdiv(auto_len, kMinChunk) * kMinChunk);
  }
  pl.C = 0;
  if (pl.mfma && weighted_plan(p)) {
    plan_weighted(p, per_bh, pl);
  } else
  for (int i = 0; i < p->num_segments; ++i) {
    const pk_segment& s = p->segments[i];
    int64_t cl;
    int64_t nc;
    if (s.splits > 0 && s.split_len > 0) {
      cl = s.split_len;
      nc = s.splits;
    } else if (s.splits > 0) {
      cl = cdiv(s.length, std::min<int64_t>(s.length, s.splits));
      nc = cdiv(s.length, cl);
    } else {
      cl = std::min<int64_t>(auto_len, s.length);
      nc = cdiv(s.length, cl);
    }
    pl.chunk_len.push_back(static_cast<int>(cl));
    pl.n_chunks.push_back(static_cast<int>(nc));
    pl.gbegin.push_back(pl.C);
    pl.C += static_cast<int>(nc);
  }
  if (pl.seg_order.empty())
    for (int i = 0; i < p->num_segments; ++i) pl.seg_order.push_back(i);
  if (p->table_count > 0) plan_table(p, per_bh, pl);
  const int64_t rows = (int64_t)p->batch * p->num_q_heads;
  auto align = [](size_t x) { return (x + 255) & ~size_t(255); };
  pl.off_m = 0;
  pl.off_l = align(pl.off_m + rows * pl.C * sizeof(float));
  pl.off_acc = align(pl.off_l + rows * pl.C * sizeof(float));
  pl.bytes = align(pl.off_acc + rows * pl.C * (size_t)hd * sizeof(float));
  return pl;
}

// Requirements of the problem on the kernel choice: a device table and
// PK_FLAG_REQUIRE_MFMA need the MFMA kernel.
static int check_plan(const pk_decode_problem* p, const Plan& pl) {
  if (pl.mfma) return PK_OK;
  if (p->table_count > 0)
    return fail("a segment table needs every other segment on the MFMA path (head_dim 64 / "
                "128, 32-token K groups, aligned rows)");
  if (p->flags & PK_FLAG_REQUIRE_MFMA)
    return fail("the MFMA kernel does not apply (head_dim 64 / 128, 32-token K groups or "
                "32-channel groups, aligned rows, whole 32-token splits, no KIVI and per-token "
                "K segments together)");
  return PK_OK;
}

static void fill_segment(SegDev& d, const pk_segment& s) {
  d.kind = s.kind;
  d.length = s.length;
  d.kbits = s.k_bits;
  d.vbits = s.v_bits;
  d.kgs = s.k_group;
  d.vgs = s.v_group;
  d.seq_lens = s.seq_lens;
  d.kd = static_cast<const uint8_t*>(s.k_data);
  d.ks = s.k_scale;
  d.km = s.k_mins;
  d.vd = static_cast<const uint8_t*>(s.v_data);
  d.vs = s.v_scale;
  d.vm = s.v_mins;
  d.kd_bs = s.k_data_bstride; d.kd_hs = s.k_data_hstride;
  d.km_bs = s.k_meta_bstride; d.km_hs = s.k_meta_hstride;
  d.vd_bs = s.v_data_bstride; d.vd_hs = s.v_data_hstride;
  d.vm_bs = s.v_meta_bstride; d.vm_hs = s.v_meta_hstride;
  d.tok_stride = s.tok_stride;
  d.kmeta_gm = s.kind == PK_SEG_KIVI && s.k_meta_layout == PK_META_GROUP_MAJOR;
  d.kdata_tm = s.kind == PK_SEG_KIVI && s.k_data_layout == PK_CODES_TOKEN_MAJOR;
}

static size_t generic_lds_bytes(const Plan& pl, int hd) {
  return sizeof(float) * ((size_t)2 * pl.HS * hd + (size_t)2 * pl.tile * (hd + 1) +
                          (size_t)pl.HS * pl.tile + 3 * pl.HS);
}

// Whether every segment of the problem takes the MFMA kernel's wave-private group path
// (what the 8-wave variants compile): FP16 segments, per-token K segments and KIVI segments
// in quantize_pack's storage (token-major codes, group-major metadata 8-byte aligned), codes
// up to 4 bits, no device table.
static bool wave_path_only(const pk_decode_problem* p) {
  if (p->table_count > 0) return false;
  for (int i = 0; i < p->num_segments; ++i) {
    const pk_segment& s = p->segments[i];
    if (s.kind == PK_SEG_FP16) continue;
    if (s.k_bits > 4 || s.v_bits > 4) return false;
    if (s.kind == PK_SEG_TOKEN) continue;
    if (s.k_data_layout != PK_CODES_TOKEN_MAJOR || s.k_meta_layout != PK_META_GROUP_MAJOR)
      return false;
    if (!aligned(s.k_scale, 8) || !aligned(s.k_mins, 8) || s.k_meta_bstride % 4 ||
        s.k_meta_hstride % 4)
      return false;
    if (cdiv((int64_t)s.length * s.k_bits, 8) >= ((int64_t)1 << 31) / p->head_dim) return false;
  }
  return true;
}

static int launch_partials(const pk_decode_problem* p, const Plan& pl, char* ws,
                           hipStream_t stream) {
  DecodeParams dp{};
  dp.B = p->batch;
  dp.Hq = p->num_q_heads;
  dp.Hkv = p->num_kv_heads;
  dp.hd = p->head_dim;
  dp.G = pl.G;
  dp.HS = pl.HS;
  dp.nslab = pl.nslab;
  dp.tile = pl.tile;
  dp.scale = 1.0f / sqrtf(static_cast<float>(p->head_dim));
  dp.q = p->q;
  dp.q_bs = p->q_bstride;
  dp.q_hs = p->q_hstride;
  dp.ws_m = reinterpret_cast<float*>(ws + pl.off_m);
  dp.ws_l = reinterpret_cast<float*>(ws + pl.off_l);
  dp.ws_acc = reinterpret_cast<float*>(ws + pl.off_acc);
  dp.C = pl.C;
  const size_t lds = generic_lds_bytes(pl, p->head_dim);
  // the inline segments, then (if any) the table's work items as one more launch entry
  const int entries = p->num_segments + (pl.tbl_items > 0 ? 1 : 0);
  for (int first = 0; first < entries; first += kMaxSeg) {
    const int n = std::min(kMaxSeg, entries - first);
    int lchunks = 0;
    for (int i = 0; i < n; ++i) {
      SegDev& d = dp.seg[i];
      if (first + i == p->num_segments) {
        d = SegDev{};
        d.kind = kSegTable;
        d.length = p->table_count;
        d.chunk_len = pl.tbl_per_item;
        d.n_chunks = pl.tbl_items;
        d.gbegin = pl.tbl_gbegin;
        d.kd = static_cast<const uint8_t*>(p->table);
        d.hd_meta = p->head_dim;
      } else {
        const int si = pl.seg_order[first + i];
        fill_segment(d, p->segments[si]);
        d.hd_meta = p->head_dim;
        d.chunk_len = pl.chunk_len[si];
        d.n_chunks = pl.n_chunks[si];
        d.gbegin = pl.gbegin[si];
      }
      d.lbegin = lchunks;
      lchunks += d.n_chunks;
    }
    dp.nseg = n;
    dp.order = pl.order;
    int rc;
    if (pl.mfma) {
      // a launch of at most one workgroup per CU whose chunks hold 8 or more groups runs
      // eight waves per workgroup where every segment allows it: two waves per SIMD hide
      // each other's group chains (measured: C3-32K -1.1 µs; with fewer groups per chunk
      // the idle waves and the wider merge cost more, C2 +0.4 µs)
      const int64_t wgs = (int64_t)lchunks * p->num_kv_heads * pl.nslab * p->batch;
      int max_groups = 0;
      for (int i = 0; i < n; ++i)
        if (dp.seg[i].kind != kSegTable) max_groups = std::max(max_groups, (dp.seg[i].chunk_len + 31) / 32);
      const char* w8 = getenv("PK_WAVES8");   // "0": four waves always, for experiments
      const int waves = (wgs <= device_cu_count() && max_groups >= 8 && wave_path_only(p) &&
                         !(w8 && w8[0] == '0')) ? 8 : 4;
      rc = launch_decode_mfma(dp, lchunks, pl.max_kbits, pl.max_vbits, waves, wave_path_only(p),
                              stream);
    } else {
      dim3 grid(lchunks, p->num_kv_heads * pl.nslab, p->batch);
      hipLaunchKernelGGL(decode_partials_generic, grid, dim3(kThreads), lds, stream, dp);
      rc = check_launch("decode_partials");
    }
    if (rc) return rc;
  }
  return PK_OK;
}

}  // namespace pk

using namespace pk;

extern "C" int pk_decode_workspace_size(const pk_decode_problem* p, size_t* bytes,
                                        int32_t* total_splits) {
  return pk::guarded("pk_decode_workspace_size", [&]() -> int {
    clear_error();
    int rc = validate_problem(p);
    if (rc) return rc;
    Plan pl = make_plan(p);
    if (int rc = check_plan(p, pl)) return rc;
    if (bytes) *bytes = pl.bytes;
    if (total_splits) *total_splits = pl.C;
    return PK_OK;
  });
}

// ---------------------------------------------------------------------------
// device segment table
// ---------------------------------------------------------------------------
namespace {
constexpr int kTableBatch = 8;   // entries per write launch (kernel argument block)

struct TableBatch {
  int n;
  SegDev seg[kTableBatch];
};

__global__ void __launch_bounds__(64) table_write_kernel(SegDev* table, TableBatch batch) {
  static_assert(sizeof(SegDev) % 4 == 0, "entries copy in words");
  const uint32_t* src = reinterpret_cast<const uint32_t*>(batch.seg);
  uint32_t* dst = reinterpret_cast<uint32_t*>(table);
  const int words = batch.n * (int)(sizeof(SegDev) / 4);
  for (int i = threadIdx.x; i < words; i += 64) dst[i] = src[i];
}

// The storage the wave-private group pipeline reads (see pk_segment_table_write).
int table_entry_check(const pk_segment& s, int hd, int i) {
  const std::string at = "table entry " + std::to_string(i) + ": ";
  if (s.kind != PK_SEG_KIVI) return fail(at + "only KIVI segments go to a segment table");
  if (s.length <= 0) return fail(at + "empty segment");
  if ((s.k_bits != 2 && s.k_bits != 4) || (s.v_bits != 2 && s.v_bits != 4))
    return fail(at + "K and V widths must be 2 or 4 bits");
  if (s.splits != 0 || s.split_len != 0) return fail(at + "segments in a table are not split");
  if (s.k_data_layout != PK_CODES_TOKEN_MAJOR || s.k_meta_layout != PK_META_GROUP_MAJOR)
    return fail(at + "K must be stored as quantize_pack writes it (token-major codes, "
                     "group-major scale / min)");
  if (!(s.k_group == 32 || (s.length <= 32 && s.k_group >= s.length)) || s.v_group != 32)
    return fail(at + "K groups of 32 (or one group) and V groups of 32 are required");
  if (!s.k_data || !s.k_scale || !s.k_mins || !s.v_data || !s.v_scale || !s.v_mins)
    return fail(at + "null K/V pointer");
  if (!aligned(s.k_data, 16) || s.k_data_bstride % 16 || s.k_data_hstride % 16)
    return fail(at + "K code rows must be 16-byte aligned");
  if (!aligned(s.k_scale, 8) || !aligned(s.k_mins, 8) || s.k_meta_bstride % 4 ||
      s.k_meta_hstride % 4)
    return fail(at + "K scale / min rows must be 8-byte aligned");
  if (!aligned(s.v_data, 16) || s.v_data_bstride % 16 || s.v_data_hstride % 16)
    return fail(at + "V code rows must be 16-byte aligned");
  const int vma = hd / 32;
  if (!aligned(s.v_scale, 2 * vma) || !aligned(s.v_mins, 2 * vma) || s.v_meta_bstride % vma ||
      s.v_meta_hstride % vma)
    return fail(at + "V scale / min rows misaligned");
  if ((int64_t)s.length * s.k_bits / 8 >= ((int64_t)1 << 31) / hd) return fail(at + "segment too long");
  return PK_OK;
}
}  // namespace

extern "C" size_t pk_segment_table_entry_bytes(void) { return sizeof(SegDev); }

extern "C" int pk_segment_table_write(void* table, int32_t first, int32_t count,
                                      const pk_segment* segments, int32_t head_dim,
                                      void* stream) {
  return pk::guarded("pk_segment_table_write", [&]() -> int {
    clear_error();
    if (!table) return fail("null table");
    if (first < 0 || count < 0) return fail("first and count must be non-negative");
    if (count > 0 && !segments) return fail("null segments");
    if (head_dim != 64 && head_dim != 128) return fail("head_dim must be 64 or 128");
    for (int i = 0; i < count; ++i) {
      const int rc = table_entry_check(segments[i], head_dim, i);
      if (rc) return rc;
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    SegDev* dst = static_cast<SegDev*>(table) + first;
    for (int i0 = 0; i0 < count; i0 += kTableBatch) {
      TableBatch batch{};
      batch.n = std::min(kTableBatch, count - i0);
      for (int i = 0; i < batch.n; ++i) {
        fill_segment(batch.seg[i], segments[i0 + i]);
        batch.seg[i].hd_meta = head_dim;
      }
      hipLaunchKernelGGL(table_write_kernel, dim3(1), dim3(64), 0, st, dst + i0, batch);
      const int rc = check_launch("segment_table_write");
      if (rc) return rc;
    }
    return PK_OK;
  });
}

extern "C" int pk_decode_partials(const pk_decode_problem* p, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  return pk::guarded("pk_decode_partials", [&]() -> int {
    clear_error();
    int rc = validate_problem(p);
    if (rc) return rc;
    Plan pl = make_plan(p);
    if (int rc = check_plan(p, pl)) return rc;
    if (!workspace || workspace_bytes < pl.bytes) return fail("workspace too small");
    return launch_partials(p, pl, static_cast<char*>(workspace), static_cast<hipStream_t>(stream));
  });
}

static int launch_combine(const float* m, const float* l, const float* acc, int64_t rows, int C,
                          int hd, uint16_t* out, float* om, float* ol, float* oacc,
                          hipStream_t stream, const char* what) {
  if (rows == 0) return PK_OK;
  const bool vec = hd % 4 == 0 && aligned(acc, 16) && (!oacc || aligned(oacc, 16));
  // "0" workgroup slices, "1" rows, "2" waves: force a kernel where it applies, for experiments
  const char* force = getenv("PK_COMBINE_KERNEL");
  const int kind = (force && *force) ? atoi(force) : -1;
  // one round trip per thread: few partials per row over many rows (measured on MI355X:
  // 4.3 -> 2.9 us at 448 rows of 8, 25.5 -> 3 us at 7168 rows of 3; no gain at 896 rows of
  // 10); a few rows (C1: 14 of 5, 224 threads) go to the wave combine, 2.62 -> 2.45 us
  const bool many_rows = rows * (hd / 4) >= 32 * kCombineRowsThreads;
  if (vec && (kind == 1 || (kind < 0 && many_rows)) && C <= kCombineLoads) {
    const int64_t blocks = (rows * (hd / 4) + kCombineRowsThreads - 1) / kCombineRowsThreads;
    if (blocks > INT32_MAX) return fail("too many output rows");
    hipLaunchKernelGGL(combine_rows_kernel, dim3((unsigned)blocks), dim3(kCombineRowsThreads), 0,
                       stream, m, l, acc, rows, C, hd, out, om, ol, oacc);
    return check_launch(what);
  }
  // one wave per (row, 16 channels): 28 rows of 35 at C2 3.46 -> 2.85 us (8 channels per
  // wave 2.97, 4 channels 3.35, 32 channels 3.11), 2.63 us with the slices grouped by XCD
  if (vec && hd % 16 == 0 && (kind < 0 || kind == 2) && C <= 16 * kCombineLoads) {
    const int64_t blocks = rows * (hd / 16);
    if (blocks > INT32_MAX) return fail("too many output rows");
    const dim3 grid((unsigned)blocks), block(64);
    if (C <= 32)
      hipLaunchKernelGGL(combine_wave_kernel<2>, grid, block, 0, stream, m, l, acc, rows, C,
                         hd, out, om, ol, oacc);
    else if (C <= 64)
      hipLaunchKernelGGL(combine_wave_kernel<4>, grid, block, 0, stream, m, l, acc, rows, C,
                         hd, out, om, ol, oacc);
    else
      hipLaunchKernelGGL(combine_wave_kernel<kCombineLoads>, grid, block, 0, stream, m, l,
                         acc, rows, C, hd, out, om, ol, oacc);
    return check_launch(what);
  }
  // about kCombineTarget partials per thread, at least 4 and at most 16 partial lanes
  int ncs = 4;
  while (ncs < 16 && ncs * kCombineTarget < C) ncs <<= 1;
  const int hs = std::min(hd, kThreads / ncs);
  const int64_t blocks = rows * (hd / hs);
  if (blocks > INT32_MAX) return fail("too many output rows");
  hipLaunchKernelGGL(combine_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, stream, m, l, acc,
                     C, hd, hs, out, om, ol, oacc);
  return check_launch(what);
}

extern "C" int pk_decode_combine(const pk_decode_problem* p, const void* workspace,
                                 uint16_t* out, float* out_m, float* out_l, float* out_acc,
                                 void* stream) {
  return pk::guarded("pk_decode_combine", [&]() -> int {
    clear_error();
    int rc = validate_problem(p);
    if (rc) return rc;
    if (!workspace) return fail("null workspace");
    if (!out && !(out_m && out_l && out_acc)) return fail("no output requested");
    Plan pl = make_plan(p);
    if (int rc = check_plan(p, pl)) return rc;
    const char* ws = static_cast<const char*>(workspace);
    return launch_combine(reinterpret_cast<const float*>(ws + pl.off_m),
                          reinterpret_cast<const float*>(ws + pl.off_l),
                          reinterpret_cast<const float*>(ws + pl.off_acc),
                          (int64_t)p->batch * p->num_q_heads, pl.C, p->head_dim, out, out_m, out_l,
                          out_acc, static_cast<hipStream_t>(stream), "decode_combine");
  });
}

extern "C" int pk_fused_decode(const pk_decode_problem* p, void* workspace, size_t workspace_bytes,
                               uint16_t* out, void* stream) {
  return pk::guarded("pk_fused_decode", [&]() -> int {
    clear_error();
    int rc = validate_problem(p);
    if (rc) return rc;
    if (!out) return fail("null output");
    Plan pl = make_plan(p);
    if (int rc = check_plan(p, pl)) return rc;
    if (!workspace || workspace_bytes < pl.bytes) return fail("workspace too small");
    hipStream_t s = static_cast<hipStream_t>(stream);
    rc = launch_partials(p, pl, static_cast<char*>(workspace), s);
    if (rc) return rc;
    const char* ws = static_cast<const char*>(workspace);
    return launch_combine(reinterpret_cast<const float*>(ws + pl.off_m),
                          reinterpret_cast<const float*>(ws + pl.off_l),
                          reinterpret_cast<const float*>(ws + pl.off_acc),
                          (int64_t)p->batch * p->num_q_heads, pl.C, p->head_dim, out, nullptr,
                          nullptr, nullptr, s, "fused_decode");
  });
}

// ---------------------------------------------------------------------------
// pk_fused_decode_noalloc: the split-K workspace in a file-scope device array
// (one per GPU, held until the process ends) instead of a caller buffer.
// ---------------------------------------------------------------------------
static __device__ __align__(256) char scratch[PK_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
char* g_scratch[kMaxDevices] = {};   // the array's device address, per device

// The scratch array's address on the current device (looked up once per device).
int scratch_address(char** ptr) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error(std::string("hipGetDevice: ") + hipGetErrorString(e));
    return PK_ERR_RUNTIME;
  }
  if (dev < 0 || dev >= kMaxDevices) return fail("device index above 63");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      set_error(std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
      return PK_ERR_RUNTIME;
    }
    g_scratch[dev] = static_cast<char*>(p);
  }
  *ptr = g_scratch[dev];
  return PK_OK;
}
}  // namespace

extern "C" int pk_fused_decode_noalloc(const pk_decode_problem* p, uint16_t* out, void* stream) {
  return pk::guarded("pk_fused_decode_noalloc", [&]() -> int {
    clear_error();
    int rc = validate_problem(p);
    if (rc) return rc;
    if (!out) return fail("null output");
    Plan pl = make_plan(p);
    if (int rc = check_plan(p, pl)) return rc;
    if (pl.bytes > (size_t)PK_NOALLOC_SCRATCH_BYTES)
      return fail("the problem needs " + std::to_string(pl.bytes) +
                  " bytes of split-K workspace; pk_fused_decode_noalloc holds " +
                  std::to_string((size_t)PK_NOALLOC_SCRATCH_BYTES) +
                  " (use pk_fused_decode with a caller workspace)");
    char* ws = nullptr;
    rc = scratch_address(&ws);
    if (rc) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    rc = launch_partials(p, pl, ws, s);
    if (rc) return rc;
    return launch_combine(reinterpret_cast<const float*>(ws + pl.off_m),
                          reinterpret_cast<const float*>(ws + pl.off_l),
                          reinterpret_cast<const float*>(ws + pl.off_acc),
                          (int64_t)p->batch * p->num_q_heads, pl.C, p->head_dim, out, nullptr,
                          nullptr, nullptr, s, "fused_decode_noalloc");
  });
}

extern "C" int pk_merge_partials(const float* m, const float* l, const float* acc, int64_t rows,
                                 int32_t n, int32_t head_dim, uint16_t* out, float* out_m,
                                 float* out_l, float* out_acc, void* stream) {
  return pk::guarded("pk_merge_partials", [&]() -> int {
    clear_error();
    if (rows < 0 || n <= 0 || head_dim <= 0) return fail("rows, n and head_dim must be positive");
    if (head_dim > kCombineMaxHd || (head_dim & (head_dim - 1)))
      return fail("head_dim must be a power of two <= 256");
    if (!m || !l || !acc) return fail("null partials");
    if (!out && !(out_m && out_l && out_acc)) return fail("no output requested");
    return launch_combine(m, l, acc, rows, n, head_dim, out, out_m, out_l, out_acc,
                          static_cast<hipStream_t>(stream), "merge_partials");
  });
}

extern "C" int pk_merge_partial_sets(const pk_partial_set* sets, int32_t nsets, int64_t outer,
                                     int64_t inner, int32_t head_dim, uint16_t* out,
                                     float* out_m, float* out_l, float* out_acc, void* stream) {
  return pk::guarded("pk_merge_partial_sets", [&]() -> int {
    clear_error();
    if (!sets || nsets < 1 || nsets > PK_MAX_PARTIAL_SETS)
      return fail("between 1 and PK_MAX_PARTIAL_SETS partial sets");
    if (outer < 0 || inner < 0) return fail("outer and inner must be >= 0");
    if (head_dim <= 0 || head_dim > kCombineMaxHd || (head_dim & (head_dim - 1)) || head_dim < 4)
      return fail("head_dim must be a power of two in [4, 256]");
    if (!out && !(out_m && out_l && out_acc)) return fail("no output requested");
    if (out_acc && !aligned(out_acc, 16)) return fail("out_acc must be 16-byte aligned");
    PartialSets ps{};
    ps.nsets = nsets;
    for (int k = 0; k < nsets; ++k) {
      const pk_partial_set& s = sets[k];
      if (!s.m || !s.l || !s.acc) return fail("null partials");
      if (!aligned(s.acc, 16)) return fail("partial acc must be 16-byte aligned");
      if (s.n <= 0 || s.rows < 0 || s.outer_stride < 0 || s.inner_stride < 0)
        return fail("partial sets need n > 0 and non-negative rows and strides");
      if (outer && inner) {
        const int64_t last = (outer - 1) * s.outer_stride + (inner - 1) * s.inner_stride;
        if (last >= s.rows) return fail("a partial set's strides reach past its rows");
      }
      ps.s[k] = PartialSetDev{s.m, s.l, s.acc, s.outer_stride, s.inner_stride, s.n};
    }
    const int64_t rows = outer * inner;
    if (rows == 0) return PK_OK;
    const int64_t blocks = (rows * (head_dim / 4) + kCombineRowsThreads - 1) / kCombineRowsThreads;
    if (blocks > INT32_MAX) return fail("too many output rows");
    hipLaunchKernelGGL(combine_sets_kernel, dim3((unsigned)blocks), dim3(kCombineRowsThreads), 0,
                       static_cast<hipStream_t>(stream), ps, outer, inner, head_dim, out, out_m,
                       out_l, out_acc);
    return check_launch("merge_partial_sets");
  });
}
