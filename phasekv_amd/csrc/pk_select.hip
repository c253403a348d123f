// Prefill-side prompt selection (gfx950): observation-window votes over the
// prefill attention, GQA aggregation, 1-D pooling of the candidate scores and a
// per-kv-head top-k, producing the sorted positions the prompt tier keeps.
//
// Semantics follow the reference:
//   select_prompt_indices   src/phasekv/prompt_tier.py:22-76
//   observation_votes       src/phasekv/hetero_cache.py:67-77
//   aggregate_to_kv_heads   src/phasekv/hetero_cache.py:55-64
//   pool_scores             src/phasekv/hetero_cache.py:80-94 (max_pool1d / avg_pool1d,
//                           stride 1, padding kernel // 2, truncated to the length)
//   topk_per_head           src/phasekv/hetero_cache.py:147-157
#include "pk_common.h"

#include <algorithm>

#pragma clang fp contract(off)

namespace {

constexpr int kVotesMaxWaves = 16;  // votes kernel: one wave per query head of the group, up to 16
constexpr int kPickThreads = 1024;   // selection kernel: 16 waves share one row's candidates
// candidates whose votes and keys are staged in LDS (8 bytes each, 144 KB)
constexpr int64_t kMaxStagedKeys = 18 * 1024;

struct AttnView {
  const void* p;
  int dtype;
  int64_t sb, sh, sq, sk;   // element strides of batch, head, query row, key
};

__device__ __forceinline__ float load_attn(const AttnView& a, int64_t off) {
  if (a.dtype == PK_DTYPE_F16) return pk_h2f(static_cast<const uint16_t*>(a.p)[off]);
  if (a.dtype == PK_DTYPE_BF16) return pk_bf2f(static_cast<const uint16_t*>(a.p)[off]);
  return static_cast<const float*>(a.p)[off];
}

// votes[b, kv, j] = sum over the group's query heads g (in order) of the sum over
// the last w query rows r (in order) of attention[b, kv * G + g, q_len - w + r, j],
// all in float32.  A workgroup takes 64 * KPL key positions of one (b, kv) and has one
// wave per query head of the group (up to kVotesMaxWaves): wave s sums the rows of
// query heads s, s + waves, ... (KPL neighbouring keys per lane in one load, 64 / KPL
// rows of raw 16-bit loads in flight, added in row order; 16 rows of converted loads for
// other dtypes and tails), and wave 0 adds the heads' sums in head order.
// A wave per head keeps every head's rows in flight at once: the launch is bound by
// the bytes in flight per CU.
constexpr int kMaxGroup = 32;

template <int KPL, typename T>
__device__ __forceinline__ void load_keys(const AttnView& a, int64_t off, float (&x)[KPL]) {
  if constexpr (KPL == 1) {
    x[0] = load_attn(a, off);
  } else {
    using V = uint16_t __attribute__((ext_vector_type(KPL)));
    const V v = *reinterpret_cast<const V*>(static_cast<const uint16_t*>(a.p) + off);
#pragma unroll
    for (int i = 0; i < KPL; ++i)
      x[i] = a.dtype == PK_DTYPE_F16 ? pk_h2f(v[i]) : pk_bf2f(v[i]);
  }
}

template <int KPL>
__global__ void __launch_bounds__(64 * kVotesMaxWaves)
votes_kernel(AttnView a, int Hkv, int G, int64_t q_len, int64_t kv_len, int w,
             float* __restrict__ votes) {
  constexpr int TILE = 64 * KPL;
  __shared__ float hs[kMaxGroup][TILE];
  const int lane = threadIdx.x & 63, slot = threadIdx.x >> 6;
  const int64_t tiles = (kv_len + TILE - 1) / TILE;
  const int64_t row = blockIdx.x / tiles;                 // b * Hkv + kv
  const int64_t j0 = (blockIdx.x - row * tiles) * TILE + lane * KPL;
  const int64_t b = row / Hkv, kv = row - b * Hkv;
  const int64_t jc = min(j0, kv_len - KPL);               // whole pieces stay inside the row
  for (int g = slot; g < G; g += (int)(blockDim.x / 64)) {
    const int64_t base = b * a.sb + (kv * G + g) * a.sh + (q_len - w) * a.sq + jc * a.sk;
    float sum[KPL];
#pragma unroll
    for (int i = 0; i < KPL; ++i) sum[i] = 0.f;
    int r = 0;
    if constexpr (KPL > 1) {
      // RB rows of raw 16-bit keys in flight (64 registers), converted as they are
      // added: the sums still run over the rows in order
      constexpr int RB = 64 / KPL;
      using V = uint16_t __attribute__((ext_vector_type(KPL)));
      const bool f16 = a.dtype == PK_DTYPE_F16;
      // the row's address is wave-uniform (scalar registers) plus this lane's 32-bit key
      // offset, so the RB loads need no address registers of their own
      const int gu = __builtin_amdgcn_readfirstlane(g);
      const uint16_t* up = static_cast<const uint16_t*>(a.p) + b * a.sb + (kv * G + gu) * a.sh +
                           (q_len - w) * a.sq;
      const uint32_t lbytes = static_cast<uint32_t>(jc * a.sk) * 2u;
      for (; r + RB <= w; r += RB) {
        V x[RB];
#pragma unroll
        for (int u = 0; u < RB; ++u)
          x[u] = *reinterpret_cast<const V*>(
              reinterpret_cast<const char*>(up + (int64_t)(r + u) * a.sq) + lbytes);
#pragma unroll
        for (int u = 0; u < RB; ++u)
#pragma unroll
          for (int i = 0; i < KPL; ++i)
            sum[i] = __fadd_rn(sum[i], f16 ? pk_h2f(x[u][i]) : pk_bf2f(x[u][i]));
      }
    }
    for (; r + 16 <= w; r += 16) {
      float x[16][KPL];
#pragma unroll
      for (int u = 0; u < 16; ++u) load_keys<KPL, void>(a, base + (r + u) * a.sq, x[u]);
#pragma unroll
      for (int u = 0; u < 16; ++u)
#pragma unroll
        for (int i = 0; i < KPL; ++i) sum[i] = __fadd_rn(sum[i], x[u][i]);
    }
    for (; r < w; ++r) {
      float x[KPL];
      load_keys<KPL, void>(a, base + r * a.sq, x);
#pragma unroll
      for (int i = 0; i < KPL; ++i) sum[i] = __fadd_rn(sum[i], x[i]);
    }
#pragma unroll
    for (int i = 0; i < KPL; ++i) hs[g][lane * KPL + i] = sum[i];
  }
  __syncthreads();
  if (slot == 0) {
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
      const int64_t j = j0 + i;
      if (j >= kv_len || j - jc >= KPL || j < jc) continue;
      float v = hs[0][lane * KPL + (int)(j - jc)];
      for (int g = 1; g < G; ++g) v = __fadd_rn(v, hs[g][lane * KPL + (int)(j - jc)]);
      votes[row * kv_len + j] = v;
    }
  }
}

// Pooled score of candidate j (0 <= j < n) of the row's candidates c[0 .. n):
// max pooling takes the max over c[j - pad .. j - pad + k - 1] inside [0, n)
// (padding never wins); average pooling adds the window's values left to right
// (padding counts as 0) and divides by k.
// Windows of up to kPoolUnroll: every neighbour is loaded first (indices clamped into
// the row, out-of-window values replaced after the load), then reduced in window order.
// A missing neighbour is -inf for the maximum, and +0 for the sum, which a running sum
// started at +0 never turns negative-zero, so both match the loop below bit for bit.
constexpr int kPoolUnroll = 8;
template <typename I>
__device__ __forceinline__ float pooled_unrolled(const float* c, I n, I j, int k, int mode) {
  const I lo = j - k / 2;
  float v[kPoolUnroll];
#pragma unroll
  for (int t = 0; t < kPoolUnroll; ++t) {
    const I x = lo + t;
    const float ld = c[x < 0 ? 0 : (x >= n ? n - 1 : x)];
    v[t] = (t < k && x >= 0 && x < n) ? ld : (mode == 0 ? -INFINITY : 0.f);
  }
  if (mode == 0) {
    float m = -INFINITY;
    bool nan = false;
#pragma unroll
    for (int t = 0; t < kPoolUnroll; ++t) {
      nan |= v[t] != v[t];
      m = fmaxf(m, v[t]);
    }
    return nan ? __int_as_float(0x7fc00000) : m;
  }
  float s = 0.f;
#pragma unroll
  for (int t = 0; t < kPoolUnroll; ++t)
    if (t < k) s = __fadd_rn(s, v[t]);
  return __fdiv_rn(s, (float)k);
}

template <typename I>
__device__ __forceinline__ float pooled(const float* c, I n, I j, int k, int mode) {
  if (k <= 1) return c[j];
  if (k <= kPoolUnroll) return pooled_unrolled<I>(c, n, j, k, mode);
  const I lo = j - k / 2;
  if (mode == 0) {
    float m = -INFINITY;
    bool nan = false;
    for (int t = 0; t < k; ++t) {
      const I x = lo + t;
      if (x < 0 || x >= n) continue;
      const float v = c[x];
      nan |= v != v;
      m = fmaxf(m, v);
    }
    return nan ? __int_as_float(0x7fc00000) : m;
  }
  float s = 0.f;
  for (int t = 0; t < k; ++t) {
    const I x = lo + t;
    if (x >= 0 && x < n) s = __fadd_rn(s, c[x]);
  }
  return __fdiv_rn(s, (float)k);
}

// Order-preserving key of a score: larger score, larger key; every NaN above +inf.
__device__ __forceinline__ uint32_t score_key(float v) {
  if (v != v) return 0xffffffffu;
  const uint32_t u = __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Exclusive prefix sum of v over the workgroup's threads (tid order); uses
// scratch[waves of the workgroup] and synchronizes the workgroup.
template <typename T>
__device__ __forceinline__ T block_exclusive_scan(T v, T* scratch) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  T inc = v;
  if constexpr (sizeof(T) == 4) {
    // 32-bit counts: DPP shifts away from lane 0 within each 16-lane row, then the
    // earlier rows' totals (their last lanes), all in the VALU
    inc += (T)__builtin_amdgcn_update_dpp(0, (int)inc, 0x111, 0xF, 0xF, false);
    inc += (T)__builtin_amdgcn_update_dpp(0, (int)inc, 0x112, 0xF, 0xF, false);
    inc += (T)__builtin_amdgcn_update_dpp(0, (int)inc, 0x114, 0xF, 0xF, false);
    inc += (T)__builtin_amdgcn_update_dpp(0, (int)inc, 0x118, 0xF, 0xF, false);
    const T t0 = (T)__builtin_amdgcn_readlane((int)inc, 15);
    const T t1 = (T)__builtin_amdgcn_readlane((int)inc, 31);
    const T t2 = (T)__builtin_amdgcn_readlane((int)inc, 47);
    const int r = lane >> 4;
    inc += (r > 0 ? t0 : 0) + (r > 1 ? t1 : 0) + (r > 2 ? t2 : 0);
  } else {
    for (int o = 1; o < 64; o <<= 1) {
      const T u = __shfl_up(inc, o);
      if (lane >= o) inc += u;
    }
  }
  if (lane == 63) scratch[wave] = inc;
  __syncthreads();
  T before = 0;
  for (int w = 0; w < wave; ++w) before += scratch[w];
  __syncthreads();
  return before + inc - v;
}

// Keys of the candidates: in LDS (staged once) when the row fits, else
// recomputed from the votes in global memory on every pass.
template <typename I>
struct KeySource {
  const float* c;
  I n;
  int pool_k, pool_mode;
  const uint32_t* lds;   // n keys, or null
  __device__ __forceinline__ uint32_t operator()(I j) const {
    return lds ? lds[j] : score_key(pooled<I>(c, n, j, pool_k, pool_mode));
  }
};

// One workgroup per (b, kv): sink positions, then the select_k best pooled
// candidates of [sink, recent_start) (ties: the earlier position), then the
// recent positions, in ascending order.  I: the candidates' index type, int for rows
// staged in LDS (at most kMaxStagedKeys candidates, 32-bit index arithmetic), int64_t
// for longer rows, whose keys are recomputed from global memory on every pass.
template <typename I>
__global__ void __launch_bounds__(kPickThreads)
select_kernel(const float* __restrict__ votes, int64_t kv_len, int64_t sink, int64_t recent_start,
              int64_t select_k, int pool_k, int pool_mode, int64_t* __restrict__ keep,
              int64_t budget) {
  constexpr bool staged = sizeof(I) == 4;
  extern __shared__ uint32_t lds_keys[];
  __shared__ uint32_t hist[256];
  __shared__ uint32_t s_prefix, s_mask, s_need;
  __shared__ I s_count[kPickThreads / 64];
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  const float* c = votes + row * kv_len + sink;
  const I n = (I)(recent_start - sink);
  int64_t* out = keep + row * budget;
  for (int64_t i = tid; i < sink; i += kPickThreads) out[i] = i;
  for (int64_t i = tid; i < kv_len - recent_start; i += kPickThreads)
    out[sink + select_k + i] = recent_start + i;
  if (select_k <= 0) return;
  KeySource<I> key_of{c, n, pool_k, pool_mode, nullptr};
  if constexpr (staged) {
    // the row's votes into LDS (8 loads in flight per thread), then the keys
    float* raw = reinterpret_cast<float*>(lds_keys + n);
    for (I j0 = tid; j0 < n; j0 += 8 * kPickThreads) {
      float x[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const I j = j0 + u * kPickThreads;
        x[u] = j < n ? c[j] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const I j = j0 + u * kPickThreads;
        if (j < n) raw[j] = x[u];
      }
    }
    __syncthreads();
    for (I j = tid; j < n; j += kPickThreads)
      lds_keys[j] = score_key(pooled<I>(raw, n, j, pool_k, pool_mode));
    key_of.lds = lds_keys;
  }
  // radix select of the select_k-th largest key, 8 bits at a time from the top
  if (tid == 0) {
    s_prefix = 0;
    s_mask = 0;
    s_need = (uint32_t)select_k;
  }
  __syncthreads();
  for (int shift = 24; shift >= 0; shift -= 8) {
    if (tid < 256) hist[tid] = 0;
    __syncthreads();
    const uint32_t prefix = s_prefix, mask = s_mask;
    for (I j = tid; j < n; j += kPickThreads) {
      const uint32_t key = key_of(j);
      if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
    }
    __syncthreads();
    // suffix sums of the histogram (thread t: keys with digit >= t), then the one
    // digit d with suffix(d) >= need > suffix(d + 1) is the threshold's digit
    // (threads 0..255, the first four waves, own one digit each)
    const uint32_t need = s_need;
    const bool digit = tid < 256;
    uint32_t suf = digit ? hist[tid] : 0u;
    // suffix sums within the wave, in the VALU: DPP shifts towards lane 0 within each
    // 16-lane row (lanes past the row's end add 0), then every row adds the later
    // rows' totals, read from their first lanes
    suf += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)suf, 0x101, 0xF, 0xF, false);
    suf += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)suf, 0x102, 0xF, 0xF, false);
    suf += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)suf, 0x104, 0xF, 0xF, false);
    suf += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)suf, 0x108, 0xF, 0xF, false);
    {
      const uint32_t t1 = __builtin_amdgcn_readlane(suf, 16);
      const uint32_t t2 = __builtin_amdgcn_readlane(suf, 32);
      const uint32_t t3 = __builtin_amdgcn_readlane(suf, 48);
      const int r = (tid & 63) >> 4;
      suf += (r < 1 ? t1 : 0u) + (r < 2 ? t2 : 0u) + (r < 3 ? t3 : 0u);
    }
    __syncthreads();
    if (digit) hist[tid] = suf;            // suffix within the wave
    __syncthreads();
    if (digit)
      for (int wv = (tid >> 6) + 1; wv < 4; ++wv) suf += hist[wv * 64];
    __syncthreads();
    if (digit) hist[tid] = suf;            // full suffix sums
    __syncthreads();
    const uint32_t next = tid < 255 ? hist[tid + 1] : 0u;
    if (digit && suf >= need && next < need) {
      s_prefix = prefix | ((uint32_t)tid << shift);
      s_mask = mask | (255u << shift);
      s_need = need - next;
    }
    __syncthreads();
  }
  // the threshold key and how many candidates equal to it are kept (the earliest)
  const uint32_t thr = s_prefix;
  const I take_equal = (I)s_need;
  // each thread scans one contiguous range: counts, then a block scan of the
  // counts gives each thread its first output slot
  const I per = (n + kPickThreads - 1) / kPickThreads;
  const I j0 = min<I>(n, tid * per), j1 = min<I>(n, j0 + per);
  I above = 0, equal = 0;
  for (I j = j0; j < j1; ++j) {
    const uint32_t key = key_of(j);
    above += key > thr;
    equal += key == thr;
  }
  // exclusive prefix of the equal counts decides which equal keys are taken
  const I eq_before = block_exclusive_scan<I>(equal, s_count);
  const I eq_take = max<I>(0, min<I>(equal, take_equal - eq_before));
  I slot = block_exclusive_scan<I>(above + eq_take, s_count);
  I eq_left = eq_take;
  for (I j = j0; j < j1; ++j) {
    const uint32_t key = key_of(j);
    bool take = key > thr;
    if (key == thr && eq_left > 0) {
      take = true;
      --eq_left;
    }
    if (take) out[sink + slot++] = sink + (int64_t)j;
  }
}

}  // namespace

extern "C" int pk_prompt_votes(const void* attention, int dtype, int64_t batch, int64_t num_q_heads,
                               int64_t q_len, int64_t kv_len, const int64_t* strides,
                               int num_kv_heads, int obs_window, float* votes, void* stream) {
  return pk::guarded("pk_prompt_votes", [&]() -> int {
    pk::clear_error();
    if (dtype != PK_DTYPE_F16 && dtype != PK_DTYPE_BF16 && dtype != PK_DTYPE_F32)
      return pk::fail("attention must be float16, bfloat16 or float32");
    if (batch <= 0 || num_q_heads <= 0 || q_len <= 0 || kv_len <= 0 || num_kv_heads <= 0)
      return pk::fail("attention shape and kv heads must be positive");
    if (num_q_heads % num_kv_heads) return pk::fail("query heads must be a multiple of kv heads");
    if (obs_window <= 0) return pk::fail("obs_window must be positive");
    if (!attention || !votes || !strides) return pk::fail("null pointer");
    if (num_q_heads / num_kv_heads > kMaxGroup) return pk::fail("more than 32 query heads per kv head");
    const int w = (int)std::min<int64_t>(obs_window, q_len);
    AttnView a{attention, dtype, strides[0], strides[1], strides[2], strides[3]};
    const int G = (int)(num_q_heads / num_kv_heads);
    // 4 keys per lane in one 8-byte load for 16-bit attention with contiguous,
    // 8-byte aligned key rows of a multiple of 4 keys; else one key per lane
    const bool vec = dtype != PK_DTYPE_F32 && strides[3] == 1 && kv_len % 4 == 0 &&
                     strides[0] % 4 == 0 && strides[1] % 4 == 0 && strides[2] % 4 == 0 &&
                     reinterpret_cast<uintptr_t>(attention) % 8 == 0;
    // 2 keys per lane (4-byte loads) when 4 per lane would leave CUs without a workgroup
    int kpl = vec ? 4 : 1;
    if (vec && batch * num_kv_heads * pk::cdiv(kv_len, 64 * 4) < pk::device_cu_count()) kpl = 2;
    const int64_t blocks = batch * num_kv_heads * pk::cdiv(kv_len, 64 * kpl);
    if (blocks > 0x7fffffff) return pk::fail("attention too large");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 threads(64 * std::min(G, kVotesMaxWaves));
    if (kpl == 4)
      hipLaunchKernelGGL(votes_kernel<4>, dim3((unsigned)blocks), threads, 0, s, a,
                         num_kv_heads, G, q_len, kv_len, w, votes);
    else if (kpl == 2)
      hipLaunchKernelGGL(votes_kernel<2>, dim3((unsigned)blocks), threads, 0, s, a,
                         num_kv_heads, G, q_len, kv_len, w, votes);
    else
      hipLaunchKernelGGL(votes_kernel<1>, dim3((unsigned)blocks), threads, 0, s, a,
                         num_kv_heads, G, q_len, kv_len, w, votes);
    return pk::check_launch("prompt_votes");
  });
}

extern "C" int pk_select_prompt(const float* votes, int64_t rows, int64_t kv_len, int64_t sink,
                                int64_t recent_start, int64_t select_k, int pool_kernel,
                                int pool_mode, int64_t* keep, void* stream) {
  return pk::guarded("pk_select_prompt", [&]() -> int {
    pk::clear_error();
    if (rows <= 0 || kv_len <= 0) return pk::fail("rows and kv_len must be positive");
    if (sink < 0 || recent_start < sink || recent_start > kv_len)
      return pk::fail("need 0 <= sink <= recent_start <= kv_len");
    if (select_k < 0 || select_k > recent_start - sink)
      return pk::fail("select_k must lie in [0, recent_start - sink]");
    if (pool_mode != 0 && pool_mode != 1) return pk::fail("pool_mode must be 0 (max) or 1 (avg)");
    if (!votes || !keep) return pk::fail("null pointer");
    const int64_t budget = sink + select_k + (kv_len - recent_start);
    const int64_t n = recent_start - sink;
    const bool staged = n <= kMaxStagedKeys;
    const size_t lds = staged ? (size_t)n * 8 : 0;
    static bool lds_opt_in = [] {
      return hipFuncSetAttribute(reinterpret_cast<const void*>(select_kernel<int>),
                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                 (int)(kMaxStagedKeys * 8)) == hipSuccess;
    }();
    if (staged && lds > 64 * 1024 && !lds_opt_in)
      return pk::fail("cannot reserve the selection kernel's LDS"), PK_ERR_RUNTIME;
    if (staged)
      hipLaunchKernelGGL(select_kernel<int>, dim3((unsigned)rows), dim3(kPickThreads), lds,
                         static_cast<hipStream_t>(stream), votes, kv_len, sink, recent_start,
                         select_k, pool_kernel, pool_mode, keep, budget);
    else
      hipLaunchKernelGGL(select_kernel<int64_t>, dim3((unsigned)rows), dim3(kPickThreads), 0,
                         static_cast<hipStream_t>(stream), votes, kv_len, sink, recent_start,
                         select_k, pool_kernel, pool_mode, keep, budget);
    return pk::check_launch("select_prompt");
  });
}
