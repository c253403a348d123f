// Sub-byte pack/unpack and grouped min/max quantization kernels (gfx950).
//
// Semantics follow src/phasekv/kernels/packing.py of the reference:
//   pack_low_bits      packing.py:41-64
//   unpack_low_bits    packing.py:67-79
//   quantize_pack      packing.py:115-155
//   unpack_dequantize  packing.py:158-175
// All float arithmetic is IEEE float32 with explicit round-to-nearest
// intrinsics (no contraction, no fast reciprocal) so the outputs are
// bit-identical to the reference run by torch.
#include "pk_common.h"
#include "pk_quant.h"

// No multiply-add contraction anywhere in this file: the reference multiplies
// and adds in separate float32 operations.
#pragma clang fp contract(off)

namespace {

constexpr int kThreads = 256;
// Element counts below this run the fast pack kernels with 32-bit index arithmetic (no
// 64-bit divisions per lane); larger tensors keep 64-bit indices.
constexpr int64_t kIndex32 = int64_t(1) << 31;
constexpr int kMaxDims = 8;

// ---------------------------------------------------------------------------
// pack / unpack of uint8 codes along the last axis
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(kThreads)
pack_low_bits_kernel(const uint8_t* __restrict__ codes, int64_t rows, int64_t length,
                     int bits, int64_t nbytes, uint8_t* __restrict__ out) {
  const int vpb = 8 / bits;
  const int64_t total = rows * nbytes;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / nbytes;
    const int64_t j = i - r * nbytes;
    const uint8_t* src = codes + r * length;
    uint32_t acc = 0;
    for (int k = 0; k < vpb; ++k) {
      const int64_t pos = j * vpb + k;
      if (pos < length) acc |= static_cast<uint32_t>(src[pos]) << (k * bits);
    }
    out[i] = static_cast<uint8_t>(acc);
  }
}

__global__ void __launch_bounds__(kThreads)
unpack_low_bits_kernel(const uint8_t* __restrict__ packed, int64_t rows, int64_t packed_len,
                       int bits, int64_t length, uint8_t* __restrict__ out) {
  const int vpb = 8 / bits;
  const uint32_t mask = (1u << bits) - 1u;
  const int64_t total = rows * length;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / length;
    const int64_t pos = i - r * length;
    const uint32_t byte = packed[r * packed_len + pos / vpb];
    out[i] = static_cast<uint8_t>((byte >> ((pos % vpb) * bits)) & mask);
  }
}

// ---------------------------------------------------------------------------
// quantize_pack
// ---------------------------------------------------------------------------
struct QuantParams {
  const void* x;
  int dtype;
  int npre;                       // number of non-axis dims
  int64_t pre_size[kMaxDims];
  int64_t pre_stride[kMaxDims];
  int64_t ax_stride;
  int64_t len;
  int bits;
  int gs;
  int64_t ngroups;
  int64_t nbytes;
  int64_t rows;
  int rows_fastest;               // thread index -> (row fastest) or (group fastest)
  int meta_gm;                    // scale/mins group major over the last dim (axis == ndim - 2)
  int codes_tm;                   // codes token-byte major over the last dim (axis == ndim - 2)
  int64_t meta_d;                 // that last dim
  uint8_t* packed;
  uint16_t* scale;
  uint16_t* mins;
};

__device__ __forceinline__ int64_t row_offset(const QuantParams& p, int64_t r) {
  int64_t off = 0;
  for (int d = p.npre - 1; d >= 0; --d) {
    const int64_t sz = p.pre_size[d];
    const int64_t idx = r % sz;
    r /= sz;
    off += idx * p.pre_stride[d];
  }
  return off;
}

// Element of scale / mins for (row, group): channel major [rows][ngroups], or
// group major [rows / D][ngroups][D] (row = outer * D + channel).
__device__ __forceinline__ int64_t meta_index(const QuantParams& p, int64_t r, int64_t g) {
  if (!p.meta_gm) return r * p.ngroups + g;
  const int64_t o = r / p.meta_d;
  return (o * p.ngroups + g) * p.meta_d + (r - o * p.meta_d);
}

// Byte b of row r of the codes: [rows][nbytes], or [rows / D][nbytes][D].
__device__ __forceinline__ int64_t code_index(const QuantParams& p, int64_t r, int64_t b) {
  if (!p.codes_tm) return r * p.nbytes + b;
  const int64_t o = r / p.meta_d;
  return (o * p.nbytes + b) * p.meta_d + (r - o * p.meta_d);
}

__device__ __forceinline__ float load_x(const QuantParams& p, int64_t off) {
  if (p.dtype == PK_DTYPE_F16) return pk_h2f(static_cast<const uint16_t*>(p.x)[off]);
  if (p.dtype == PK_DTYPE_BF16) return pk_bf2f(static_cast<const uint16_t*>(p.x)[off]);
  return static_cast<const float*>(p.x)[off];
}

using pk::GroupStats;
using pk::nan_max;
using pk::nan_min;
using pk::quant_code;

// Statistics of group g of the row at base offset `off`.  The reference pads the
// tail group with copies of the last element, which changes neither its min nor
// its max, so only the real elements are scanned.
__device__ __forceinline__ GroupStats group_stats(const QuantParams& p, int64_t off, int64_t g) {
  const int64_t begin = g * p.gs;
  const int64_t end = min(begin + p.gs, p.len);
  float mn = load_x(p, off + begin * p.ax_stride);
  float mx = mn;
  for (int64_t i = begin + 1; i < end; ++i) {
    const float v = load_x(p, off + i * p.ax_stride);
    mn = nan_min(mn, v);
    mx = nan_max(mx, v);
  }
  return pk::group_stats_from(mn, mx, p.bits);
}

// One thread per (row, group) when whole groups cover whole bytes (gs % vpb == 0).
__global__ void __launch_bounds__(kThreads)
quantize_groups_kernel(QuantParams p) {
  const int vpb = 8 / p.bits;
  const int64_t total = p.rows * p.ngroups;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    int64_t r, g;
    if (p.rows_fastest) { g = i / p.rows; r = i - g * p.rows; }
    else { r = i / p.ngroups; g = i - r * p.ngroups; }
    const int64_t off = row_offset(p, r);
    const GroupStats s = group_stats(p, off, g);
    p.scale[meta_index(p, r, g)] = pk_f2h(s.scale);
    p.mins[meta_index(p, r, g)] = pk_f2h(s.mn);
    const int64_t begin = g * p.gs;
    const int64_t end = min(begin + p.gs, p.len);
    for (int64_t b0 = begin; b0 < end; b0 += vpb) {
      uint32_t byte = 0;
      for (int k = 0; k < vpb; ++k) {
        const int64_t pos = b0 + k;
        if (pos < end) byte |= quant_code(load_x(p, off + pos * p.ax_stride), s, p.bits) << (k * p.bits);
      }
      p.packed[code_index(p, r, b0 / vpb)] = static_cast<uint8_t>(byte);
    }
  }
}

// ---------------------------------------------------------------------------
// Fast paths for the cache's own layouts: fp16 input, contiguous, groups of 32.
// Same arithmetic as group_stats / quant_code, element for element.
// ---------------------------------------------------------------------------
typedef uint32_t pk_u4 __attribute__((ext_vector_type(4)));

// The 32 values of a group are spread over a lane quad (quarter = lane & 3,
// tokens or channels 8q .. 8q + 7), so a launch has four times the waves of a
// thread-per-group kernel and each wave fewer loads in its chain.  Min / max:
// each lane folds its eight values in order, then the quad combines them as
// ((0, 1), (2, 3)) with the earlier quarter on the left.  nan_min / nan_max keep
// their left operand on ties and take a NaN right operand, so this tree picks
// the same element (sign of zero and NaN included) as the sequential fold over
// all 32 values.  Quarter q then packs its eight codes into bytes
// q * BITS .. q * BITS + BITS - 1 of the group (LSB-first along the group).
__device__ __forceinline__ void quad_minmax(float& mn, float& mx, int quarter) {
#pragma unroll
  for (int o = 1; o <= 2; o <<= 1) {
    const float pmn = __shfl_xor(mn, o), pmx = __shfl_xor(mx, o);
    const bool first = (quarter & o) == 0;
    mn = first ? nan_min(mn, pmn) : nan_min(pmn, mn);
    mx = first ? nan_max(mx, pmx) : nan_max(pmx, mx);
  }
}

__device__ __forceinline__ GroupStats quad_stats(const float (&v)[8], int quarter, int bits) {
  float mn = v[0], mx = v[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) {
    mn = nan_min(mn, v[i]);
    mx = nan_max(mx, v[i]);
  }
  quad_minmax(mn, mx, quarter);
  return pk::group_stats_from(mn, mx, bits);
}

template <int BITS>
__device__ __forceinline__ uint64_t pack8(const float (&v)[8], const GroupStats& s) {
  uint64_t x = 0;
#pragma unroll
  for (int t = 0; t < 8; ++t) x |= static_cast<uint64_t>(quant_code(v[t], s, BITS)) << (t * BITS);
  return x;
}

// BITS bytes of one quarter (dst is BITS-aligned for 2 and 4 bits, 4-aligned for 8)
template <int BITS>
__device__ __forceinline__ void store_quarter(uint8_t* dst, uint64_t x) {
  if constexpr (BITS == 2) {
    *reinterpret_cast<uint16_t*>(dst) = static_cast<uint16_t>(x);
  } else if constexpr (BITS == 4) {
    *reinterpret_cast<uint32_t*>(dst) = static_cast<uint32_t>(x);
  } else {
    reinterpret_cast<uint32_t*>(dst)[0] = static_cast<uint32_t>(x);
    reinterpret_cast<uint32_t*>(dst)[1] = static_cast<uint32_t>(x >> 32);
  }
}

// Groups along the contiguous axis (V, per token along head_dim): a lane quad
// per (row, group), the group index fastest; each lane one 16-byte load.
// `block` / `nblocks`: this workgroup's place in the part of the grid doing this work.
template <int BITS, typename I>
__device__ __forceinline__ void inner32_body(const uint16_t* __restrict__ x, int64_t rows,
                                             int64_t len, int64_t ngroups, int64_t nbytes,
                                             uint8_t* __restrict__ packed,
                                             uint16_t* __restrict__ scale,
                                             uint16_t* __restrict__ mins, int64_t block,
                                             int64_t nblocks) {
  const I total = (I)(rows * ngroups * 4);     // whole quads: every quad runs one iteration
  const I ng = (I)ngroups;
  for (I i = (I)(block * blockDim.x + threadIdx.x); i < total; i += (I)(nblocks * blockDim.x)) {
    const int quarter = (int)(i & 3);
    const I j = i >> 2;
    const I r = j / ng, g = j - r * ng;
    const pk_u4 q = *reinterpret_cast<const pk_u4*>(x + (r * (I)len + g * 32 + quarter * 8));
    float v[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[2 * k] = pk_h2f((uint16_t)(q[k] & 0xFFFFu));
      v[2 * k + 1] = pk_h2f((uint16_t)(q[k] >> 16));
    }
    const GroupStats st = quad_stats(v, quarter, BITS);
    if (quarter == 0) {
      scale[j] = pk_f2h(st.scale);
      mins[j] = pk_f2h(st.mn);
    }
    store_quarter<BITS>(packed + (r * (I)nbytes + g * 4 * BITS + quarter * BITS), pack8<BITS>(v, st));
  }
}

template <int BITS, typename I>
__global__ void __launch_bounds__(kThreads)
quantize_inner32_kernel(const uint16_t* __restrict__ x, int64_t rows, int64_t len, int64_t ngroups,
                        int64_t nbytes, uint8_t* __restrict__ packed, uint16_t* __restrict__ scale,
                        uint16_t* __restrict__ mins) {
  inner32_body<BITS, I>(x, rows, len, ngroups, nbytes, packed, scale, mins, blockIdx.x, gridDim.x);
}

// Groups along the second-innermost axis with a contiguous innermost dim D
// (K, per channel along tokens): a lane quad per (outer, group, channel pair),
// quarter fastest, then the channel pair, so each load instruction of a wave
// reads 64-byte runs of four token rows; each quad stores two channels' packed
// group and metadata.
template <int BITS, typename I>
__device__ __forceinline__ void outer32_body(const uint16_t* __restrict__ x, int64_t outer,
                                             int64_t len, int64_t D, int64_t ngroups,
                                             int64_t nbytes, uint8_t* __restrict__ packed,
                                             uint16_t* __restrict__ scale,
                                             uint16_t* __restrict__ mins, int meta_gm,
                                             int codes_tm, int64_t block, int64_t nblocks) {
  const I pairs = (I)(D / 2), ng = (I)ngroups, Di = (I)D;
  const I total = (I)(outer * ngroups * (D / 2) * 4);
  for (I i = (I)(block * blockDim.x + threadIdx.x); i < total; i += (I)(nblocks * blockDim.x)) {
    const int quarter = (int)(i & 3);
    const I rest = i >> 2;
    const I rest2 = rest / pairs;
    const I cp = rest - rest2 * pairs;
    const I o = rest2 / ng;
    const I g = rest2 - o * ng;
    const uint32_t* src =
        reinterpret_cast<const uint32_t*>(x + ((o * (I)len + g * 32 + quarter * 8) * Di + 2 * cp));
    float a[8], b[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const uint32_t q = src[t * (D / 2)];
      a[t] = pk_h2f((uint16_t)(q & 0xFFFFu));
      b[t] = pk_h2f((uint16_t)(q >> 16));
    }
    uint64_t code[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const float (&v)[8] = k ? b : a;
      const GroupStats st = quad_stats(v, quarter, BITS);
      const I row = o * Di + 2 * cp + k;
      if (quarter == 0) {
        const I mi = meta_gm ? (o * ng + g) * Di + 2 * cp + k : row * ng + g;
        scale[mi] = pk_f2h(st.scale);
        mins[mi] = pk_f2h(st.mn);
      }
      code[k] = pack8<BITS>(v, st);
      if (!codes_tm)
        store_quarter<BITS>(packed + (row * (I)nbytes + g * 4 * BITS + quarter * BITS), code[k]);
    }
    if (codes_tm) {
      // byte jj of the quarter for both channels: one 2-byte store into [bytes][D]
      uint8_t* base = packed + ((o * (I)nbytes + g * 4 * BITS + quarter * BITS) * Di + 2 * cp);
#pragma unroll
      for (int jj = 0; jj < BITS; ++jj) {
        const uint32_t lo = static_cast<uint32_t>(code[0] >> (8 * jj)) & 0xFFu;
        const uint32_t hi = static_cast<uint32_t>(code[1] >> (8 * jj)) & 0xFFu;
        *reinterpret_cast<uint16_t*>(base + jj * Di) = (uint16_t)(lo | (hi << 8));
      }
    }
  }
}

template <int BITS, typename I>
__global__ void __launch_bounds__(kThreads)
quantize_outer32_kernel(const uint16_t* __restrict__ x, int64_t outer, int64_t len, int64_t D,
                        int64_t ngroups, int64_t nbytes, uint8_t* __restrict__ packed,
                        uint16_t* __restrict__ scale, uint16_t* __restrict__ mins, int meta_gm,
                        int codes_tm) {
  outer32_body<BITS, I>(x, outer, len, D, ngroups, nbytes, packed, scale, mins, meta_gm, codes_tm,
                        blockIdx.x, gridDim.x);
}

// The cache's K/V block pack in one launch: workgroups [0, k_blocks) pack K
// [B, H, S, D] per channel along tokens (token-major codes, group-major
// metadata), the rest pack V per token along head_dim.
struct KVPackArgs {
  const uint16_t* k; const uint16_t* v;
  int64_t outer, S, D;
  uint8_t* kp; uint16_t* ks; uint16_t* km;
  uint8_t* vp; uint16_t* vs; uint16_t* vm;
  int k_blocks;
};

template <int BITS, typename I>
__global__ void __launch_bounds__(kThreads)
quantize_kv32_kernel(const KVPackArgs a) {
  if ((int)blockIdx.x < a.k_blocks)
    outer32_body<BITS, I>(a.k, a.outer, a.S, a.D, a.S / 32, a.S * BITS / 8, a.kp, a.ks, a.km, 1,
                          1, blockIdx.x, a.k_blocks);
  else
    inner32_body<BITS, I>(a.v, a.outer * a.S, a.D, a.D / 32, a.D * BITS / 8, a.vp, a.vs, a.vm,
                          blockIdx.x - a.k_blocks, gridDim.x - a.k_blocks);
}

// General group sizes: metadata per (row, group) ...
__global__ void __launch_bounds__(kThreads)
quantize_meta_kernel(QuantParams p) {
  const int64_t total = p.rows * p.ngroups;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / p.ngroups;
    const int64_t g = i - r * p.ngroups;
    const GroupStats s = group_stats(p, row_offset(p, r), g);
    p.scale[meta_index(p, r, g)] = pk_f2h(s.scale);
    p.mins[meta_index(p, r, g)] = pk_f2h(s.mn);
  }
}

// ... and codes per (row, output byte); a byte may straddle groups.
__global__ void __launch_bounds__(kThreads)
quantize_bytes_kernel(QuantParams p) {
  const int vpb = 8 / p.bits;
  const int64_t total = p.rows * p.nbytes;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / p.nbytes;
    const int64_t j = i - r * p.nbytes;
    const int64_t off = row_offset(p, r);
    uint32_t byte = 0;
    int64_t cur_g = -1;
    GroupStats s{0.f, 1.f};
    for (int k = 0; k < vpb; ++k) {
      const int64_t pos = j * vpb + k;
      if (pos >= p.len) break;
      const int64_t g = pos / p.gs;
      if (g != cur_g) { s = group_stats(p, off, g); cur_g = g; }
      byte |= quant_code(load_x(p, off + pos * p.ax_stride), s, p.bits) << (k * p.bits);
    }
    p.packed[code_index(p, r, j)] = static_cast<uint8_t>(byte);
  }
}

// ---------------------------------------------------------------------------
// unpack_dequantize: one thread per output element in the original layout
// ---------------------------------------------------------------------------
struct DequantParams {
  const uint8_t* packed;
  const uint16_t* scale;
  const uint16_t* mins;
  int ndim;
  int axis;
  int64_t shape[kMaxDims];
  int64_t len;
  int64_t nbytes;
  int64_t ngroups;
  int bits;
  int gs;
  int64_t total;
  uint16_t* out;
};

__global__ void __launch_bounds__(kThreads)
unpack_dequantize_kernel(DequantParams p) {
  const int vpb = 8 / p.bits;
  const uint32_t mask = (1u << p.bits) - 1u;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < p.total;
       e += (int64_t)gridDim.x * blockDim.x) {
    int64_t rem = e, r = 0, rmul = 1, j = 0;
    for (int d = p.ndim - 1; d >= 0; --d) {
      const int64_t idx = rem % p.shape[d];
      rem /= p.shape[d];
      if (d == p.axis) { j = idx; }
      else { r += idx * rmul; rmul *= p.shape[d]; }
    }
    const uint32_t byte = p.packed[r * p.nbytes + j / vpb];
    const float code = static_cast<float>((byte >> ((j % vpb) * p.bits)) & mask);
    const int64_t g = j / p.gs;
    const float sc = pk_h2f(p.scale[r * p.ngroups + g]);
    const float mn = pk_h2f(p.mins[r * p.ngroups + g]);
    p.out[e] = pk_f2h(__fadd_rn(__fmul_rn(code, sc), mn));
  }
}

inline int grid_for(int64_t total) {
  const int64_t blocks = pk::cdiv(total, kThreads);
  const int64_t cap = static_cast<int64_t>(pk::device_cu_count()) * 32;
  return static_cast<int>(blocks < cap ? (blocks > 0 ? blocks : 1) : cap);
}

}  // namespace

// ---------------------------------------------------------------------------
// C entry points
// ---------------------------------------------------------------------------
extern "C" int pk_pack_low_bits(const uint8_t* codes, int64_t rows, int64_t length, int bits,
                                uint8_t* out, void* stream) {
  return pk::guarded("pk_pack_low_bits", [&]() -> int {
    pk::clear_error();
    if (!pk::valid_bits(bits)) return pk::fail("bits must be one of (2, 4, 8)");
    if (rows < 0 || length < 0) return pk::fail("rows and length must be non-negative");
    const int64_t nbytes = pk::cdiv(length, 8 / bits);
    if (rows * nbytes == 0) return PK_OK;
    if (!codes || !out) return pk::fail("null pointer");
    hipLaunchKernelGGL(pack_low_bits_kernel, dim3(grid_for(rows * nbytes)), dim3(kThreads), 0,
                       static_cast<hipStream_t>(stream), codes, rows, length, bits, nbytes, out);
    return pk::check_launch("pack_low_bits");
  });
}

extern "C" int pk_unpack_low_bits(const uint8_t* packed, int64_t rows, int64_t packed_len,
                                  int bits, int64_t length, uint8_t* out, void* stream) {
  return pk::guarded("pk_unpack_low_bits", [&]() -> int {
    pk::clear_error();
    if (!pk::valid_bits(bits)) return pk::fail("bits must be one of (2, 4, 8)");
    if (rows < 0 || length < 0 || packed_len < 0) return pk::fail("sizes must be non-negative");
    if (length > packed_len * (8 / bits)) return pk::fail("length exceeds the packed codes");
    if (rows * length == 0) return PK_OK;
    if (!packed || !out) return pk::fail("null pointer");
    hipLaunchKernelGGL(unpack_low_bits_kernel, dim3(grid_for(rows * length)), dim3(kThreads), 0,
                       static_cast<hipStream_t>(stream), packed, rows, packed_len, bits, length, out);
    return pk::check_launch("unpack_low_bits");
  });
}

extern "C" int pk_quantize_pack(const void* x, int dtype, int ndim, const int64_t* shape,
                                const int64_t* strides, int axis, int bits, int group_size,
                                uint8_t* out_packed, uint16_t* out_scale, uint16_t* out_mins,
                                int layout, void* stream) {
  return pk::guarded("pk_quantize_pack", [&]() -> int {
    pk::clear_error();
    if (!pk::valid_bits(bits)) return pk::fail("bits must be one of (2, 4, 8)");
    if (dtype != PK_DTYPE_F16 && dtype != PK_DTYPE_BF16 && dtype != PK_DTYPE_F32)
      return pk::fail("x must be float16, bfloat16 or float32");
    if (ndim < 1 || ndim > kMaxDims) return pk::fail("x must have 1..8 dims");
    if (axis < 0 || axis >= ndim) return pk::fail("axis out of range");
    if (layout & ~(PK_LAYOUT_META_TRANSPOSED | PK_LAYOUT_CODES_TRANSPOSED))
      return pk::fail("unknown layout flags");
    if (layout && (ndim < 2 || axis != ndim - 2))
      return pk::fail("transposed storage needs axis == ndim - 2");
    QuantParams p{};
    p.x = x;
    p.meta_gm = (layout & PK_LAYOUT_META_TRANSPOSED) != 0;
    p.codes_tm = (layout & PK_LAYOUT_CODES_TRANSPOSED) != 0;
    p.meta_d = ndim >= 2 ? shape[ndim - 1] : 1;
    p.dtype = dtype;
    p.len = shape[axis];
    p.ax_stride = strides[axis];
    p.rows = 1;
    int n = 0;
    for (int d = 0; d < ndim; ++d) {
      if (shape[d] < 0) return pk::fail("negative dimension");
      if (d == axis) continue;
      p.pre_size[n] = shape[d];
      p.pre_stride[n] = strides[d];
      p.rows *= shape[d];
      ++n;
    }
    p.npre = n;
    if (p.len <= 0 || p.rows == 0) {
      if (p.len <= 0) return pk::fail("quantized axis must be non-empty");
      return PK_OK;
    }
    if (group_size <= 0 || group_size > p.len) return pk::fail("group_size must be in [1, len]");
    if (!x || !out_packed || !out_scale || !out_mins) return pk::fail("null pointer");
    p.bits = bits;
    p.gs = group_size;
    p.ngroups = pk::cdiv(p.len, group_size);
    p.nbytes = pk::cdiv(p.len, 8 / bits);
    // Threads walk adjacent rows when the quantized axis is not the contiguous one,
    // so neighbouring lanes read neighbouring addresses.
    p.rows_fastest = (p.ax_stride != 1) ? 1 : 0;
    p.packed = out_packed;
    p.scale = out_scale;
    p.mins = out_mins;
    hipStream_t s = static_cast<hipStream_t>(stream);
    // the cache's layouts: fp16, contiguous, whole groups of 32 along the last or
    // second-to-last axis
    bool contiguous = true;
    {
      int64_t expect = 1;
      for (int d = ndim - 1; d >= 0; --d) {
        if (shape[d] != 1 && strides[d] != expect) contiguous = false;
        expect *= shape[d];
      }
    }
    const bool fast = dtype == PK_DTYPE_F16 && contiguous && group_size == 32 && p.len % 32 == 0 &&
                      reinterpret_cast<uintptr_t>(x) % 16 == 0;
    if (fast && axis == ndim - 1 && !layout) {
      const int64_t lanes = p.rows * p.ngroups * 4;
      const bool i32 = p.rows * p.len < kIndex32;   // every element and byte index fits int
  #define PK_INNER(B, I) hipLaunchKernelGGL((quantize_inner32_kernel<B, I>), dim3(grid_for(lanes)), \
                                            dim3(kThreads), 0, s, static_cast<const uint16_t*>(x), p.rows, \
                                            p.len, p.ngroups, p.nbytes, out_packed, out_scale, out_mins)
      if (i32) {
        if (bits == 2) PK_INNER(2, int); else if (bits == 4) PK_INNER(4, int); else PK_INNER(8, int);
      } else {
        if (bits == 2) PK_INNER(2, int64_t); else if (bits == 4) PK_INNER(4, int64_t); else PK_INNER(8, int64_t);
      }
  #undef PK_INNER
      return pk::check_launch("quantize_pack");
    }
    if (fast && axis == ndim - 2 && shape[ndim - 1] % 2 == 0) {
      const int64_t D = shape[ndim - 1];
      const int64_t outer = p.rows / D;
      const int64_t threads = outer * p.ngroups * (D / 2) * 4;
      const bool i32 = p.rows * p.len < kIndex32;
  #define PK_OUTER(B, I) hipLaunchKernelGGL((quantize_outer32_kernel<B, I>), dim3(grid_for(threads)), \
                                            dim3(kThreads), 0, s, static_cast<const uint16_t*>(x), outer, \
                                            p.len, D, p.ngroups, p.nbytes, out_packed, out_scale, out_mins, \
                                            p.meta_gm, p.codes_tm)
      if (i32) {
        if (bits == 2) PK_OUTER(2, int); else if (bits == 4) PK_OUTER(4, int); else PK_OUTER(8, int);
      } else {
        if (bits == 2) PK_OUTER(2, int64_t); else if (bits == 4) PK_OUTER(4, int64_t); else PK_OUTER(8, int64_t);
      }
  #undef PK_OUTER
      return pk::check_launch("quantize_pack");
    }
    if (group_size % (8 / bits) == 0) {
      hipLaunchKernelGGL(quantize_groups_kernel, dim3(grid_for(p.rows * p.ngroups)),
                         dim3(kThreads), 0, s, p);
    } else {
      hipLaunchKernelGGL(quantize_meta_kernel, dim3(grid_for(p.rows * p.ngroups)), dim3(kThreads),
                         0, s, p);
      int rc = pk::check_launch("quantize_pack(meta)");
      if (rc) return rc;
      hipLaunchKernelGGL(quantize_bytes_kernel, dim3(grid_for(p.rows * p.nbytes)), dim3(kThreads),
                         0, s, p);
    }
    return pk::check_launch("quantize_pack");
  });
}

extern "C" int pk_quantize_pack_kv(const uint16_t* k, const uint16_t* v, int batch,
                                   int num_kv_heads, int64_t seq_len, int head_dim, int bits,
                                   uint8_t* k_packed, uint16_t* k_scale, uint16_t* k_mins,
                                   uint8_t* v_packed, uint16_t* v_scale, uint16_t* v_mins,
                                   void* stream) {
  return pk::guarded("pk_quantize_pack_kv", [&]() -> int {
    pk::clear_error();
    if (!pk::valid_bits(bits)) return pk::fail("bits must be one of (2, 4, 8)");
    if (!k || !v || !k_packed || !k_scale || !k_mins || !v_packed || !v_scale || !v_mins)
      return pk::fail("null K / V / output pointer");
    if (batch <= 0 || num_kv_heads <= 0 || seq_len <= 0 || head_dim <= 0)
      return pk::fail("batch, num_kv_heads, seq_len and head_dim must be positive");
    if (seq_len % 32 || head_dim % 32)
      return pk::fail("the one-launch K/V pack needs seq_len and head_dim multiples of 32");
    if (reinterpret_cast<uintptr_t>(k) % 16 || reinterpret_cast<uintptr_t>(v) % 16 ||
        reinterpret_cast<uintptr_t>(k_packed) % 4 || reinterpret_cast<uintptr_t>(v_packed) % 4)
      return pk::fail("K / V must be 16-byte aligned and the code buffers 4-byte aligned");
    KVPackArgs a{k, v, (int64_t)batch * num_kv_heads, seq_len, head_dim, k_packed, k_scale,
                 k_mins, v_packed, v_scale, v_mins, 0};
    const int64_t k_lanes = a.outer * (seq_len / 32) * (head_dim / 2) * 4;
    const int64_t v_lanes = a.outer * seq_len * (head_dim / 32) * 4;
    a.k_blocks = grid_for(k_lanes);
    const int grid = a.k_blocks + grid_for(v_lanes);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool i32 = a.outer * seq_len * head_dim < kIndex32;   // K and V indices fit int
    if (i32) {
      if (bits == 2)
        hipLaunchKernelGGL((quantize_kv32_kernel<2, int>), dim3(grid), dim3(kThreads), 0, s, a);
      else if (bits == 4)
        hipLaunchKernelGGL((quantize_kv32_kernel<4, int>), dim3(grid), dim3(kThreads), 0, s, a);
      else
        hipLaunchKernelGGL((quantize_kv32_kernel<8, int>), dim3(grid), dim3(kThreads), 0, s, a);
    } else {
      if (bits == 2)
        hipLaunchKernelGGL((quantize_kv32_kernel<2, int64_t>), dim3(grid), dim3(kThreads), 0, s, a);
      else if (bits == 4)
        hipLaunchKernelGGL((quantize_kv32_kernel<4, int64_t>), dim3(grid), dim3(kThreads), 0, s, a);
      else
        hipLaunchKernelGGL((quantize_kv32_kernel<8, int64_t>), dim3(grid), dim3(kThreads), 0, s, a);
    }
    return pk::check_launch("quantize_pack_kv");
  });
}

extern "C" int pk_unpack_dequantize(const uint8_t* packed, const uint16_t* scale,
                                    const uint16_t* mins, int ndim, const int64_t* orig_shape,
                                    int axis, int bits, int group_size, int64_t n_groups,
                                    uint16_t* out, void* stream) {
  return pk::guarded("pk_unpack_dequantize", [&]() -> int {
    pk::clear_error();
    if (!pk::valid_bits(bits)) return pk::fail("bits must be one of (2, 4, 8)");
    if (ndim < 1 || ndim > kMaxDims) return pk::fail("orig_shape must have 1..8 dims");
    if (axis < 0 || axis >= ndim) return pk::fail("axis out of range");
    DequantParams p{};
    p.ndim = ndim;
    p.axis = axis;
    p.total = 1;
    for (int d = 0; d < ndim; ++d) {
      if (orig_shape[d] < 0) return pk::fail("negative dimension");
      p.shape[d] = orig_shape[d];
      p.total *= orig_shape[d];
    }
    p.len = orig_shape[axis];
    if (p.total == 0) return PK_OK;
    if (group_size <= 0) return pk::fail("group_size must be positive");
    if (n_groups * group_size < p.len) return pk::fail("scale/mins hold fewer groups than the axis needs");
    if (!packed || !scale || !mins || !out) return pk::fail("null pointer");
    p.packed = packed;
    p.scale = scale;
    p.mins = mins;
    p.bits = bits;
    p.gs = group_size;
    p.ngroups = n_groups;
    p.nbytes = pk::cdiv(p.len, 8 / bits);
    p.out = out;
    hipLaunchKernelGGL(unpack_dequantize_kernel, dim3(grid_for(p.total)), dim3(kThreads), 0,
                       static_cast<hipStream_t>(stream), p);
    return pk::check_launch("unpack_dequantize");
  });
}
