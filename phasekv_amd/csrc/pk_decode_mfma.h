// MFMA decode attention over packed KIVI segments and FP16 segments (gfx950).
//
// Same work list, partial layout and combine as the generic kernel; this file
// is the fast path for head_dim 64 / 128, KIVI segments with group size 32 (or
// a single group) and FP16 segments.  Reference semantics: the per-segment
// kernel src/phasekv/kernels/attention_triton.py:514-596 and the FP16 hot
// partial attention_triton.py:285-297.
//
// One workgroup = 4 waves = one (chunk, batch row, kv head, head slab).  Each
// wave takes 32-token groups (one K quantization group) of the chunk round
// robin, keeps its own online softmax state and prefetches its next group
// while computing the current one; the waves merge through LDS and the
// workgroup writes one partial.
//
// Math per 32-token quantization group (K is packed per channel, V per token):
//   scores  S^T[t][h] = sum_c code_K[t][c] * (q[h][c] * sK[c][g])  +  sum_c q[h][c] * mK[c][g]
//   output  O^T[c][h] = sum_t code_V[t][c] * (p[t][h] * sV[t][cg]) +  sum_t p[t][h] * mV[t][cg]
// so the per-channel K scale is folded into q and the per-token V scale into
// p; the code matrices go straight into v_mfma_f32_16x16x32_f16.
//
// Codes reach the MFMA without any int->float conversion: a byte permute puts
// two codes (two channels of one token for K, two tokens of one channel for
// V) into the low bits of the two fp16 halves of a register and an AND keeps
// them.  An fp16 with exponent field 0 is the subnormal  mantissa * 2^-24,
// so the register holds  code * 2^(24 - position bits)  exactly; the matrix
// cores take fp16 subnormals without flushing, and the power-of-two factors
// are undone on the fp32 results (per score row, per output row).
//
// MFMA 16x16x32 f16 operand layout (lane l, slot j): A[l%16][8*(l/16)+j],
// B[8*(l/16)+j][l%16]; result D[4*(l/16)+e][l%16] in register e.
#pragma once

#include "pk_common.h"
#include "pk_decode.h"

#include <math.h>

#include <algorithm>

namespace pk {
namespace {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u2_t __attribute__((ext_vector_type(2)));

constexpr int kWaves = 4;
constexpr int kTile = 32;            // tokens per wave step (one K group)
constexpr float kTwo24 = 16777216.0f;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr uint32_t kOnes2 = 0x3C003C00u;   // fp16 pair (1.0, 1.0)

__device__ __forceinline__ f4_t mfma(u4_t a, u4_t b, f4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8_t, a),
                                                __builtin_bit_cast(h8_t, b), c, 0, 0, 0);
}

// result byte k <- selector byte k: 0..3 pick bytes of `lo`, 4..7 bytes of `hi`, 0x0c gives 0
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

// selector: byte b of lo -> byte 0, byte b of hi -> byte 2, zeros elsewhere
__device__ __forceinline__ uint32_t sel_bytes(int b) {
  return (uint32_t)b | (0x0cu << 8) | ((uint32_t)(4 + b) << 16) | (0x0cu << 24);
}

// selector: half hh of lo -> low half, half hh of hi -> high half
__device__ __forceinline__ uint32_t sel_halves(int hh) {
  const uint32_t b = 2u * hh;
  return b | ((b + 1) << 8) | ((b + 4) << 16) | ((b + 5) << 24);
}

__device__ __forceinline__ uint32_t pkmul(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2_t, a) * __builtin_bit_cast(h2_t, b));
}

// a * b - c with one rounding (v_pk_fma_f16): the residual of c = fp16(a * b)
__device__ __forceinline__ uint32_t pkfms(uint32_t a, uint32_t b, uint32_t c) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(h2_t, a),
                                                                __builtin_bit_cast(h2_t, b),
                                                                -__builtin_bit_cast(h2_t, c)));
}

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, a), __builtin_bit_cast(h2_t, b), c, false);
}

__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
  h2_t v = {(_Float16)a, (_Float16)b};
  return __builtin_bit_cast(uint32_t, v);
}

// Sums / maxima over the four 16-lane rows of a wave that hold the same head
// column: v_permlane16_swap and v_permlane32_swap exchange rows in the VALU,
// with no trip through the LDS crossbar.
__device__ __forceinline__ float xsum4(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  const float v2 = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v2), __float_as_uint(v2), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

__device__ __forceinline__ float xmax4(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  const float v2 = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v2), __float_as_uint(v2), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// One of two uniform base pointers per lane, as an offset select: a select of
// the pointers themselves can be lowered through a small stack array.
template <typename T>
__device__ __forceinline__ const T* pick(bool first, const T* a, const T* b) {
  return a + (first ? (ptrdiff_t)0 : (b - a));
}

__device__ __forceinline__ u4_t lds_u4(const char* p) { return *reinterpret_cast<const u4_t*>(p); }
__device__ __forceinline__ u2_t lds_u2(const char* p) { return *reinterpret_cast<const u2_t*>(p); }
__device__ __forceinline__ uint32_t lds_u32(const char* p) { return *reinterpret_cast<const uint32_t*>(p); }

// Running softmax state of one wave (lane = head column n, lane group g4).
template <int HD>
struct WaveAcc {
  f4_t o[HD / 16];     // O^T blocks: rows 4*g4 + e of channel block b, column = head
  f4_t vbl;            // KIVI: matrix-core accumulator, row c < HD/32 = sum_t p mV of channel
                       // group c, row HD/32 = sum_t p (rows 4*g4 + e as for o)
  float m;             // reference max of p = 2^(s - m), log2 units, same in the 4 lane groups
  float mx;            // true running max of the scores
  float l;             // FP16 segments: sum_t p (this lane's tokens)
};

// The reference max only moves when a group's max exceeds it by more than
// kLazyLog2, so p = 2^(s - m) <= 2^kLazyLog2 stays well inside fp16 and the
// accumulators are rescaled only when some head of the wave needs it (a
// wave-uniform branch), instead of every group.  Returns the reference max to
// use for this group's p.
constexpr float kLazyLog2 = 8.0f;

template <int HD>
__device__ __forceinline__ float lazy_rescale(WaveAcc<HD>& acc, float mt, float lazy = kLazyLog2) {
  acc.mx = fmaxf(acc.mx, mt);
  const bool grow = mt > acc.m + lazy;
  if (__any(grow)) {
    const float m_new = grow ? mt : acc.m;
    const float alpha = __builtin_amdgcn_exp2f(acc.m - m_new);
    acc.m = m_new;
    acc.l *= alpha;
    acc.vbl *= alpha;
#pragma unroll
    for (int b = 0; b < HD / 16; ++b) acc.o[b] *= alpha;
  }
  return acc.m;
}

// ---------------------------------------------------------------------------
// fp16 range of the folded operands.  q * sK and p * sV are rounded to fp16 for
// the matrix cores.
//  * q is normalized per workgroup: q' = q * 2^-e with 2^e >= max |q| of the
//    workgroup's heads (e >= 0), and 2^e goes into the score factor.  Then
//    |q' * sK| <= sK <= 65504: the K fold cannot overflow.
//  * p = 2^(s - m) reaches 2^kLazyLog2, so p * sV stays in fp16 while sV <=
//    255.875.  Each staged group's V scales are checked as they are stored (one
//    compare per token); a group with a larger scale runs with lazy bound 0
//    (p <= 1, so p * sV <= sV <= 65504).
// ---------------------------------------------------------------------------
// LDS written by the lanes of a wave, then read by other lanes of the same wave:
// a wave's LDS operations run in order, so only the compiler must not move them
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

constexpr uint32_t kVScaleSafe = 0x5BFFu;   // 255.875: 2^8 times it stays below 65504

// largest of the four fp16 bit patterns (non-negative values compare as integers)
__device__ __forceinline__ uint32_t hmax4(u2_t x) {
  const uint32_t a = max(x[0] & 0xffffu, x[0] >> 16), b = max(x[1] & 0xffffu, x[1] >> 16);
  return max(a, b);
}

// The workgroup's q normalization exponent e: the smallest e >= 0 with every |q| of
// the lane's registers and of the wave (every wave holds all heads of the
// workgroup) at most 2^e.
// UP: also negative e, the smallest e with every |q| at most 2^e (largest |q'| in
// (1/2, 1]; e >= -15 for any fp16 q).
template <int KS, bool UP = false>
__device__ __forceinline__ int q_norm_shift(const u4_t (&qb)[KS]) {
  uint32_t m = 0;
#pragma unroll
  for (int s = 0; s < KS; ++s)
#pragma unroll
    for (int j = 0; j < 4; ++j) m = max(m, hmax4(u2_t{qb[s][j] & 0x7fff7fffu, 0u}));
  // over the wave: within rows of 16 lanes by DPP (quad swaps, half-row and row
  // mirrors), then across the 4 rows by permlane swaps, all in the VALU
  m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0xB1, 0xF, 0xF, false));
  m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x4E, 0xF, 0xF, false));
  m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x141, 0xF, 0xF, false));
  m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x140, 0xF, 0xF, false));
  {
    const auto a = __builtin_amdgcn_permlane16_swap(m, m, false, false);
    m = max(a[0], a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(m, m, false, false);
    m = max(b[0], b[1]);
  }
  // fp16 bits: exponent field (m >> 10) - 15, rounded up unless m is a power of two;
  // inf / NaN: the largest finite exponent (the result is not finite anyway)
  m = __builtin_amdgcn_readfirstlane(min(m, 0x7BFFu));
  const int e = (int)(m >> 10) - 15 + ((m & 0x3ffu) ? 1 : 0);
  return (UP || e > 0) ? e : 0;
}

// q' = q * 2^-e (|q'| <= 1) and sl2 * 2^e: the K fold q' * sK stays in fp16.  Called
// by the KIVI paths after their first group's loads are issued (it waits for q).
template <int HD, bool UP = false>
__device__ __forceinline__ void normalize_q(u4_t (&qb)[HD / 32], float& sl2) {
  const int e = q_norm_shift<HD / 32, UP>(qb);
  const uint32_t f = pack_h2(ldexpf(1.f, -e), ldexpf(1.f, -e));
#pragma unroll
  for (int k = 0; k < HD / 32; ++k)
#pragma unroll
    for (int m = 0; m < 4; ++m) qb[k][m] = pkmul(qb[k][m], f);
  // (uniform: a score factor held in a VGPR would cost registers in every loop)
  sl2 = __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(ldexpf(sl2, e))));
}

// Whether this lane's V scales (4 halves) keep p * sV in fp16 at the lazy bound.
__device__ __forceinline__ bool vscale_big(bool has_v, u2_t vscale) {
  return has_v && hmax4(vscale) > kVScaleSafe;
}

// ---------------------------------------------------------------------------
// LDS staging of a 128-token stage: four 32-token groups, one per wave.  The
// workgroup loads a stage together, in 16-byte pieces where the rows allow,
// because the token-packed K codes and the per-channel K scales put every
// channel in its own cache line: one wide request per channel and stage costs
// far fewer L1 -> L2 requests than one narrow request per channel and group.
// The store to LDS transposes what the matrix operands need transposed:
//   Kw  uint32 [4 KB][HD + 16/KB]  word w of every channel's K codes; the row
//                                  padding puts the KB pieces a wave stores
//                                  at once in distinct banks (channel-major codes)
//   Kt  bytes [16 KB][HD + 16]     token-major codes as stored: byte row j holds
//                                  the j-th code byte of every channel
//   Ks, Km  fp16 [4][HD]           K scale / min of the stage's groups
//   V   VB = 8: [128][HD*VB/8] the stage's V rows as stored.  VB = 2, 4: per
//       group [word w][byte b][token pair tp] uint32 = (byte b of word w of
//       token 2 tp, 0, the same byte of token 2 tp + 1, 0): the PV operand
//       pairs of one channel, so the matrix operand is one AND of a 16-byte
//       read (groups padded by 16 words so the stores spread over the banks)
//   Vs  fp16 [HD/32][128]          V scale, channel group major
//   Vm  fp16 [HD/32 + 1][128]      V min, channel group major; the extra row
//                                  holds ones (the sum_t p row of the bias product)
// ---------------------------------------------------------------------------
constexpr int kStage = 128;

template <int HD, int KB, int VB>
struct StageLayout {
  static constexpr int kw_row = HD + 16 / KB;             // words per Kw row
  // token-major codes: 16 KB byte rows of HD channels; the 8-byte pad puts rows
  // r and r + 8 of an operand read in different banks
  static constexpr int kt_pitch = HD + 8;
  static constexpr int kt_bytes = 16 * KB * kt_pitch;
  static constexpr int kw_bytes = (4 * KB * kw_row * 4 > kt_bytes) ? 4 * KB * kw_row * 4 : kt_bytes;
  static constexpr int off_ks = kw_bytes;
  static constexpr int off_km = off_ks + 4 * HD * 2;
  static constexpr int off_vw = off_km + 4 * HD * 2;
  static constexpr int vrow_words = HD * VB / 32;
  static constexpr int vrow_bytes = HD * VB / 8;
  static constexpr bool vspread = VB != 8;
  // spread V (per group of 16 token pairs): dword (word w, byte b, token pair tp)
  // at 64 s + 16 b + (tp ^ vswz(s, b)), s = vslot(w).  A lane stores the PW words
  // of one slice qw of a token pair (NQ slices per row), and words are
  // interleaved by slice, s = (w % PW) NQ + w / PW, so s and qw have the same
  // parity.  With the store order of the byte rows (one half of the slices
  // stores them as 1 0 3 2) the 32 stores of a half wave hit 32 banks, and the
  // swizzle (bit 3 of tp, which keeps runs of 4 token pairs contiguous) puts
  // byte rows b and b + 2 of an operand read in different banks.
  static constexpr int vpw = (vrow_words >= 16) ? 4 : 2;
  static constexpr int vnq = vrow_words / vpw;
  static constexpr int vgrp_words = vrow_words * 64;           // spread group stride (words)
  // 8-bit V rows padded by 16 bytes: the token rows 4 apart that one half wave
  // reads sit 16 banks apart
  static constexpr int vrow_pitch = vrow_bytes + 16;
  static constexpr int vw_bytes = vspread ? 4 * vgrp_words * 4 : kStage * vrow_pitch;
  // V scale / min rows of kStage tokens, padded so the rows of the bias
  // operand read start 4 banks apart
  static constexpr int vms = kStage + 8;
  static constexpr int off_vs = off_vw + vw_bytes;
  static constexpr int off_vm = off_vs + (HD / 32) * vms * 2;
  // uint32 per group: nonzero if a V scale of the group is above kVScaleSafe
  static constexpr int off_vbig = (off_vm + (HD / 32 + 1) * vms * 2 + 3) & ~3;
  static constexpr int bytes = off_vbig + 16;
  __device__ static constexpr int vslot(int w) { return (w % vpw) * vnq + w / vpw; }
  __device__ static constexpr int vswz(int s, int b) { return 8 * ((s ^ (b >> 1)) & 1); }
};

// One lane's share of a stage's global loads (256 lanes).
template <int HD, int KB, int VB>
struct StageRegs {
  static constexpr int KP = HD * KB;                      // 16-byte K pieces (KB per channel)
  static constexpr int NK = (KP + kThreads - 1) / kThreads;
  static constexpr int VP = HD * VB;                      // 16-byte V pieces (the stage's rows)
  static constexpr int NV = (VP + kThreads - 1) / kThreads;
  // spread V (VB = 2, 4): items (token pair, PW-word slice of both rows), slice fastest
  static constexpr int W = HD * VB / 32;                  // words per V row
  static constexpr int PW = (W >= 16) ? 4 : 2;
  static constexpr int NQ = W / PW;                       // slices per row
  static constexpr int VI = 64 * NQ;                      // items per stage
  static constexpr int NVI = (VI + kThreads - 1) / kThreads;
  static constexpr bool spread = VB != 8;
  u4_t k[NK];
  u4_t v[spread ? 1 : NV];
  u4_t va[spread ? NVI : 1], vb[spread ? NVI : 1];   // slices of tokens 2 tp and 2 tp + 1
  u2_t km;     // lanes < 2 HD: the 4 group scales (lane < HD) or mins of channel lane % HD
  u2_t vm;     // V scales (lanes < 128) or mins of token lane % 128 (HD = 64: low word only)
};

// V slice loads of a stage (spread layout): rows 2 tp and 2 tp + 1, clamped to t_last
template <int HD, int KB, int VB>
__device__ __forceinline__ void load_vslices(StageRegs<HD, KB, VB>& r, const uint8_t* vseg, int ts,
                                             int t_last, int tid) {
  using R = StageRegs<HD, KB, VB>;
  constexpr int RB = HD * VB / 8;
#pragma unroll
  for (int i = 0; i < R::NVI; ++i) {
    const int q = (tid + kThreads * i) % R::VI;
    const int tp = q / R::NQ, qw = q - tp * R::NQ;
    const int ta = min(ts + 2 * tp, t_last), tb = min(ts + 2 * tp + 1, t_last);
    const uint8_t* pa = vseg + (int64_t)ta * RB + qw * R::PW * 4;
    const uint8_t* pb = vseg + (int64_t)tb * RB + qw * R::PW * 4;
    if constexpr (R::PW == 4) {
      r.va[i] = *reinterpret_cast<const u4_t*>(pa);
      r.vb[i] = *reinterpret_cast<const u4_t*>(pb);
    } else {
      const u2_t a = *reinterpret_cast<const u2_t*>(pa);
      const u2_t b = *reinterpret_cast<const u2_t*>(pb);
      r.va[i] = u4_t{a[0], a[1], 0u, 0u};
      r.vb[i] = u4_t{b[0], b[1], 0u, 0u};
    }
  }
}

struct SegOffsets {
  int64_t kd, km, vd, vm;
};

// How a segment's K rows can be read: 16-byte pieces, dwords or bytes.
struct KivLoad {
  int64_t row_bytes;   // bytes of one channel's K codes
  int row_groups;      // K groups per channel
  int kmode;           // 16, 4 or 1
  bool kmeta4;         // channel major: the 4 group scales of a stage are one aligned 8-byte load
  bool kmeta_gm;       // group major: a stage's scales are [4][HD] contiguous (8-byte loads)
  bool gm_elems;       // group major but not 8-byte aligned: per-element loads
  bool kdata_tm;       // token-major K codes: a stage is 16 KB rows of HD bytes, contiguous
  int64_t k_rows;      // token-major: code byte rows of the segment
};

// K scale/min of a stage: in lane order.  Channel major: lane (tensor, channel)
// holds the stage's 4 groups of its channel.  Group major: lane (tensor, group,
// channel quad) holds 4 channels of one group, stored as read (no transpose).
template <int HD>
__device__ __forceinline__ u2_t load_kmeta(const SegDev& s, const SegOffsets& o, const KivLoad& kl,
                                           int ts, int tid) {
  const int g0 = min(ts / 32, kl.row_groups - 1);
  if (kl.kmeta_gm) {
    const int q = tid & (2 * HD - 1);
    const int g = min(g0 + (q & (HD - 1)) / (HD / 4), kl.row_groups - 1);
    const int c4 = q & (HD / 4 - 1);
    const uint16_t* m = pick(q < HD, s.ks, s.km) + o.km + (int64_t)g * HD + 4 * c4;
    return *reinterpret_cast<const u2_t*>(m);
  }
  const int c = tid % HD;
  const uint16_t* base = pick((tid & (2 * HD - 1)) < HD, s.ks, s.km) + o.km;
  if (kl.gm_elems) {
    uint32_t x[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) x[g] = base[(int64_t)min(g0 + g, kl.row_groups - 1) * HD + c];
    return u2_t{x[0] | (x[1] << 16), x[2] | (x[3] << 16)};
  }
  const uint16_t* m = base + (int64_t)c * kl.row_groups;
  if (kl.kmeta4) return *reinterpret_cast<const u2_t*>(m + g0);
  uint32_t x[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) x[g] = m[min(g0 + g, kl.row_groups - 1)];
  return u2_t{x[0] | (x[1] << 16), x[2] | (x[3] << 16)};
}

// Loads of the stage starting at token ts (ts - segment start is a multiple of
// 32).  Addresses stay inside the segment: K pieces past a row's end are not
// loaded (their codes only feed masked scores), V rows and metadata are
// clamped to the last valid token t_last, K metadata to the last group.
template <int HD, int KB, int VB>
__device__ __forceinline__ void load_stage(StageRegs<HD, KB, VB>& r, const SegDev& s,
                                           const SegOffsets& o, const KivLoad& kl, int ts,
                                           int t_last, int tid) {
  using R = StageRegs<HD, KB, VB>;
  using L = StageLayout<HD, KB, VB>;
  const int64_t byte0 = (int64_t)ts * KB / 8;
  const uint8_t* krows = s.kd + o.kd;
  if (kl.kdata_tm) {
    // the stage's byte rows are contiguous; pieces past the last row repeat it
    const int64_t last = (kl.k_rows - byte0) * (HD / 16) - 1;
#pragma unroll
    for (int i = 0; i < R::NK; ++i) {
      const int q = tid + kThreads * i;
      if (R::KP % kThreads == 0 || q < R::KP)
        r.k[i] = *reinterpret_cast<const u4_t*>(krows + byte0 * HD + min((int64_t)q, last) * 16);
    }
  } else
#pragma unroll
  for (int i = 0; i < R::NK; ++i) {
    const int q = tid + kThreads * i;
    if (R::KP % kThreads == 0 || q < R::KP) {
      const int c = q / KB, j = q - c * KB;
      const int64_t off = byte0 + 16 * j;
      const uint8_t* src = krows + c * kl.row_bytes + off;
      u4_t v = {0u, 0u, 0u, 0u};
      if (kl.kmode == 16) {
        if (off < kl.row_bytes) v = *reinterpret_cast<const u4_t*>(src);
      } else if (kl.kmode == 4) {
#pragma unroll
        for (int w = 0; w < 4; ++w)
          if (off + 4 * w < kl.row_bytes) v[w] = *reinterpret_cast<const uint32_t*>(src + 4 * w);
      } else {
#pragma unroll
        for (int bt = 0; bt < 16; ++bt)
          if (off + bt < kl.row_bytes) v[bt >> 2] |= (uint32_t)src[bt] << (8 * (bt & 3));
      }
      r.k[i] = v;
    }
  }
  if (tid < 2 * HD) r.km = load_kmeta<HD>(s, o, kl, ts, tid);
  if constexpr (R::spread) {
    load_vslices<HD, KB, VB>(r, s.vd + o.vd, ts, t_last, tid);
  } else {
    const int last_piece = (t_last - ts + 1) * (L::vrow_bytes / 16) - 1;
    const uint8_t* vsrc = s.vd + o.vd + (int64_t)ts * L::vrow_bytes;
#pragma unroll
    for (int i = 0; i < R::NV; ++i) {
      const int q = tid + kThreads * i;
      if (R::VP % kThreads == 0 || q < R::VP)
        r.v[i] = *reinterpret_cast<const u4_t*>(vsrc + (int64_t)min(q, last_piece) * 16);
    }
  }
  {
    const int t = min(ts + (tid & (kStage - 1)), t_last);
    const uint16_t* m = pick(tid < kStage, s.vs, s.vm) + o.vm + (int64_t)t * (HD / 32);
    if (HD == 128) {
      r.vm = *reinterpret_cast<const u2_t*>(m);
    } else {
      r.vm = u2_t{*reinterpret_cast<const uint32_t*>(m), 0u};
    }
  }
}

// Per-lane offsets of the fast stage loads, fixed for a segment.
template <int HD, int KB, int VB>
struct FastOffsets {
  uint32_t krow[StageRegs<HD, KB, VB>::NK];   // channel row start of each K piece
  uint32_t mrow;                             // K metadata: channel-major lane offset (elements)
  uint32_t mgrp;                             // K metadata, group major: the lane's group in the stage
  uint32_t mcol;                             // K metadata, group major: the lane's first channel
};

// Stage loads for segments whose K rows are 16-byte aligned and hold a
// multiple of 128 tokens' K groups: every lane issues the same loads, with no
// predicate and no branch, so the compiler's wait counts stay exact and the
// next stages' loads are not waited for.  Lanes without a piece of their own
// (head_dim 64) load a neighbour's, which the store skips.
template <int HD, int KB, int VB>
__device__ __forceinline__ void load_stage_fast(StageRegs<HD, KB, VB>& r, const SegDev& s,
                                                const SegOffsets& o, const KivLoad& kl,
                                                const FastOffsets<HD, KB, VB>& fo, int ts,
                                                int t_last, int tid) {
  using R = StageRegs<HD, KB, VB>;
  using L = StageLayout<HD, KB, VB>;
  const uint32_t byte0 = (uint32_t)ts * KB / 8;
  const uint32_t kmax = (uint32_t)kl.row_bytes - 16;
  const uint8_t* krows = s.kd + o.kd;
  // token-major: the stage's rows are contiguous from byte0 * HD, the last piece
  // repeated past the segment's last row; channel-major: one row span per channel
  const uint32_t tlast = (uint32_t)((kl.k_rows - byte0) * (HD / 16)) - 1;
#pragma unroll
  for (int i = 0; i < R::NK; ++i) {
    const uint32_t q = (uint32_t)((tid + kThreads * i) & (R::KP - 1));
    const uint32_t kj = 16u * ((tid + kThreads * i) % KB);   // piece within the row span
    const uint32_t off = kl.kdata_tm ? byte0 * HD + 16u * min(q, tlast)
                                     : fo.krow[i] + min(byte0 + kj, kmax);
    r.k[i] = *reinterpret_cast<const u4_t*>(krows + off);
  }
  {
    // both layouts are one aligned 8-byte load per lane; group major clamps the
    // lane's group to the segment's last one
    const int q = tid & (2 * HD - 1);
    const uint16_t* m = pick(q < HD, s.ks, s.km) + o.km;
    const uint32_t g = min((uint32_t)(ts / 32) + fo.mgrp, (uint32_t)kl.row_groups - 1u);
    const uint32_t off = kl.kmeta_gm ? g * HD + fo.mcol : fo.mrow + (uint32_t)(ts / 32);
    r.km = *reinterpret_cast<const u2_t*>(m + off);
  }
  if constexpr (R::spread) {
    load_vslices<HD, KB, VB>(r, s.vd + o.vd, ts, t_last, tid);
  } else {
    const int last_piece = (t_last - ts + 1) * (L::vrow_bytes / 16) - 1;
    const uint8_t* vsrc = s.vd + o.vd + (int64_t)ts * L::vrow_bytes;
#pragma unroll
    for (int i = 0; i < R::NV; ++i) {
      const int q = (tid + kThreads * i) & (R::VP - 1);
      r.v[i] = *reinterpret_cast<const u4_t*>(vsrc + min(q, last_piece) * 16);
    }
  }
  {
    const int t = min(ts + (tid & (kStage - 1)), t_last);
    const uint16_t* m = pick(tid < kStage, s.vs, s.vm) + o.vm + (int64_t)t * (HD / 32);
    if (HD == 128) r.vm = *reinterpret_cast<const u2_t*>(m);
    else r.vm = u2_t{*reinterpret_cast<const uint32_t*>(m), 0u};
  }
}

template <int HD, int KB, int VB>
__device__ __forceinline__ void store_stage(const StageRegs<HD, KB, VB>& r, bool kmeta_gm,
                                            bool kdata_tm, int tid, char* st) {
  using L = StageLayout<HD, KB, VB>;
  using R = StageRegs<HD, KB, VB>;
  {
    // lanes < kStage hold the V scales of token tid: waves 0 and 1 flag the
    // stage's groups 0, 1 and 2, 3 (32 lanes each)
    const uint64_t big = __ballot(vscale_big(tid < kStage, r.vm));
    if ((tid & 63) == 0 && tid < kStage) {
      uint32_t* f = reinterpret_cast<uint32_t*>(st + L::off_vbig) + 2 * (tid >> 6);
      f[0] = (uint32_t)big;
      f[1] = (uint32_t)(big >> 32);
    }
  }
  uint32_t* kw = reinterpret_cast<uint32_t*>(st);
  if (kdata_tm) {
#pragma unroll
    for (int i = 0; i < R::NK; ++i) {
      const int q = tid + kThreads * i;
      if (R::KP % kThreads == 0 || q < R::KP) {
        u2_t* dst = reinterpret_cast<u2_t*>(st + (q / (HD / 16)) * L::kt_pitch + (q % (HD / 16)) * 16);
        dst[0] = u2_t{r.k[i][0], r.k[i][1]};
        dst[1] = u2_t{r.k[i][2], r.k[i][3]};
      }
    }
  } else
#pragma unroll
  for (int i = 0; i < R::NK; ++i) {
    const int q = tid + kThreads * i;
    if (R::KP % kThreads == 0 || q < R::KP) {
      const int c = q / KB, j = q - c * KB;
#pragma unroll
      for (int w = 0; w < 4; ++w) kw[(4 * j + w) * L::kw_row + c] = r.k[i][w];
    }
  }
  if (tid < 2 * HD) {
    uint16_t* m = reinterpret_cast<uint16_t*>(st + ((tid < HD) ? L::off_ks : L::off_km));
    if (kmeta_gm) {
      // lane (tensor, group, channel quad): already [group][channel]
      const int q = tid & (HD - 1);
      *reinterpret_cast<u2_t*>(m + (q / (HD / 4)) * HD + 4 * (q & (HD / 4 - 1))) = r.km;
    } else {
      const int c = tid % HD;
#pragma unroll
      for (int g = 0; g < 4; ++g) m[g * HD + c] = (uint16_t)(r.km[g >> 1] >> (16 * (g & 1)));
    }
  }
  if constexpr (R::spread) {
    uint32_t* vsp = reinterpret_cast<uint32_t*>(st + L::off_vw);
#pragma unroll
    for (int i = 0; i < R::NVI; ++i) {
      const int q = tid + kThreads * i;
      if (R::VI % kThreads == 0 || q < R::VI) {
        const int tp = q / R::NQ, qw = q - tp * R::NQ;
        // slices in the upper half of each 4 (NQ = 4) or 2 (NQ = 2) store byte rows 1 0 3 2
        const int flip = ((R::NQ == 4) ? (qw >> 1) : qw) & 1;
        uint32_t* dst = vsp + (tp >> 4) * L::vgrp_words + qw * 64;
#pragma unroll
        for (int k = 0; k < R::PW; ++k)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int b = j ^ flip;
            // slot k NQ + qw has the parity of qw; b >> 1 == j >> 1
            const int sw = 8 * ((qw ^ (j >> 1)) & 1);
            dst[k * R::NQ * 64 + b * 16 + ((tp & 15) ^ sw)] = perm(r.vb[i][k], r.va[i][k], sel_bytes(b));
          }
      }
    }
  } else {
    constexpr int PR = L::vrow_bytes / 16;   // 16-byte pieces per row
#pragma unroll
    for (int i = 0; i < R::NV; ++i) {
      const int q = tid + kThreads * i;
      if (R::VP % kThreads == 0 || q < R::VP)
        *reinterpret_cast<u4_t*>(st + L::off_vw + (q / PR) * L::vrow_pitch + (q % PR) * 16) = r.v[i];
    }
  }
  {
    uint16_t* m = reinterpret_cast<uint16_t*>(st + ((tid < kStage) ? L::off_vs : L::off_vm));
    const int t = tid & (kStage - 1);
#pragma unroll
    for (int cg = 0; cg < HD / 32; ++cg)
      m[cg * L::vms + t] = (uint16_t)(r.vm[cg >> 1] >> (16 * (cg & 1)));
  }
}

// token (within the group) of QK result row rr of instance h
template <int KB>
__device__ __forceinline__ int qk_token(int h, int rr) {
  if (KB == 2) return 4 * (rr >> 1) + 2 * h + (rr & 1);
  if (KB == 4) return 2 * rr + h;
  return 16 * h + rr;
}

// power-of-two factor the K code of result row rr carries (2^(bit position))
template <int KB>
__device__ __forceinline__ float qk_posfactor(int h, int e) {
  if (KB == 2) return (float)(1 << (2 * (2 * h + (e & 1))));
  if (KB == 4) return h ? 16.0f : 1.0f;
  return 1.0f;
}

// token of the lane's PV slot j
template <int KB>
__device__ __forceinline__ int pv_token(int g4, int j) {
  if (KB == 8) return 16 * (j >> 2) + 4 * g4 + (j & 3);
  return 8 * g4 + j;
}

// PV slot of QK result (h, e)
template <int KB>
__device__ __forceinline__ int pv_slot(int h, int e) {
  if (KB == 2) return 4 * (e >> 1) + 2 * h + (e & 1);
  if (KB == 4) return 2 * e + h;
  return 4 * h + e;
}

// ---------------------------------------------------------------------------
// one staged 32-token KIVI group, in two phases: kivi_qk reads the group's K
// codes and K scale / min rows, kivi_softmax_pv its V codes and V scale / min
// rows, so a wave can run the QK phase of its next group before the softmax
// and PV phase of the current one
// ---------------------------------------------------------------------------
// QK phase result: the raw S^T accumulators of instances h = 0, 1 (codes times
// q', before the position and score factors) and the K-min bias in log2 units.
struct QkOut {
  f4_t d[2];
  float bias;
  float lazy;   // the group's lazy bound (kLazyLog2, or 0 for large V scales)
};

template <int HD, int KB, typename L>
__device__ __forceinline__ QkOut kivi_qk(const char* st, int grp, bool ktm,
                                         const u4_t (&qb)[HD / 32], float sl2, int lane,
                                         float lazy) {
  const char* kwg = st + grp * KB * L::kw_row * 4;        // the group's Kw rows
  const char* ktg = st + grp * 4 * KB * L::kt_pitch;      // the group's Kt byte rows
  const char* ksg = st + L::off_ks + grp * HD * 2;
  const char* kmg = st + L::off_km + grp * HD * 2;
  constexpr int KS = HD / 32;
  const int r = lane & 15;     // A row (token row) / B column (head)
  const int g4 = lane >> 4;
  // ---- the K-min bias sum_c q mK on the matrix cores (every A row holds the
  // mins, so every result row is the bias) ----
  f4_t db = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < KS; ++s) db = mfma(lds_u4(kmg + (32 * s + 8 * g4) * 2), qb[s], db);
  const float bias = db[0] * sl2;
  // ---- q folded with the group's K scale, channels 32 s .. 32 s + 31: q' = q * sK
  // as an fp16 pair, qp (rounded) + ql (its residual, also fp16), so the scores
  // carry q * sK to about 22 bits; the codes times each part are exact ----
  auto fold = [&](int s, u4_t& qp, u4_t& ql) {
    const u4_t sc8 = lds_u4(ksg + (32 * s + 8 * g4) * 2);
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      qp[m] = pkmul(qb[s][m], sc8[m]);
      ql[m] = pkfms(qb[s][m], sc8[m], qp[m]);
    }
  };
  // (kept apart from the products below: interleaved by the scheduler, the two
  // loops' LDS reads held enough registers to spill)
  __builtin_amdgcn_sched_barrier(0);
  // ---- S^T = codes_K * q' for instances h = 0, 1 (16 tokens each) ----
  f4_t d[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
  if (ktm) {
    // token-major codes: one 8-byte read gives this lane's 8 channels of a code
    // byte row; byte pairs (2m, 2m + 1) go to the two fp16 halves of operand m
    uint32_t mask[2];
    if (KB == 2) {
      mask[0] = 0x00030003u << (2 * (r & 1));
      mask[1] = 0x00030003u << (2 * (2 + (r & 1)));
    } else {
      mask[0] = 0x000F000Fu;
      mask[1] = 0x00F000F0u;
    }
    const uint32_t sel0 = 0u | (0x0cu << 8) | (1u << 16) | (0x0cu << 24);
    const uint32_t sel1 = 2u | (0x0cu << 8) | (3u << 16) | (0x0cu << 24);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      u4_t qp, ql;
      fold(s, qp, ql);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        // code byte row of token qk_token(h, r): r / 2 (2-bit), r (4-bit), 16 h + r (8-bit)
        if (KB != 8 && h == 1) break;
        const int row = (KB == 2) ? (r >> 1) : (KB == 4) ? r : 16 * h + r;
        const u2_t x = lds_u2(ktg + row * L::kt_pitch + 32 * s + 8 * g4);
        uint32_t u[4];
        u[0] = perm(x[0], x[0], sel0);
        u[1] = perm(x[0], x[0], sel1);
        u[2] = perm(x[1], x[1], sel0);
        u[3] = perm(x[1], x[1], sel1);
        if constexpr (KB == 8) {
          d[h] = mfma(u4_t{u[0], u[1], u[2], u[3]}, qp, d[h]);
          d[h] = mfma(u4_t{u[0], u[1], u[2], u[3]}, ql, d[h]);
        } else {
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            u4_t a;
#pragma unroll
            for (int m = 0; m < 4; ++m) a[m] = u[m] & mask[hh];
            d[hh] = mfma(a, qp, d[hh]);
            d[hh] = mfma(a, ql, d[hh]);
          }
        }
      }
    }
  } else if constexpr (KB == 8) {
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      u4_t qp, ql;
      fold(s, qp, ql);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int w = 4 * h + (r >> 2);
        const uint32_t sel = sel_bytes(r & 3);
        const u4_t w0 = lds_u4(kwg + (w * L::kw_row + 32 * s + 8 * g4) * 4);
        const u4_t w1 = lds_u4(kwg + (w * L::kw_row + 32 * s + 8 * g4 + 4) * 4);
        u4_t a;
        a[0] = perm(w0[1], w0[0], sel);
        a[1] = perm(w0[3], w0[2], sel);
        a[2] = perm(w1[1], w1[0], sel);
        a[3] = perm(w1[3], w1[2], sel);
        d[h] = mfma(a, qp, d[h]);
        d[h] = mfma(a, ql, d[h]);
      }
    }
  } else {
    const int w = (KB == 2) ? (r >> 3) : (r >> 2);
    const uint32_t sel = sel_bytes(KB == 2 ? ((r >> 1) & 3) : (r & 3));
    uint32_t mask[2];
    if (KB == 2) {
      mask[0] = 0x00030003u << (2 * (r & 1));
      mask[1] = 0x00030003u << (2 * (2 + (r & 1)));
    } else {
      mask[0] = 0x000F000Fu;
      mask[1] = 0x00F000F0u;
    }
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      u4_t qp, ql;
      fold(s, qp, ql);
      const u4_t w0 = lds_u4(kwg + (w * L::kw_row + 32 * s + 8 * g4) * 4);
      const u4_t w1 = lds_u4(kwg + (w * L::kw_row + 32 * s + 8 * g4 + 4) * 4);
      uint32_t u[4];
      u[0] = perm(w0[1], w0[0], sel);
      u[1] = perm(w0[3], w0[2], sel);
      u[2] = perm(w1[1], w1[0], sel);
      u[3] = perm(w1[3], w1[2], sel);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        u4_t a;
#pragma unroll
        for (int m = 0; m < 4; ++m) a[m] = u[m] & mask[h];
        d[h] = mfma(a, qp, d[h]);
        d[h] = mfma(a, ql, d[h]);
      }
    }
  }
  return QkOut{{d[0], d[1]}, bias, lazy};
}

// Online softmax of one group's scores and O^T += codes_V^T * (p * sV) + the
// V-min bias, from the group's V codes and V scale / min rows in LDS.
template <int HD, int KB, int VB, bool FULL, typename L>
__device__ __forceinline__ void kivi_softmax_pv(const QkOut& qk, int nvalid, const char* st,
                                                int grp, WaveAcc<HD>& acc, float sl2, int lane) {
  const char* vsg = st + L::off_vs + grp * kTile * 2;     // channel group stride vms
  const char* vmg = st + L::off_vm + grp * kTile * 2;
  constexpr int NB = HD / 16;
  constexpr int CG = HD / 32;
  const int r = lane & 15;
  const int g4 = lane >> 4;
  const f4_t (&d)[2] = qk.d;
  const float bias = qk.bias;
  // ---- scores (log2 units) ----
  float sc[2][4];
  float mt = -INFINITY;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int tok = qk_token<KB>(h, 4 * g4 + e);
      const float f = kTwo24 * sl2 / qk_posfactor<KB>(h, e);
      const float v = (FULL || tok < nvalid) ? fmaf(d[h][e], f, bias) : -INFINITY;
      sc[h][e] = v;
      mt = fmaxf(mt, v);
    }
  }
  mt = xmax4(mt);
  // ---- online softmax with a lagging reference max ----
  const float m_new = lazy_rescale(acc, mt, qk.lazy);
  float p[8];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int e = 0; e < 4; ++e) p[pv_slot<KB>(h, e)] = __builtin_amdgcn_exp2f(sc[h][e] - m_new);
  }
  // p is rounded to fp16 once; the sum l, P' and the V-min bias all use that
  // rounded value, so the rounding only perturbs the softmax weights.
  u4_t p2;
#pragma unroll
  for (int m = 0; m < 4; ++m) p2[m] = pack_h2(p[2 * m], p[2 * m + 1]);
  // 8 fp16 of channel-group row c of Vs / Vm for this lane's PV tokens
  auto vmeta8 = [&](const char* base, int c) -> u4_t {
    if constexpr (KB == 8) {
      const u2_t x0 = lds_u2(base + (c * L::vms + 4 * g4) * 2);
      const u2_t x1 = lds_u2(base + (c * L::vms + 16 + 4 * g4) * 2);
      return u4_t{x0[0], x0[1], x1[0], x1[1]};
    } else {
      return lds_u4(base + (c * L::vms + 8 * g4) * 2);
    }
  };
  // ---- V-min bias and sum_t p on the matrix cores: A row c < CG holds the
  // mins of channel group c, row CG ones (rows above are not used) ----
  acc.vbl = mfma(vmeta8(vmg, min(r, CG)), p2, acc.vbl);
  // ---- P' = p * sV per channel group ----
  u4_t pp[CG];
#pragma unroll
  for (int c = 0; c < CG; ++c) {
    const u4_t sv = vmeta8(vsg, c);
#pragma unroll
    for (int m = 0; m < 4; ++m) pp[c][m] = pkmul(p2[m], sv[m]);
  }
  // ---- O^T += codes_V^T * P' : channel block b, row r <-> channel 16 b + r ----
  const char* vw = st + L::off_vw + grp * kTile * L::vrow_pitch;
  int tok[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) tok[j] = pv_token<KB>(g4, j);
  if constexpr (L::vspread) {
    // spread rows: word w, byte b, token pair; row r of block bb is channel 16 bb + r
    const uint32_t* vsp = reinterpret_cast<const uint32_t*>(st + L::off_vw) + grp * L::vgrp_words;
    const int byte = (VB == 2) ? (r >> 2) : ((r >> 1) & 3);
    const uint32_t vmask = (VB == 2) ? (0x00030003u << (2 * (r & 3))) : (0x000F000Fu << (4 * (r & 1)));
#pragma unroll
    for (int bb = 0; bb < NB; ++bb) {
      const int w = (VB == 2) ? bb : (2 * bb + (r >> 3));
      const int sl = L::vslot(w);
      const uint32_t* src = vsp + sl * 64 + byte * 16;
      const int sw = L::vswz(sl, byte);
      u4_t x;
      if constexpr (KB == 8) {
        // PV slots (2m, 2m + 1) hold the token pair 8 (m >> 1) + 2 g4 + (m & 1)
        const u2_t x0 = *reinterpret_cast<const u2_t*>(src + ((2 * g4) ^ sw));
        const u2_t x1 = *reinterpret_cast<const u2_t*>(src + ((8 + 2 * g4) ^ sw));
        x = u4_t{x0[0], x0[1], x1[0], x1[1]};
      } else {
        x = *reinterpret_cast<const u4_t*>(src + ((4 * g4) ^ sw));
      }
      u4_t a;
#pragma unroll
      for (int m = 0; m < 4; ++m) a[m] = x[m] & vmask;
      acc.o[bb] = mfma(a, pp[bb >> 1], acc.o[bb]);
    }
  } else {
    const uint32_t vsel = sel_bytes(r & 3);
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int w = 4 * b + (r >> 2);
      u4_t a;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const uint32_t wa = lds_u32(vw + tok[2 * m] * L::vrow_pitch + w * 4);
        const uint32_t wb = lds_u32(vw + tok[2 * m + 1] * L::vrow_pitch + w * 4);
        a[m] = perm(wb, wa, vsel);
      }
      acc.o[b] = mfma(a, pp[b >> 1], acc.o[b]);
    }
  }
}

// One staged 32-token KIVI group.  L: the LDS layout (StageLayout for a workgroup
// stage, GroupLayout for a wave's own group buffer); grp is the group within it.
template <int HD, int KB, int VB, bool FULL, typename L = StageLayout<HD, KB, VB>>
__device__ __forceinline__ void kivi_group(int nvalid, const char* st, int grp, bool ktm,
                                           const u4_t (&qb)[HD / 32], WaveAcc<HD>& acc, float sl2,
                                           int lane, float lazy) {
  const QkOut qk = kivi_qk<HD, KB, L>(st, grp, ktm, qb, sl2, lane, lazy);
  kivi_softmax_pv<HD, KB, VB, FULL, L>(qk, nvalid, st, grp, acc, sl2, lane);
}

// ---------------------------------------------------------------------------
// FP16 segment: operands straight from global memory, 32 tokens per step.
// Token addresses are clamped into the segment: rows past the end only feed
// masked scores (K) or p = 0 weights (V).
// ---------------------------------------------------------------------------
template <int HD>
__device__ __forceinline__ void fp16_group(const uint16_t* kbase, const uint16_t* vbase, int64_t tok_stride,
                           int t0, int nvalid, const u4_t (&qb)[HD / 32], WaveAcc<HD>& acc,
                           float sl2, int lane) {
  constexpr int KS = HD / 32;
  constexpr int NB = HD / 16;
  constexpr int VW = NB / 2;   // 32-bit words per token and lane
  const int r = lane & 15;
  const int g4 = lane >> 4;
  u4_t kk[2][KS];
  uint32_t vv[8][VW];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int t = min(16 * h + r, nvalid - 1);
    const uint16_t* krow = kbase + (int64_t)(t0 + t) * tok_stride;
#pragma unroll
    for (int s = 0; s < KS; ++s) kk[h][s] = *reinterpret_cast<const u4_t*>(krow + 32 * s + 8 * g4);
  }
  // V^T rows: instance b, row r <-> channel NB * r + b; each lane reads its NB channels per token
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int t = min(16 * (j >> 2) + 4 * g4 + (j & 3), nvalid - 1);
    const uint16_t* vrow = vbase + (int64_t)(t0 + t) * tok_stride + NB * r;
    if constexpr (VW == 4) {
      const u4_t x = *reinterpret_cast<const u4_t*>(vrow);
#pragma unroll
      for (int k = 0; k < 4; ++k) vv[j][k] = x[k];
    } else {
      const u2_t x = *reinterpret_cast<const u2_t*>(vrow);
      vv[j][0] = x[0];
      vv[j][1] = x[1];
    }
  }
  f4_t d[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
  for (int s = 0; s < KS; ++s)
#pragma unroll
    for (int h = 0; h < 2; ++h) d[h] = mfma(kk[h][s], qb[s], d[h]);
  float sc[2][4];
  float mt = -INFINITY;
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = 16 * h + 4 * g4 + e;
      const float v = (t < nvalid) ? d[h][e] * sl2 : -INFINITY;
      sc[h][e] = v;
      mt = fmaxf(mt, v);
    }
  mt = xmax4(mt);
  const float m_new = lazy_rescale(acc, mt);
  float p[8];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int e = 0; e < 4; ++e) p[4 * h + e] = __builtin_amdgcn_exp2f(sc[h][e] - m_new);
  u4_t p2;
  float psum = 0.f;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    p2[m] = pack_h2(p[2 * m], p[2 * m + 1]);
    psum = dot2(p2[m], kOnes2, psum);
  }
  acc.l += psum;
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const uint32_t sel = sel_halves(b & 1);
    u4_t a;
#pragma unroll
    for (int m = 0; m < 4; ++m) a[m] = perm(vv[2 * m + 1][b >> 1], vv[2 * m][b >> 1], sel);
    acc.o[b] = mfma(a, p2, acc.o[b]);
  }
}

// ---------------------------------------------------------------------------
// the kernel
// ---------------------------------------------------------------------------
// one 32-token group of stage i (wave w computes group w of each stage)
template <int HD, int KB, int VB>
__device__ __forceinline__ void stage_group(const char* st, int i, int t_first, int t_stride,
                                            int t_end, bool ktm, int wave, int lane,
                                            const u4_t (&qb)[HD / 32], WaveAcc<HD>& acc,
                                            float sl2) {
  using L = StageLayout<HD, KB, VB>;
  const int t0 = t_first + i * t_stride + kTile * wave;
  if (t0 < t_end) {
    const int nvalid = min(kTile, t_end - t0);
    const float lazy = __builtin_amdgcn_readfirstlane(
                           reinterpret_cast<const uint32_t*>(st + L::off_vbig)[wave]) ? 0.f
                                                                                     : kLazyLog2;
    if (nvalid == kTile)
      kivi_group<HD, KB, VB, true>(nvalid, st, wave, ktm, qb, acc, sl2, lane, lazy);
    else
      kivi_group<HD, KB, VB, false>(nvalid, st, wave, ktm, qb, acc, sl2, lane, lazy);
  }
}

// Register sets of stage loads in flight: two for the small 2-bit stages, one
// otherwise (the register budget of two workgroups per CU)
__host__ __device__ constexpr int kivi_depth(int kb, int vb, int maxb) {
  return (kb + vb <= 4) ? 2 : 1;
}

// Every wave of the workgroup runs this with the same arguments (the stage
// barriers are workgroup-wide).  Stage i lives in LDS buffer i % 2 and is
// loaded into register set i % D; while the waves compute stage i, the loads of
// stages i + 2 .. i + 1 + D are in flight.  The steady-state loop is unrolled D
// times so every register set index is a constant.
// FAST: the unconditional loads of load_stage_fast; the compiler then waits
// only for the stage it stores.  Otherwise the general loads of load_stage.
template <int HD, int KB, int VB, int MAXB, bool FAST>
__device__ __forceinline__ void kivi_stages(const SegDev& s, const SegOffsets& o,
                                            const KivLoad& kl, int t_first, int t_stride, int nst,
                                            int t_end, int wave, int lane, int tid, char* lds,
                                            int stage_bytes, u4_t (&qb)[HD / 32],
                                            WaveAcc<HD>& acc, float& sl2) {
  using R = StageRegs<HD, KB, VB>;
  constexpr int D = kivi_depth(KB, VB, MAXB);
  const int t_last = t_end - 1;
  FastOffsets<HD, KB, VB> fo;
  if constexpr (FAST) {
#pragma unroll
    for (int i = 0; i < R::NK; ++i) {
      const int q = (tid + kThreads * i) & (R::KP - 1);
      fo.krow[i] = (uint32_t)((q / KB) * kl.row_bytes);
    }
    {
      const int q = tid & (HD - 1);
      fo.mgrp = (uint32_t)(q / (HD / 4));
      fo.mcol = (uint32_t)(4 * (q & (HD / 4 - 1)));
      fo.mrow = (uint32_t)(q * kl.row_groups);
    }
  }
  auto load = [&](R& r, int st) {
    if constexpr (FAST) load_stage_fast<HD, KB, VB>(r, s, o, kl, fo, t_first + st * t_stride, t_last, tid);
    else load_stage<HD, KB, VB>(r, s, o, kl, t_first + st * t_stride, t_last, tid);
  };
  char* buf0 = lds;
  char* buf1 = lds + stage_bytes;
  {
    // the ones row of both buffers' V-min block (never overwritten by the stages)
    using L = StageLayout<HD, KB, VB>;
    constexpr int CG = HD / 32;
    for (int t = tid; t < kStage; t += kThreads) {
      reinterpret_cast<uint16_t*>(buf0 + L::off_vm)[CG * L::vms + t] = 0x3C00;
      reinterpret_cast<uint16_t*>(buf1 + L::off_vm)[CG * L::vms + t] = 0x3C00;
    }
  }
  auto buf = [&](int st) { return (st & 1) ? buf1 : buf0; };
  R r[D];
  // stage 0 goes out alone: every workgroup starts at once, and its first
  // stage should not queue behind everybody's next ones
  load(r[0], 0);
  normalize_q<HD>(qb, sl2);
  store_stage<HD, KB, VB>(r[0], kl.kmeta_gm, kl.kdata_tm, tid, buf0);
#pragma unroll
  for (int k = 1; k <= D; ++k)
    if (k < nst) load(r[k % D], k);
  __syncthreads();
  int i = 0;
  // steady state: stage i + j computed, i + j + 1 stored, i + j + 1 + D loaded
  for (; i + 2 * D < nst; i += D) {
#pragma unroll
    for (int j = 0; j < D; ++j) {
      stage_group<HD, KB, VB>(buf(i + j), i + j, t_first, t_stride, t_end, kl.kdata_tm, wave, lane, qb,
                              acc, sl2);
      store_stage<HD, KB, VB>(r[(j + 1) % D], kl.kmeta_gm, kl.kdata_tm, tid, buf(i + j + 1));
      load(r[(j + 1) % D], i + j + 1 + D);
      __syncthreads();
    }
  }
  // tail: at most 2 D stages left, none loaded beyond nst; one copy of the
  // group code, the register set picked by constant index
  for (; i < nst; ++i) {
    stage_group<HD, KB, VB>(buf(i), i, t_first, t_stride, t_end, kl.kdata_tm, wave, lane, qb, acc,
                            sl2);
    if (i + 1 < nst) {
      const int set = (i + 1) % D;
#pragma unroll
      for (int k = 0; k < D; ++k) {
        if (set == k) {
          store_stage<HD, KB, VB>(r[k], kl.kmeta_gm, kl.kdata_tm, tid, buf(i + 1));
          if (i + 1 + D < nst) load(r[k], i + 1 + D);
        }
      }
      __syncthreads();
    }
  }
}

// ---------------------------------------------------------------------------
// Wave-private groups.  For token-major K codes with group-major K metadata
// (the storage quantize_pack writes) every piece of a 32-token group is one
// contiguous block, so each wave streams its own groups (wave, wave + 4, ...)
// through two LDS buffers of its own and the waves of a workgroup meet only at
// the final merge: no workgroup barrier per stage, no waiting for the slowest
// wave.  Widths up to 4 bits (two buffers per wave fit the LDS of two
// workgroups per CU).
// ---------------------------------------------------------------------------
template <int HD, int KB, int VB>
struct GroupLayout {
  static_assert(VB != 8, "8-bit V groups use the workgroup stages");
  static constexpr int kw_row = HD;                       // channel-major K rows: not used
  static constexpr int kt_pitch = HD + 8;                 // as StageLayout
  static constexpr int off_ks = 4 * KB * kt_pitch;
  static constexpr int off_km = off_ks + HD * 2;
  static constexpr int off_vw = off_km + HD * 2;
  static constexpr int vrow_words = HD * VB / 32;
  static constexpr int vrow_bytes = HD * VB / 8;
  static constexpr bool vspread = true;
  static constexpr int vpw = (vrow_words >= 16) ? 4 : 2;
  static constexpr int vnq = vrow_words / vpw;
  static constexpr int vgrp_words = vrow_words * 64;
  static constexpr int vrow_pitch = vrow_bytes + 16;
  // V scale / min rows of one group's 32 tokens: 40 halves apart, so the rows
  // of the bias operand read start 20 banks apart
  static constexpr int vms = kTile + 8;
  static constexpr int off_vs = off_vw + vgrp_words * 4;
  static constexpr int off_vm = off_vs + (HD / 32) * vms * 2;
  static constexpr int bytes = (off_vm + (HD / 32 + 1) * vms * 2 + 15) & ~15;
  __device__ static constexpr int vslot(int w) { return (w % vpw) * vnq + w / vpw; }
  __device__ static constexpr int vswz(int s, int b) { return 8 * ((s ^ (b >> 1)) & 1); }
};

// ---------------------------------------------------------------------------
// The V side of a wave-private 32-token group (V per token, 32-channel groups),
// shared by the KIVI and the per-token K groups.  VB = 2, 4: the spread layout of
// StageLayout (items (token pair, PW-word slice), slice fastest); every lane
// loads unconditionally, rows clamped to t_last.
// ---------------------------------------------------------------------------
template <int HD, int VB>
struct VGroupShape {
  static constexpr int W = HD * VB / 32;        // words per V row
  static constexpr int PW = (W >= 16) ? 4 : 2;
  static constexpr int NQ = W / PW;
  static constexpr int VI = 16 * NQ;            // V items (token pair, slice) of a group
};

// t0: wave-uniform first token of the group
template <int HD, int VB>
__device__ __forceinline__ void load_group_vcodes(u4_t& va, u4_t& vb, const SegDev& s,
                                                  const SegOffsets& o, int t0, int t_last,
                                                  int lane) {
  using V = VGroupShape<HD, VB>;
  constexpr int RB = HD * VB / 8;
  const int q = lane % V::VI;
  const uint32_t tp = q / V::NQ, qw = q - tp * V::NQ;
  const uint32_t dt = (uint32_t)(t_last - t0);
  const uint8_t* vrow = s.vd + o.vd + (int64_t)t0 * RB;
  const uint8_t* pa = vrow + (min(2u * tp, dt) * RB + qw * V::PW * 4);
  const uint8_t* pb = vrow + (min(2u * tp + 1u, dt) * RB + qw * V::PW * 4);
  if constexpr (V::PW == 4) {
    va = *reinterpret_cast<const u4_t*>(pa);
    vb = *reinterpret_cast<const u4_t*>(pb);
  } else {
    const u2_t a = *reinterpret_cast<const u2_t*>(pa);
    const u2_t b = *reinterpret_cast<const u2_t*>(pb);
    va = u4_t{a[0], a[1], 0u, 0u};
    vb = u4_t{b[0], b[1], 0u, 0u};
  }
}

// V scales (lanes < 32) or mins (lanes >= 32) of token lane % 32 (HD = 64: low word only)
template <int HD>
__device__ __forceinline__ void load_group_vmeta(u2_t& vm, const SegDev& s, const SegOffsets& o,
                                                 int t0, int t_last, int lane) {
  const uint32_t dt = min((uint32_t)(lane & (kTile - 1)), (uint32_t)(t_last - t0));
  const uint16_t* m = pick(lane < kTile, s.vs, s.vm) + (o.vm + (int64_t)t0 * (HD / 32)) + dt * (HD / 32);
  if (HD == 128) vm = *reinterpret_cast<const u2_t*>(m);
  else vm = u2_t{*reinterpret_cast<const uint32_t*>(m), 0u};
}

template <int HD, int VB, typename L>
__device__ __forceinline__ void store_group_vcodes(const u4_t& va, const u4_t& vb, int lane, char* st) {
  using V = VGroupShape<HD, VB>;
  if (V::VI == 64 || lane < V::VI) {
    // the store order of StageLayout: 32 stores of a half wave in 32 banks
    const int tp = lane / V::NQ, qw = lane - tp * V::NQ;
    const int flip = ((V::NQ == 4) ? (qw >> 1) : qw) & 1;
    uint32_t* dst = reinterpret_cast<uint32_t*>(st + L::off_vw) + qw * 64;
#pragma unroll
    for (int k = 0; k < V::PW; ++k)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int b = j ^ flip;
        const int sw = 8 * ((qw ^ (j >> 1)) & 1);
        dst[k * V::NQ * 64 + b * 16 + (tp ^ sw)] = perm(vb[k], va[k], sel_bytes(b));
      }
  }
}

// Returns whether a V scale of the group is above kVScaleSafe.
template <int HD, typename L>
__device__ __forceinline__ bool store_group_vmeta(const u2_t& vm, int lane, char* st) {
  uint16_t* m = reinterpret_cast<uint16_t*>(st + ((lane < kTile) ? L::off_vs : L::off_vm));
  const int t = lane & (kTile - 1);
#pragma unroll
  for (int cg = 0; cg < HD / 32; ++cg)
    m[cg * L::vms + t] = (uint16_t)(vm[cg >> 1] >> (16 * (cg & 1)));
  // lanes < 32 hold one token's V scales
  return __ballot(vscale_big(lane < kTile, vm)) != 0;
}

// One lane's share of a group's loads (64 lanes).
template <int HD, int KB, int VB>
struct GroupRegs {
  static constexpr int KP = 4 * KB * HD / 16;   // 16-byte K pieces (4 KB byte rows of HD)
  static constexpr int NK = (KP + 63) / 64;
  u4_t k[NK];
  u4_t va, vb;
  u2_t km;     // lanes < HD / 2: 4 channels of the group's K scales (lane < HD / 4) or mins
  u2_t vm;     // V scales (lanes < 32) or mins of token lane % 32 (HD = 64: low word only)
};

// Loads of the group at token t0 (a multiple of 32 from the segment start); every
// lane loads unconditionally, addresses clamped into the segment.
template <int HD, int KB, int VB>
__device__ __forceinline__ void load_group(GroupRegs<HD, KB, VB>& r, const SegDev& s,
                                           const SegOffsets& o, const KivLoad& kl, int t0_,
                                           int t_last, int lane) {
  using R = GroupRegs<HD, KB, VB>;
  // t0 is the same on every lane of the wave: each load below is a scalar base
  // plus a 32-bit lane offset (no 64-bit address arithmetic per lane)
  const int t0 = __builtin_amdgcn_readfirstlane(t0_);
  const uint32_t row0 = (uint32_t)t0 * KB / 8;
  const uint32_t last = (uint32_t)((kl.k_rows - row0) * (HD / 16)) - 1u;
  const uint8_t* kbase = s.kd + o.kd + (int64_t)row0 * HD;
#pragma unroll
  for (int i = 0; i < R::NK; ++i) {
    const uint32_t q = min((uint32_t)(lane + 64 * i), (uint32_t)R::KP - 1u);
    r.k[i] = *reinterpret_cast<const u4_t*>(kbase + 16u * min(q, last));
  }
  {
    constexpr int QL = HD / 4;    // lanes per tensor, 4 channels each
    const int q = lane & (2 * QL - 1);
    const int64_t mrow = o.km + (int64_t)(t0 / kTile) * HD;
    const uint16_t* m = pick(q < QL, s.ks, s.km) + mrow + 4 * (q & (QL - 1));
    r.km = *reinterpret_cast<const u2_t*>(m);
  }
  load_group_vcodes<HD, VB>(r.va, r.vb, s, o, t0, t_last, lane);
  load_group_vmeta<HD>(r.vm, s, o, t0, t_last, lane);
}

// The group's registers into the wave's buffer (GroupLayout).
// Returns whether a V scale of the group is above kVScaleSafe.
template <int HD, int KB, int VB>
__device__ __forceinline__ bool store_group(const GroupRegs<HD, KB, VB>& r, int lane, char* st) {
  using L = GroupLayout<HD, KB, VB>;
  using R = GroupRegs<HD, KB, VB>;
#pragma unroll
  for (int i = 0; i < R::NK; ++i) {
    const int q = lane + 64 * i;
    if (R::KP % 64 == 0 || q < R::KP) {
      u2_t* dst = reinterpret_cast<u2_t*>(st + (q / (HD / 16)) * L::kt_pitch + (q % (HD / 16)) * 16);
      dst[0] = u2_t{r.k[i][0], r.k[i][1]};
      dst[1] = u2_t{r.k[i][2], r.k[i][3]};
    }
  }
  {
    constexpr int QL = HD / 4;
    if (lane < 2 * QL) {
      uint16_t* m = reinterpret_cast<uint16_t*>(st + ((lane < QL) ? L::off_ks : L::off_km));
      *reinterpret_cast<u2_t*>(m + 4 * (lane & (QL - 1))) = r.km;
    }
  }
  store_group_vcodes<HD, VB, L>(r.va, r.vb, lane, st);
  return store_group_vmeta<HD, L>(r.vm, lane, st);
}

// Waves with at least this many groups of a two-register-set (2-bit K and V)
// segment run the pipelined group loop.
constexpr int kPipeMinGroups = 8;

// The wave's groups of the chunk [t_first, t_end): group i at t_first + 32 (wave + 4 i),
// in buffer i % 2 of the wave, loaded into register set i % D.
//
// Long runs of 2-bit groups are pipelined by one group: iteration i runs the QK
// phase of group i + 1 (buffer (i + 1) % 2), then the softmax / PV phase of group
// i (buffer i % 2), so the QK matrix products of one group overlap the softmax and
// PV chain of the other; then group i + 2 goes into buffer i % 2.  The loads of
// groups 0 .. D go out together.  Short runs take one group at a time and load
// group 0 alone first: when every wave of the launch has only a few groups, the
// first group's latency decides the finish, and the wider first burst of loads
// delays it (measured on MI355X).
// The wave takes groups wslot, wslot + wstride, ... of [t_first, t_end): (wave, 4)
// when the four waves share a chunk, (0, 1) when the wave owns a whole segment of a
// device table.  Its two buffers start at lds + wave * wbytes (the waves of a table
// item can hold different widths, so there wbytes covers the widest layout).  norm:
// normalize q (first segment of the workgroup).
template <int HD, int KB, int VB>
__device__ __forceinline__ void kivi_wave_groups(const SegDev& s, const SegOffsets& o,
                                                 const KivLoad& kl, int t_first, int t_end,
                                                 int wave, int wslot, int wstride, int lane,
                                                 char* lds, int wbytes, u4_t (&qb)[HD / 32],
                                                 WaveAcc<HD>& acc, float& sl2, bool norm) {
  using L = GroupLayout<HD, KB, VB>;
  using R = GroupRegs<HD, KB, VB>;
  constexpr int D = (KB + VB <= 4) ? 2 : 1;
  constexpr int CG = HD / 32;
  const int ng = (t_end - t_first + kTile - 1) / kTile;
  const int n = (ng - wslot + wstride - 1) / wstride;
  if (n <= 0) return;
  const int t_last = t_end - 1;
  char* b0 = lds + wave * wbytes;
  char* b1 = b0 + L::bytes;
  // the ones row of both buffers' V-min block (never overwritten by the groups)
  if (lane < kTile) {
    reinterpret_cast<uint16_t*>(b0 + L::off_vm)[CG * L::vms + lane] = 0x3C00;
    reinterpret_cast<uint16_t*>(b1 + L::off_vm)[CG * L::vms + lane] = 0x3C00;
  }
  auto tok = [&](int i) { return t_first + kTile * (wslot + wstride * i); };
  auto buf = [&](int i) { return (i & 1) ? b1 : b0; };
  auto load = [&](R& r, int i) { load_group<HD, KB, VB>(r, s, o, kl, tok(i), t_last, lane); };
  // whether the group in buffer 0 / 1 has a large V scale (set when it is stored)
  bool big0 = false, big1 = false;
  auto lazy = [&](int i) { return ((i & 1) ? big1 : big0) ? 0.f : kLazyLog2; };
  auto store = [&](const R& r, int i) {
    const bool f = store_group<HD, KB, VB>(r, lane, buf(i));
    if (i & 1) big1 = f;
    else big0 = f;
  };
  if constexpr (D == 2) {
    if (n >= kPipeMinGroups) {
      auto qk = [&](int i) {
        return kivi_qk<HD, KB, L>(buf(i), 0, true, qb, sl2, lane, lazy(i));
      };
      // set g % D holds group g >= 1 from its load until its store
      R r0, r[D];
      load(r0, 0);
#pragma unroll
      for (int k = 1; k <= D; ++k) load(r[k % D], k);
      if (norm) normalize_q<HD>(qb, sl2);
      store(r0, 0);
      wave_lds_sync();
      QkOut cur = qk(0);
      store(r[1], 1);
      load(r[1], 1 + D);
      wave_lds_sync();
      // groups i and i + 1 are in their buffers and cur holds QK(i); groups
      // i .. i + D + 1 of the steady loop are full
      int i = 0;
      for (; i + 2 * D + 1 < n; i += D) {
#pragma unroll
        for (int j = 0; j < D; ++j) {
          const QkOut nxt = qk(i + j + 1);
          kivi_softmax_pv<HD, KB, VB, true, L>(cur, kTile, buf(i + j), 0, acc, sl2, lane);
          store(r[(j + 2) % D], i + j + 2);
          load(r[(j + 2) % D], i + j + 2 + D);
          wave_lds_sync();
          cur = nxt;
        }
      }
      for (; i < n; ++i) {
        QkOut nxt = cur;
        if (i + 1 < n) nxt = qk(i + 1);
        const int nvalid = min(kTile, t_end - tok(i));
        if (nvalid == kTile) kivi_softmax_pv<HD, KB, VB, true, L>(cur, nvalid, buf(i), 0, acc, sl2, lane);
        else kivi_softmax_pv<HD, KB, VB, false, L>(cur, nvalid, buf(i), 0, acc, sl2, lane);
        if (i + 2 < n) {
          const int set = (i + 2) % D;
#pragma unroll
          for (int k = 0; k < D; ++k) {
            if (set == k) {
              store(r[k], i + 2);
              if (i + 2 + D < n) load(r[k], i + 2 + D);
            }
          }
          wave_lds_sync();
        }
        cur = nxt;
      }
      return;
    }
  }
  auto group = [&](int i) {
    const int nvalid = min(kTile, t_end - tok(i));
    if (nvalid == kTile)
      kivi_group<HD, KB, VB, true, L>(nvalid, buf(i), 0, true, qb, acc, sl2, lane, lazy(i));
    else
      kivi_group<HD, KB, VB, false, L>(nvalid, buf(i), 0, true, qb, acc, sl2, lane, lazy(i));
  };
  R r[D];
  // group 0 goes out alone, then groups 1 .. D
  load(r[0], 0);
  if (norm) normalize_q<HD>(qb, sl2);
  store(r[0], 0);
#pragma unroll
  for (int k = 1; k <= D; ++k)
    if (k < n) load(r[k % D], k);
  wave_lds_sync();
  int i = 0;
  for (; i + 2 * D < n; i += D) {
#pragma unroll
    for (int j = 0; j < D; ++j) {
      group(i + j);
      store(r[(j + 1) % D], i + j + 1);
      load(r[(j + 1) % D], i + j + 1 + D);
      wave_lds_sync();
    }
  }
  for (; i < n; ++i) {
    group(i);
    if (i + 1 < n) {
      const int set = (i + 1) % D;
#pragma unroll
      for (int k = 0; k < D; ++k) {
        if (set == k) {
          store(r[k], i + 1);
          if (i + 1 + D < n) load(r[k], i + 1 + D);
        }
      }
      wave_lds_sync();
    }
  }
}

// Stages of the chunk: t_first + i t_stride (i < nst), tokens below t_end.  NW: waves of
// the workgroup.  WO: a wave-path-only variant (every 8-wave variant, and the 4-wave ones
// for launches that need no more), which takes only what the wave-private groups read (the
// host checks it) and is a fraction of the code; the 128-token workgroup stages need 4 waves.
template <int HD, int KB, int VB, int MAXB, int NW, bool WO>
__device__ __forceinline__ void kivi_chunk(const SegDev& s, const SegOffsets& o, int t_first,
                                           int t_stride, int nst, int t_end, int wave, int lane,
                                           int tid, char* lds, int stage_bytes,
                                           u4_t (&qb)[HD / 32], WaveAcc<HD>& acc,
                                           float& sl2) {
  KivLoad kl;
  kl.row_bytes = ((int64_t)s.length * KB + 7) / 8;
  kl.row_groups = (s.length + s.kgs - 1) / s.kgs;
  kl.k_rows = kl.row_bytes;
  const int64_t byte_begin = (int64_t)t_first * KB / 8;
  const uintptr_t kaddr = reinterpret_cast<uintptr_t>(s.kd + o.kd);
  // token-major rows are HD bytes (the host sends only 16-byte aligned ones here)
  kl.kdata_tm = s.kdata_tm;
  if (kl.kdata_tm) kl.kmode = 16;
  else if (kl.row_bytes % 16 == 0 && byte_begin % 16 == 0 && kaddr % 16 == 0) kl.kmode = 16;
  else if (kl.row_bytes % 4 == 0 && byte_begin % 4 == 0 && kaddr % 4 == 0) kl.kmode = 4;
  else kl.kmode = 1;
  const bool meta8 = (reinterpret_cast<uintptr_t>(s.ks + o.km) % 8 == 0) &&
                     (reinterpret_cast<uintptr_t>(s.km + o.km) % 8 == 0);
  kl.kmeta_gm = s.kmeta_gm && meta8;
  kl.gm_elems = s.kmeta_gm && !meta8;
  kl.kmeta4 = !s.kmeta_gm && (kl.row_groups % 4 == 0) && (t_first % kStage == 0) &&
              (t_stride % kStage == 0) && meta8;
  if constexpr (KB <= 4 && VB <= 4) {
    if (WO || (kl.kdata_tm && kl.kmeta_gm && kl.row_bytes < ((int64_t)1 << 31) / HD)) {
      kivi_wave_groups<HD, KB, VB>(s, o, kl, t_first, t_end, wave, wave, NW, lane, lds,
                                   2 * GroupLayout<HD, KB, VB>::bytes, qb, acc, sl2, true);
      return;
    }
  }
  if constexpr (!WO) {
    static_assert(NW == kWaves, "the workgroup stages take four waves");
    if (kl.kmode == 16 && (kl.kmeta4 || kl.kmeta_gm) && kl.row_bytes < ((int64_t)1 << 31) / HD)
      kivi_stages<HD, KB, VB, MAXB, true>(s, o, kl, t_first, t_stride, nst, t_end, wave, lane, tid, lds,
                                    stage_bytes, qb, acc, sl2);
    else
      kivi_stages<HD, KB, VB, MAXB, false>(s, o, kl, t_first, t_stride, nst, t_end, wave, lane, tid, lds,
                                     stage_bytes, qb, acc, sl2);
  }
}

// ---------------------------------------------------------------------------
// Per-token K groups (PK_SEG_TOKEN: the reference's legacy layout,
// src/phasekv/kernels/attention_triton.py:145-282).  K is packed along head_dim
// like V, with one scale / min per (token, 32-channel group g):
//   S^T[t][h] = sum_g sK[t][g] * D_g[t][h] + sum_g mK[t][g] * Q_g[h],
//   D_g[t][h] = sum_{c in g} code_K[t][c] * q[h][c],   Q_g[h] = sum_{c in g} q[h][c].
// One MFMA per (16 tokens, group) gives D_g in fp32 and the per-token scale and
// min act on the fp32 results: no fp16 fold, the scores keep fp32 precision.
// A K code byte holds channels, so the codes of one operand sit at different bit
// positions (the fp16 subnormal code * 2^(pos - 24)); each channel's factor
// 2^-pos is folded into the q operand once per segment (exact powers of two, q
// normalized so that its largest element is in (1/2, 1]).
//
// LDS of one group (the wave's buffer):
//   Kc  [32 tokens][lane group g4][group g][KB bytes]: the KB-byte unit of channels
//       32 g + 8 g4 .. + 7, so one read gives a lane its token's operands of every
//       group (the store transposes the row as loaded)
//   Km  [32 tokens][sK of the HD/32 groups | mK of the HD/32 groups] fp16
//   V, Vs, Vm as GroupLayout; VB = 8: the rows as stored, StageLayout's pitch
// Results come in the token order of 8-bit KIVI K (row r of instance h = token
// 16 h + r), which kivi_softmax_pv<.., KB = 8, ..> follows.
// ---------------------------------------------------------------------------
template <int HD, int KB, int VB>
struct TokLayout {
  static constexpr int NS = HD / 32;                      // channel groups
  static constexpr int krow = HD * KB / 8;                // code bytes per token
  static constexpr int kunits = NS * KB;                  // code bytes a lane reads per token
  // padded so that the 16 token rows of one operand read spread over the banks
  static constexpr int kpitch = krow + ((kunits >= 16) ? 16 : 8);
  static constexpr int kmeta_row = 4 * NS;
  static constexpr int off_kmeta = kTile * kpitch;
  static constexpr int off_vw = off_kmeta + kTile * kmeta_row;
  static constexpr int vrow_words = HD * VB / 32;
  static constexpr int vrow_bytes = HD * VB / 8;
  static constexpr bool vspread = VB != 8;
  static constexpr int vpw = (vrow_words >= 16) ? 4 : 2;
  static constexpr int vnq = vrow_words / vpw;
  static constexpr int vgrp_words = vrow_words * 64;
  static constexpr int vrow_pitch = vrow_bytes + 16;
  static constexpr int vw_bytes = vspread ? vgrp_words * 4 : kTile * vrow_pitch;
  static constexpr int vms = kTile + 8;
  static constexpr int off_vs = off_vw + vw_bytes;
  static constexpr int off_vm = off_vs + NS * vms * 2;
  static constexpr int bytes = (off_vm + (NS + 1) * vms * 2 + 15) & ~15;
  __device__ static constexpr int vslot(int w) { return (w % vpw) * vnq + w / vpw; }
  __device__ static constexpr int vswz(int s, int b) { return 8 * ((s ^ (b >> 1)) & 1); }
};

// One lane's share of a per-token group's loads (64 lanes).
template <int HD, int KB, int VB>
struct TokRegs {
  static constexpr int KP = kTile * HD * KB / 128;        // 16-byte K pieces
  static constexpr int NK = (KP + 63) / 64;
  static constexpr int VP = kTile * HD / 16;              // 16-byte V pieces at 8 bits
  static constexpr int NV = (VB == 8) ? (VP + 63) / 64 : 1;
  u4_t k[NK];
  u2_t km;         // sK (lanes < 32) or mK (lanes >= 32) of token lane % 32 (HD = 64: low word)
  u4_t va, vb;     // VB = 2, 4
  u4_t v[NV];      // VB = 8
  u2_t vm;
};

template <int HD, int KB, int VB>
__device__ __forceinline__ void load_tok_group(TokRegs<HD, KB, VB>& r, const SegDev& s,
                                               const SegOffsets& o, int t0_, int t_last, int lane) {
  using R = TokRegs<HD, KB, VB>;
  constexpr int NS = HD / 32;
  constexpr int KR = HD * KB / 8;       // code bytes per token
  constexpr int PR = KR / 16;           // 16-byte pieces per token
  const int t0 = __builtin_amdgcn_readfirstlane(t0_);
  const uint32_t dt = (uint32_t)(t_last - t0);
  const uint8_t* kbase = s.kd + o.kd + (int64_t)t0 * KR;
#pragma unroll
  for (int i = 0; i < R::NK; ++i) {
    const uint32_t q = min((uint32_t)(lane + 64 * i), (uint32_t)R::KP - 1u);
    r.k[i] = *reinterpret_cast<const u4_t*>(kbase + min(q / PR, dt) * KR + 16u * (q % PR));
  }
  {
    const uint32_t tq = min((uint32_t)(lane & (kTile - 1)), dt);
    const uint16_t* m = pick(lane < kTile, s.ks, s.km) + (o.km + (int64_t)t0 * NS) + tq * NS;
    if (HD == 128) r.km = *reinterpret_cast<const u2_t*>(m);
    else r.km = u2_t{*reinterpret_cast<const uint32_t*>(m), 0u};
  }
  if constexpr (VB == 8) {
    constexpr int PV = HD / 16;
    const uint8_t* vbase = s.vd + o.vd + (int64_t)t0 * HD;
#pragma unroll
    for (int i = 0; i < R::NV; ++i) {
      const uint32_t q = min((uint32_t)(lane + 64 * i), (uint32_t)R::VP - 1u);
      r.v[i] = *reinterpret_cast<const u4_t*>(vbase + min(q / PV, dt) * HD + 16u * (q % PV));
    }
  } else {
    load_group_vcodes<HD, VB>(r.va, r.vb, s, o, t0, t_last, lane);
  }
  load_group_vmeta<HD>(r.vm, s, o, t0, t_last, lane);
}

// The group's registers into the wave's buffer (TokLayout).  Returns whether a V
// scale of the group is above kVScaleSafe.
template <int HD, int KB, int VB>
__device__ __forceinline__ bool store_tok_group(const TokRegs<HD, KB, VB>& r, int lane, char* st) {
  using L = TokLayout<HD, KB, VB>;
  using R = TokRegs<HD, KB, VB>;
  constexpr int NS = HD / 32;
  constexpr int PR = L::krow / 16;
#pragma unroll
  for (int i = 0; i < R::NK; ++i) {
    const int q = lane + 64 * i;
    if (R::KP % 64 == 0 || q < R::KP) {
      const int p = q % PR;
      char* row = st + (q / PR) * L::kpitch;
      const u4_t w = r.k[i];
      if constexpr (KB == 2) {
        // the piece holds groups 2 p and 2 p + 1; unit (g, g4) = bytes 2 g4, 2 g4 + 1 of
        // the group's 8 bytes.  Units (2 p, g4) and (2 p + 1, g4) are neighbours.
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4)
          *reinterpret_cast<uint32_t*>(row + 2 * (g4 * NS + 2 * p)) =
              perm(w[2 + (g4 >> 1)], w[g4 >> 1], sel_halves(g4 & 1));
      } else if constexpr (KB == 4) {
        // the piece is group p; unit (p, g4) = word g4
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) *reinterpret_cast<uint32_t*>(row + 4 * (g4 * NS + p)) = w[g4];
      } else {
        // the piece is half p % 2 of group p / 2: units g4 = 2 (p % 2) and 2 (p % 2) + 1
#pragma unroll
        for (int u = 0; u < 2; ++u)
          *reinterpret_cast<u2_t*>(row + 8 * ((2 * (p & 1) + u) * NS + (p >> 1))) =
              u2_t{w[2 * u], w[2 * u + 1]};
      }
    }
  }
  {
    char* m = st + L::off_kmeta + (lane & (kTile - 1)) * L::kmeta_row + ((lane < kTile) ? 0 : 2 * NS);
    if (HD == 128) *reinterpret_cast<u2_t*>(m) = r.km;
    else *reinterpret_cast<uint32_t*>(m) = r.km[0];
  }
  if constexpr (VB == 8) {
    constexpr int PV = HD / 16;
#pragma unroll
    for (int i = 0; i < R::NV; ++i) {
      const int q = lane + 64 * i;
      if (R::VP % 64 == 0 || q < R::VP)
        *reinterpret_cast<u4_t*>(st + L::off_vw + (q / PV) * L::vrow_pitch + (q % PV) * 16) = r.v[i];
    }
  } else {
    store_group_vcodes<HD, VB, L>(r.va, r.vb, lane, st);
  }
  return store_group_vmeta<HD, L>(r.vm, lane, st);
}

// fp16 pair (2^-pos of slot 2 m, 2^-pos of slot 2 m + 1): the bit positions of the
// codes in operand register m (tok_qk)
template <int KB>
__device__ __forceinline__ uint32_t tok_posfactors(int m) {
  if (KB == 2) return (m & 1) ? 0x24002C00u : 0x34003C00u;   // (1/16, 1/64) : (1, 1/4)
  if (KB == 4) return 0x2C003C00u;                           // (1, 1/16)
  return kOnes2;
}

// The q operand of the per-token K products (q' times the position factors) and the
// group sums Q_g of q' (times 2^-24, the scale of the code products), for this
// lane's head.
template <int HD, int KB>
__device__ __forceinline__ void tok_q_operands(const u4_t (&qb)[HD / 32], u4_t (&qt)[HD / 32],
                                               float (&qs)[HD / 32]) {
#pragma unroll
  for (int g = 0; g < HD / 32; ++g) {
    float sum = 0.f;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      qt[g][m] = pkmul(qb[g][m], tok_posfactors<KB>(m));
      sum = dot2(qb[g][m], kOnes2, sum);
    }
    qs[g] = xsum4(sum) * (1.0f / kTwo24);
  }
}

__device__ __forceinline__ float half_lo(uint32_t w) {
  return (float)__builtin_bit_cast(h2_t, w)[0];
}
__device__ __forceinline__ float half_hi(uint32_t w) {
  return (float)__builtin_bit_cast(h2_t, w)[1];
}

// QK phase of a per-token group: the scores of instances h = 0, 1 times 2^-24 / sl2
// (the factor kivi_softmax_pv applies for 8-bit K), bias 0.
template <int HD, int KB, typename L>
__device__ __forceinline__ QkOut tok_qk(const char* st, const u4_t (&qt)[HD / 32],
                                        const float (&qs)[HD / 32], int lane, float lazy) {
  constexpr int NS = HD / 32;
  constexpr int NW = L::kunits / 4;     // words a lane reads per token
  const int r = lane & 15;
  const int g4 = lane >> 4;
  f4_t out[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const char* kp = st + (16 * h + r) * L::kpitch + g4 * L::kunits;
    uint32_t w[NW];
    if constexpr (NW == 1) {
      w[0] = lds_u32(kp);
    } else if constexpr (NW == 2) {
      const u2_t x = lds_u2(kp);
      w[0] = x[0];
      w[1] = x[1];
    } else {
#pragma unroll
      for (int k = 0; k < NW / 4; ++k) {
        const u4_t x = lds_u4(kp + 16 * k);
#pragma unroll
        for (int j = 0; j < 4; ++j) w[4 * k + j] = x[j];
      }
    }
    f4_t dg[NS];
#pragma unroll
    for (int g = 0; g < NS; ++g) {
      u4_t a;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        if constexpr (KB == 2) {
          // operand m: byte m / 2 of the unit; slots 2 m, 2 m + 1 at bit positions
          // 0, 2 (m even) or 4, 6 (m odd)
          const uint32_t x = w[g >> 1];
          a[m] = perm(x, x, sel_bytes(2 * (g & 1) + (m >> 1))) & ((m & 1) ? 0x00C00030u : 0x000C0003u);
        } else if constexpr (KB == 4) {
          // operand m: byte m, low nibble (slot 2 m) and high nibble (slot 2 m + 1)
          a[m] = perm(w[g], w[g], sel_bytes(m)) & 0x00F0000Fu;
        } else {
          // operand m: bytes 2 m, 2 m + 1 of the unit
          const uint32_t x = w[2 * g + (m >> 1)];
          const uint32_t b0 = 2u * (m & 1);
          a[m] = perm(x, x, b0 | (0x0cu << 8) | ((b0 + 1u) << 16) | (0x0cu << 24));
        }
      }
      dg[g] = mfma(a, qt[g], f4_t{0.f, 0.f, 0.f, 0.f});
    }
    // per-token scale and min of the lane's result rows (tokens 16 h + 4 g4 + e)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const char* mr = st + L::off_kmeta + (16 * h + 4 * g4 + e) * L::kmeta_row;
      uint32_t sk[2], mk[2];
      if constexpr (NS == 4) {
        const u4_t x = lds_u4(mr);
        sk[0] = x[0]; sk[1] = x[1]; mk[0] = x[2]; mk[1] = x[3];
      } else {
        const u2_t x = lds_u2(mr);
        sk[0] = x[0]; sk[1] = 0u; mk[0] = x[1]; mk[1] = 0u;
      }
      float t = 0.f;
#pragma unroll
      for (int g = 0; g < NS; ++g) {
        const uint32_t sw = sk[g >> 1], mw = mk[g >> 1];
        const float sg = (g & 1) ? half_hi(sw) : half_lo(sw);
        const float mg = (g & 1) ? half_hi(mw) : half_lo(mw);
        t = fmaf(sg, dg[g][e], fmaf(mg, qs[g], t));
      }
      out[h][e] = t;
    }
  }
  return QkOut{{out[0], out[1]}, 0.f, lazy};
}

// The wave's per-token groups of the chunk [t_first, t_end): groups wave, wave + 4,
// ... through the wave's two buffers, the next D groups' loads in flight.
template <int HD, int KB, int VB, int NW>
__device__ __forceinline__ void tok_wave_groups(const SegDev& s, const SegOffsets& o, int t_first,
                                                int t_end, int wave, int lane, char* lds,
                                                u4_t (&qb)[HD / 32], WaveAcc<HD>& acc,
                                                float& sl2) {
  using L = TokLayout<HD, KB, VB>;
  using R = TokRegs<HD, KB, VB>;
  constexpr int D = (KB + VB <= 8) ? 2 : 1;
  constexpr int NS = HD / 32;
  const int ng = (t_end - t_first + kTile - 1) / kTile;
  const int n = (ng - wave + NW - 1) / NW;
  if (n <= 0) return;
  const int t_last = t_end - 1;
  char* b0 = lds + wave * 2 * L::bytes;
  char* b1 = b0 + L::bytes;
  // the ones row of both buffers' V-min block (never overwritten by the groups)
  if (lane < kTile) {
    reinterpret_cast<uint16_t*>(b0 + L::off_vm)[NS * L::vms + lane] = 0x3C00;
    reinterpret_cast<uint16_t*>(b1 + L::off_vm)[NS * L::vms + lane] = 0x3C00;
  }
  auto tok = [&](int i) { return t_first + kTile * (wave + NW * i); };
  auto buf = [&](int i) { return (i & 1) ? b1 : b0; };
  auto load = [&](R& r, int i) { load_tok_group<HD, KB, VB>(r, s, o, tok(i), t_last, lane); };
  bool big0 = false, big1 = false;
  auto store = [&](const R& r, int i) {
    const bool f = store_tok_group<HD, KB, VB>(r, lane, buf(i));
    if (i & 1) big1 = f;
    else big0 = f;
  };
  R r[D];
  load(r[0], 0);
  normalize_q<HD, true>(qb, sl2);
  u4_t qt[NS];
  float qs[NS];
  tok_q_operands<HD, KB>(qb, qt, qs);
  store(r[0], 0);
#pragma unroll
  for (int k = 1; k <= D; ++k)
    if (k < n) load(r[k % D], k);
  wave_lds_sync();
  auto group = [&](int i) {
    const int nvalid = min(kTile, t_end - tok(i));
    const QkOut qk = tok_qk<HD, KB, L>(buf(i), qt, qs, lane, ((i & 1) ? big1 : big0) ? 0.f : kLazyLog2);
    if (nvalid == kTile) kivi_softmax_pv<HD, 8, VB, true, L>(qk, nvalid, buf(i), 0, acc, sl2, lane);
    else kivi_softmax_pv<HD, 8, VB, false, L>(qk, nvalid, buf(i), 0, acc, sl2, lane);
  };
  int i = 0;
  for (; i + 2 * D < n; i += D) {
#pragma unroll
    for (int j = 0; j < D; ++j) {
      group(i + j);
      store(r[(j + 1) % D], i + j + 1);
      load(r[(j + 1) % D], i + j + 1 + D);
      wave_lds_sync();
    }
  }
  for (; i < n; ++i) {
    group(i);
    if (i + 1 < n) {
      const int set = (i + 1) % D;
#pragma unroll
      for (int k = 0; k < D; ++k) {
        if (set == k) {
          store(r[k], i + 1);
          if (i + 1 + D < n) load(r[k], i + 1 + D);
        }
      }
      wave_lds_sync();
    }
  }
}

// V code position factor of result row e (4 g4 + e of a block): the power of two
// the PV product of a VB-bit segment carries on that row.
__device__ __forceinline__ float v_posfactor(int vb, int e) {
  return (vb == 2) ? (float)(1 << (2 * e)) : (vb == 4) ? ((e & 1) ? 16.f : 1.f) : 1.f;
}

// The segments of a device segment table (pk_segment_table_write) that one work
// item covers: entries 4 item .. 4 item + 3 of ts (kind kSegTable: kd = the table,
// length = entries), entry 4 item + w to wave w.  The wave runs its segment whole
// through the wave-private group pipeline (the host admits only segments that path
// reads).  One segment per wave keeps this straight-line code: in a loop over
// entries the compiler hoists every bit width's invariants and spills.  Returns the
// V width of the wave's segment (0 if it had none).
template <int HD, int MAXB>
__device__ __forceinline__ int table_entry(const SegDev& ts, int item, int b, int kvh, int wave,
                                           int lane, char* lds, u4_t (&qb)[HD / 32],
                                           WaveAcc<HD>& acc, float& sl2) {
  const int e = __builtin_amdgcn_readfirstlane(kWaves * item + wave);
  if (e >= ts.length) return 0;
  // only what the wave path reads, with the (batch, kv head) offsets folded into
  // the pointers: the entry's other fields never occupy registers
  const SegDev* tp = reinterpret_cast<const SegDev*>(ts.kd) + e;
  int len = tp->length;
  if (tp->seq_lens) len = min(len, tp->seq_lens[b]);
  if (len <= 0) return 0;
  const int kbits = tp->kbits, vbits = tp->vbits;
  SegDev s{};
  s.length = tp->length;
  s.kbits = kbits;
  s.vbits = vbits;
  s.kgs = tp->kgs;
  s.kd = tp->kd + (b * tp->kd_bs + kvh * tp->kd_hs);
  s.ks = tp->ks + (b * tp->km_bs + kvh * tp->km_hs);
  s.km = tp->km + (b * tp->km_bs + kvh * tp->km_hs);
  s.vd = tp->vd + (b * tp->vd_bs + kvh * tp->vd_hs);
  s.vs = tp->vs + (b * tp->vm_bs + kvh * tp->vm_hs);
  s.vm = tp->vm + (b * tp->vm_bs + kvh * tp->vm_hs);
  const SegOffsets o = {0, 0, 0, 0};
  // the waves of the item may hold different widths: buffers for the widest layout
  constexpr int B22 = GroupLayout<HD, 2, 2>::bytes, B24 = GroupLayout<HD, 2, 4>::bytes;
  constexpr int B42 = GroupLayout<HD, 4, 2>::bytes, B44 = GroupLayout<HD, 4, 4>::bytes;
  constexpr int B2x = B22 > B24 ? B22 : B24, B4x = B42 > B44 ? B42 : B44;
  constexpr int WB = 2 * ((MAXB >= 4) ? (B2x > B4x ? B2x : B4x) : B22);
  KivLoad kl;
  kl.row_bytes = ((int64_t)s.length * kbits + 7) / 8;
  kl.row_groups = (s.length + s.kgs - 1) / s.kgs;
  kl.k_rows = kl.row_bytes;
  kl.kmode = 16;
  kl.kdata_tm = true;
  kl.kmeta_gm = true;
  kl.gm_elems = false;
  kl.kmeta4 = false;
  switch (kbits * 16 + vbits) {
    case 0x22:
      kivi_wave_groups<HD, 2, 2>(s, o, kl, 0, len, wave, 0, 1, lane, lds, WB, qb, acc, sl2, true);
      break;
    case 0x24:
      if constexpr (MAXB >= 4)
        kivi_wave_groups<HD, 2, 4>(s, o, kl, 0, len, wave, 0, 1, lane, lds, WB, qb, acc, sl2, true);
      break;
    case 0x42:
      if constexpr (MAXB >= 4)
        kivi_wave_groups<HD, 4, 2>(s, o, kl, 0, len, wave, 0, 1, lane, lds, WB, qb, acc, sl2, true);
      break;
    case 0x44:
      if constexpr (MAXB >= 4)
        kivi_wave_groups<HD, 4, 4>(s, o, kl, 0, len, wave, 0, 1, lane, lds, WB, qb, acc, sl2, true);
      break;
    default:
      return 0;
  }
  return vbits;
}

// Every 64-byte line of the argument block read at once, at entry.  The fields a
// workgroup needs (header, segment table, launch sizes) are spread over about 25
// lines; read where they are used, each new line is a dependent scalar-cache
// miss.  Afterwards those loads hit.
__device__ __forceinline__ void touch_params(const DecodeParams& p) {
  constexpr int kWords = (int)(sizeof(DecodeParams) / 4);
  static_assert(kWords <= 26 * 16, "argument block above 26 lines");
  const uint32_t* w = reinterpret_cast<const uint32_t*>(&p);
  // one statement consumes every value: all 26 loads are in flight together
  asm volatile("" ::
               "s"(w[min(0, kWords - 1)]), "s"(w[min(16, kWords - 1)]), "s"(w[min(32, kWords - 1)]), "s"(w[min(48, kWords - 1)]),
               "s"(w[min(64, kWords - 1)]), "s"(w[min(80, kWords - 1)]), "s"(w[min(96, kWords - 1)]), "s"(w[min(112, kWords - 1)]),
               "s"(w[min(128, kWords - 1)]), "s"(w[min(144, kWords - 1)]), "s"(w[min(160, kWords - 1)]), "s"(w[min(176, kWords - 1)]),
               "s"(w[min(192, kWords - 1)]), "s"(w[min(208, kWords - 1)]), "s"(w[min(224, kWords - 1)]), "s"(w[min(240, kWords - 1)]),
               "s"(w[min(256, kWords - 1)]), "s"(w[min(272, kWords - 1)]), "s"(w[min(288, kWords - 1)]), "s"(w[min(304, kWords - 1)]),
               "s"(w[min(320, kWords - 1)]), "s"(w[min(336, kWords - 1)]), "s"(w[min(352, kWords - 1)]), "s"(w[min(368, kWords - 1)]),
               "s"(w[min(384, kWords - 1)]), "s"(w[min(400, kWords - 1)]));
}

// Two workgroups (8 waves) per CU: the register budget is capped so a second
// wave per SIMD hides LDS and dependency latency.
// TOK: the variant for launches of per-token K segments (and FP16 segments); the
// other variant takes KIVI segments, device tables and FP16 segments.  NW: waves per
// workgroup, 4 (two workgroups per CU) or 8 (one workgroup of two waves per SIMD, for
// launches of at most one workgroup per CU whose segments all take the wave-private
// group path; no device tables).  WO: only the wave-private group path (no workgroup
// stages, no device tables), for launches that need no more; the 8-wave variants are WO.
template <int HD, int MAXB, bool TOK, int NW, bool WO>
__global__ void __launch_bounds__(64 * NW, 8 / NW)
decode_mfma_kernel(const DecodeParams p) {
  static_assert(NW == kWaves || WO, "eight-wave variants take the wave path only");
  extern __shared__ __attribute__((aligned(16))) char lds[];
  constexpr int NB = HD / 16;
  constexpr int KS = HD / 32;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int n = lane & 15;
  const int g4 = lane >> 4;

  touch_params(p);
  const Block3 blk = p.order ? chunk_major_block() : xcd_block();
  const int b = blk.z;
  const int kvh = blk.y / p.nslab;
  const int slab = blk.y - kvh * p.nslab;
  const int h0 = kvh * p.G + slab * p.HS;
  const int nh = min(p.HS, p.G - slab * p.HS);

  // a register copy: fields read inside the group loop must not be reloaded
  // from the argument block (such a reload would sit in the in-order memory
  // counter behind the prefetched group and stall on it).  Segment 0 is read
  // before the segment is known: the host lists the segment with the costliest
  // (usually the most) chunks first, so most workgroups save one dependent round
  // trip.
  SegDev s = p.seg[0];
  if (p.nseg > 1 && blk.x >= p.seg[1].lbegin) {
    int si = 1;
    while (si + 1 < p.nseg && blk.x >= p.seg[si + 1].lbegin) ++si;
    s = p.seg[si];
  }
  const int local = blk.x - s.lbegin;
  const int cg = s.gbegin + local;
  int len_b = s.length;
  if (s.seq_lens) len_b = min(len_b, s.seq_lens[b]);
  const int t_begin = local * s.chunk_len;
  const int t_end = min(t_begin + s.chunk_len, len_b);

  // q of head n, lane's channels 32 s + 8 g4 .. + 7.  Padding columns (n >= nh)
  // repeat the slab's last head; their results are never written, and the
  // loads stay unconditional so they do not serialize with the first group's.
  u4_t qb[KS];
  const int nq = min(n, nh - 1);
#pragma unroll
  for (int k = 0; k < KS; ++k)
    qb[k] = *reinterpret_cast<const u4_t*>(p.q + (int64_t)b * p.q_bs + (int64_t)(h0 + nq) * p.q_hs +
                                           32 * k + 8 * g4);

  float sl2 = p.scale * kLog2e;

  WaveAcc<HD> acc;
#pragma unroll
  for (int i = 0; i < NB; ++i) acc.o[i] = f4_t{0.f, 0.f, 0.f, 0.f};
  acc.vbl = f4_t{0.f, 0.f, 0.f, 0.f};
  acc.m = -INFINITY;
  acc.mx = -INFINITY;
  acc.l = 0.f;

  int vb_bits = s.vbits;   // the V width the accumulators carry (KIVI, per-token K)
  auto fp16_chunk = [&]() {
    const uint16_t* kbase = reinterpret_cast<const uint16_t*>(s.kd) + b * s.kd_bs + kvh * s.kd_hs;
    const uint16_t* vbase = reinterpret_cast<const uint16_t*>(s.vd) + b * s.vd_bs + kvh * s.vd_hs;
    for (int t0 = t_begin + 32 * wave; t0 < t_end; t0 += 32 * NW)
      fp16_group<HD>(kbase, vbase, s.tok_stride, t0, min(32, t_end - t0), qb, acc, sl2, lane);
  };
  if constexpr (TOK) {
    if (s.kind == PK_SEG_FP16) {
      fp16_chunk();
    } else if (t_end > t_begin) {
      SegOffsets o;
      o.kd = b * s.kd_bs + kvh * s.kd_hs;
      o.km = b * s.km_bs + kvh * s.km_hs;
      o.vd = b * s.vd_bs + kvh * s.vd_hs;
      o.vm = b * s.vm_bs + kvh * s.vm_hs;
#define PK_TOK_CASE(KB_, VB_)                                                                  \
  case KB_ * 16 + VB_:                                                                         \
    if constexpr (KB_ <= MAXB && VB_ <= MAXB)                                                  \
      tok_wave_groups<HD, KB_, VB_, NW>(s, o, t_begin, t_end, wave, lane, lds, qb, acc, sl2);  \
    break;
      switch (s.kbits * 16 + s.vbits) {
        PK_TOK_CASE(2, 2) PK_TOK_CASE(2, 4) PK_TOK_CASE(2, 8)
        PK_TOK_CASE(4, 2) PK_TOK_CASE(4, 4) PK_TOK_CASE(4, 8)
        PK_TOK_CASE(8, 2) PK_TOK_CASE(8, 4) PK_TOK_CASE(8, 8)
        default: break;
      }
#undef PK_TOK_CASE
    }
  } else if (s.kind == kSegTable) {
    if constexpr (!WO)
      vb_bits = table_entry<HD, MAXB>(s, local, b, kvh, wave, lane, lds, qb, acc, sl2);
  } else if (s.kind == PK_SEG_FP16) {
    fp16_chunk();
  } else {
    SegOffsets o;
    o.kd = b * s.kd_bs + kvh * s.kd_hs;
    o.km = b * s.km_bs + kvh * s.km_hs;
    o.vd = b * s.vd_bs + kvh * s.vd_hs;
    o.vm = b * s.vm_bs + kvh * s.vm_hs;
    // the chunk's 128-token stages (none when a ragged row ends before it)
    const int kt_first = t_begin, kt_stride = kStage, kt_end = t_end;
    const int knst = (kt_end > kt_first) ? (kt_end - kt_first - 1) / kt_stride + 1 : 0;
    // only the bit widths up to MAXB are compiled into this kernel variant,
    // which keeps the register budget of the common 2/4-bit cases low
    // one switch: the cases exclude each other, so the q registers each case
    // normalizes in place are not carried from one case into the next
#define PK_KIVI_CASE(KB_, VB_)                                                                 \
  case KB_ * 16 + VB_:                                                                         \
    if constexpr (KB_ <= MAXB && VB_ <= MAXB)                                                  \
      kivi_chunk<HD, KB_, VB_, MAXB, NW, WO>(s, o, kt_first, kt_stride, knst, kt_end, wave, lane, tid, lds,  \
                                     p.stage_lds, qb, acc, sl2);                               \
    break;
    if (knst > 0) {
      switch (s.kbits * 16 + s.vbits) {
        PK_KIVI_CASE(2, 2) PK_KIVI_CASE(2, 4) PK_KIVI_CASE(2, 8)
        PK_KIVI_CASE(4, 2) PK_KIVI_CASE(4, 4) PK_KIVI_CASE(4, 8)
        PK_KIVI_CASE(8, 2) PK_KIVI_CASE(8, 4) PK_KIVI_CASE(8, 8)
        default: break;
      }
    }
#undef PK_KIVI_CASE
  }

  // ---- report (m, l, acc) against the true max of the wave's scores ----
  if (acc.mx != -INFINITY) {
    const float alpha = __builtin_amdgcn_exp2f(acc.m - acc.mx);
    acc.m = acc.mx;
    acc.l *= alpha;
    acc.vbl *= alpha;
#pragma unroll
    for (int i = 0; i < NB; ++i) acc.o[i] *= alpha;
  }
  // ---- wave results -> LDS, merge the 4 waves ----
  __syncthreads();
  // rows padded by 16 bytes: the 16 rows of one 16-byte store start 4 banks apart
  // (unpadded, every row of a store would hit the same 4 banks)
  constexpr int MP = HD + 4;
  float* mo = reinterpret_cast<float*>(lds);               // [NW][16][MP]
  float* mm = mo + NW * 16 * MP;                            // [NW][16]
  float* ml = mm + NW * 16;                                 // [NW][16]
  float l_full;
  if (s.kind == PK_SEG_FP16) {
    l_full = xsum4(acc.l);
    // result row r of block bb is channel NB r + bb: 8 consecutive channels per (g4, e)
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int bb = 0; bb < NB; bb += 4)
        *reinterpret_cast<f4_t*>(mo + (wave * 16 + n) * MP + NB * (4 * g4 + e) + bb) =
            f4_t{acc.o[bb][e], acc.o[bb + 1][e], acc.o[bb + 2][e], acc.o[bb + 3][e]};
  } else {
    // rows c < HD/32 of the bias product sit in lane group 0, row HD/32 in lane
    // group HD/128 (register (HD/32) % 4)
    constexpr int CG = HD / 32;
    float vbf[CG];
#pragma unroll
    for (int c = 0; c < CG; ++c) vbf[c] = __shfl(acc.vbl[c], n);
    l_full = __shfl(acc.vbl[CG % 4], 16 * (CG / 4) + n);
    // V code position factor of result row 4 g4 + e
    f4_t f;
#pragma unroll
    for (int e = 0; e < 4; ++e) f[e] = kTwo24 / v_posfactor(vb_bits, e);
#pragma unroll
    for (int bb = 0; bb < NB; ++bb)
      *reinterpret_cast<f4_t*>(mo + (wave * 16 + n) * MP + 16 * bb + 4 * g4) =
          acc.o[bb] * f + vbf[bb >> 1];
  }
  if (g4 == 0) {
    mm[wave * 16 + n] = acc.m;
    ml[wave * 16 + n] = l_full;
  }
  __syncthreads();
  // thread -> (head, 4 channels): the four waves' weights once per head, then
  // one 16-byte read per wave and one 16-byte store
  constexpr int Q = HD / 4;
  for (int i = tid; i < nh * Q; i += 64 * NW) {
    const int hh = i / Q, c = 4 * (i - hh * Q);
    float mw[NW];
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      mw[w] = mm[w * 16 + hh];
      M = fmaxf(M, mw[w]);
    }
    f4_t o = {0.f, 0.f, 0.f, 0.f};
    float L = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float wt = __builtin_amdgcn_exp2f(mw[w] - M);
        o += wt * *reinterpret_cast<const f4_t*>(mo + (w * 16 + hh) * MP + c);
        L += wt * ml[w * 16 + hh];
      }
    }
    const int64_t row = (int64_t)b * p.Hq + h0 + hh;
    *reinterpret_cast<f4_t*>(p.ws_acc + (row * p.C + cg) * HD + c) = o;
    if (c == 0) {
      p.ws_m[row * p.C + cg] = (M == -INFINITY) ? -INFINITY : M * kLn2;
      p.ws_l[row * p.C + cg] = L;
    }
  }
}

}  // namespace

// LDS bytes of one stage buffer: the largest layout of any (K, V) bit width
// pair a segment of the launch can have (K up to kb, V up to vb bits)
template <int HD>
inline int kivi_stage_bytes_hd(int kb, int vb) {
  const int sizes[3][3] = {
      {StageLayout<HD, 2, 2>::bytes, StageLayout<HD, 2, 4>::bytes, StageLayout<HD, 2, 8>::bytes},
      {StageLayout<HD, 4, 2>::bytes, StageLayout<HD, 4, 4>::bytes, StageLayout<HD, 4, 8>::bytes},
      {StageLayout<HD, 8, 2>::bytes, StageLayout<HD, 8, 4>::bytes, StageLayout<HD, 8, 8>::bytes}};
  int best = 0;
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 3; ++j)
      if ((2 << i) <= kb && (2 << j) <= vb) best = std::max(best, sizes[i][j]);
  return best;
}

// LDS bytes of one wave's group buffer (widths up to 4 bits; 0 if none fit)
template <int HD>
inline int kivi_group_bytes_hd(int kb, int vb) {
  const int sizes[2][2] = {{GroupLayout<HD, 2, 2>::bytes, GroupLayout<HD, 2, 4>::bytes},
                           {GroupLayout<HD, 4, 2>::bytes, GroupLayout<HD, 4, 4>::bytes}};
  int best = 0;
  for (int i = 0; i < 2; ++i)
    for (int j = 0; j < 2; ++j)
      if ((2 << i) <= kb && (2 << j) <= vb) best = std::max(best, sizes[i][j]);
  return best;
}

// LDS bytes of one wave's per-token group buffer (widths up to kb / vb bits)
template <int HD>
inline int tok_group_bytes_hd(int kb, int vb) {
  const int sizes[3][3] = {
      {TokLayout<HD, 2, 2>::bytes, TokLayout<HD, 2, 4>::bytes, TokLayout<HD, 2, 8>::bytes},
      {TokLayout<HD, 4, 2>::bytes, TokLayout<HD, 4, 4>::bytes, TokLayout<HD, 4, 8>::bytes},
      {TokLayout<HD, 8, 2>::bytes, TokLayout<HD, 8, 4>::bytes, TokLayout<HD, 8, 8>::bytes}};
  int best = 0;
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 3; ++j)
      if ((2 << i) <= kb && (2 << j) <= vb) best = std::max(best, sizes[i][j]);
  return best;
}

// The launch of one kernel variant (instantiated by one pk_decode_mfma[_tok][_w8|_wo]_<HD>_<MAXB>.hip
// each, so that the variants compile in parallel).
template <int HD, int MAXB, bool TOK, int NW, bool WO>
int launch_decode_mfma_variant(const DecodeParams& dp, dim3 grid, size_t lds, hipStream_t stream) {
  hipLaunchKernelGGL(HIP_KERNEL_NAME(decode_mfma_kernel<HD, MAXB, TOK, NW, WO>), grid, dim3(64 * NW), lds,
                     stream, dp);
  return check_launch("decode_mfma");
}

#define PK_DECLARE_MFMA_VARIANT(HD_, MB_)                                                        \
  int launch_decode_mfma_##HD_##_##MB_(const DecodeParams& dp, dim3 grid, size_t lds, hipStream_t stream); \
  int launch_decode_mfma_tok_##HD_##_##MB_(const DecodeParams& dp, dim3 grid, size_t lds, hipStream_t stream);
#define PK_DECLARE_MFMA_W8_VARIANT(HD_, MB_)                                                     \
  int launch_decode_mfma_w8_##HD_##_##MB_(const DecodeParams& dp, dim3 grid, size_t lds, hipStream_t stream); \
  int launch_decode_mfma_tok_w8_##HD_##_##MB_(const DecodeParams& dp, dim3 grid, size_t lds, hipStream_t stream); \
  int launch_decode_mfma_wo_##HD_##_##MB_(const DecodeParams& dp, dim3 grid, size_t lds, hipStream_t stream);
PK_DECLARE_MFMA_VARIANT(64, 2)
PK_DECLARE_MFMA_VARIANT(64, 4)
PK_DECLARE_MFMA_VARIANT(64, 8)
PK_DECLARE_MFMA_VARIANT(128, 2)
PK_DECLARE_MFMA_VARIANT(128, 4)
PK_DECLARE_MFMA_VARIANT(128, 8)
PK_DECLARE_MFMA_W8_VARIANT(64, 2)
PK_DECLARE_MFMA_W8_VARIANT(64, 4)
PK_DECLARE_MFMA_W8_VARIANT(128, 2)
PK_DECLARE_MFMA_W8_VARIANT(128, 4)
#undef PK_DECLARE_MFMA_W8_VARIANT
#undef PK_DECLARE_MFMA_VARIANT

}  // namespace pk

#ifdef PK_MFMA_HD
// one variant of the kernel per translation unit (PK_MFMA_TOK: the per-token K variant;
// PK_MFMA_W8: eight waves per workgroup; PK_MFMA_WO: four waves, wave-private group path
// only)
#ifndef PK_MFMA_W8
#define PK_MFMA_W8 0
#endif
#ifndef PK_MFMA_WO
#define PK_MFMA_WO 0
#endif
namespace pk {
#define PK_CAT3(a, b, c) a##b##_##c
#if PK_MFMA_WO
#define PK_VARIANT_NAME(HD_, MB_) PK_CAT3(launch_decode_mfma_wo_, HD_, MB_)
#define PK_VARIANT_TOK false
#elif defined(PK_MFMA_TOK) && PK_MFMA_W8
#define PK_VARIANT_NAME(HD_, MB_) PK_CAT3(launch_decode_mfma_tok_w8_, HD_, MB_)
#define PK_VARIANT_TOK true
#elif defined(PK_MFMA_TOK)
#define PK_VARIANT_NAME(HD_, MB_) PK_CAT3(launch_decode_mfma_tok_, HD_, MB_)
#define PK_VARIANT_TOK true
#elif PK_MFMA_W8
#define PK_VARIANT_NAME(HD_, MB_) PK_CAT3(launch_decode_mfma_w8_, HD_, MB_)
#define PK_VARIANT_TOK false
#else
#define PK_VARIANT_NAME(HD_, MB_) PK_CAT3(launch_decode_mfma_, HD_, MB_)
#define PK_VARIANT_TOK false
#endif
int PK_VARIANT_NAME(PK_MFMA_HD, PK_MFMA_MAXB)(const DecodeParams& dp, dim3 grid, size_t lds,
                                              hipStream_t stream) {
  return launch_decode_mfma_variant<PK_MFMA_HD, PK_MFMA_MAXB, PK_VARIANT_TOK,
                                    PK_MFMA_W8 ? 8 : kWaves, PK_MFMA_W8 || PK_MFMA_WO>(
      dp, grid, lds, stream);
}
#undef PK_VARIANT_TOK
#undef PK_VARIANT_NAME
#undef PK_CAT3
}  // namespace pk
#endif
