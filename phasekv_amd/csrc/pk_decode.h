// Device-side descriptors of the decode work list (shared by the decode kernels).
#pragma once

#include "pk_common.h"

namespace pk {

constexpr int kThreads = 256;                 // threads per decode workgroup
constexpr int kMaxSeg = PK_MAX_SEGMENTS_PER_LAUNCH;
constexpr int kCombineMaxHd = 256;            // largest head_dim handled by the combine
constexpr int kCombineLoads = 8;             // partials in flight per combine thread
constexpr int kCombineTarget = 4;            // partials per combine thread the host aims at
constexpr int kCombineRowsThreads = 128;     // threads per workgroup of the many-rows combine
constexpr int kMinChunk = 64;                 // auto chunk lengths are multiples of this

constexpr uint32_t kXcds = 8;                 // accelerator complex dies of an MI355X
// Launch-internal segment kind: the work items over a device segment table (kd =
// the table of SegDev entries, length = entries, chunk_len = entries per item).
constexpr int kSegTable = 8;

// The workgroup's coordinates in an XCD-contiguous order.  The dispatcher hands
// consecutive workgroups (x fastest, then y, then z) round-robin to the 8 XCDs,
// each with its own L2.  Renumbering the linear id so that XCD i runs the i-th
// contiguous eighth of the grid makes neighbouring chunks of one kv row, which
// share the cache lines of the token-packed K codes and of the K scales, meet
// in one L2 instead of being fetched once per XCD.
struct Block3 {
  int x, y, z;
};
__device__ inline Block3 xcd_block() {
  const uint32_t gx = gridDim.x, gy = gridDim.y;
  const uint32_t n = gx * gy * gridDim.z;
  const uint32_t lin = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
  const uint32_t xcd = lin % kXcds, k = lin / kXcds;
  const uint32_t q = n / kXcds, r = n % kXcds;
  const uint32_t id = xcd * q + (xcd < r ? xcd : r) + k;
  Block3 o;
  o.x = (int)(id % gx);
  o.y = (int)((id / gx) % gy);
  o.z = (int)(id / (gx * gy));
  return o;
}

// Chunk-major order: the hardware dispatches workgroups in linear order, so with
// the chunk index varying slowest every row's chunk 0 goes out first.  The host
// numbers the costliest chunks first, so that workgroups beyond the resident
// capacity are the cheap ones.  (No XCD grouping: with token-major K and
// group-major metadata neighbouring chunks share no lines.)
__device__ inline Block3 chunk_major_block() {
  const uint32_t gx = gridDim.x, gy = gridDim.y;
  const uint32_t rows = gy * gridDim.z;
  const uint32_t lin = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
  const uint32_t r = lin % rows;
  Block3 o;
  o.x = (int)(lin / rows);
  o.y = (int)(r % gy);
  o.z = (int)(r / gy);
  return o;
}

// One segment as the kernels see it (element strides, see pk_segment).
struct SegDev {
  int kind, length, kbits, vbits, kgs, vgs;
  int chunk_len;      // tokens per chunk (work item)
  int n_chunks;       // chunks of this segment
  int gbegin;         // index of its first chunk among all chunks of a (batch, kv head)
  int lbegin;         // index of its first chunk within this launch (blockIdx.x)
  int kmeta_gm;       // KIVI K scale/min stored group major ([groups][hd] per batch row, kv head)
  int kdata_tm;       // KIVI K codes stored token-byte major ([bytes][hd] per batch row, kv head)
  int hd_meta;        // head_dim (the group-major row length)
  const int32_t* seq_lens;
  const uint8_t* kd; const uint16_t* ks; const uint16_t* km;
  const uint8_t* vd; const uint16_t* vs; const uint16_t* vm;
  int64_t kd_bs, kd_hs, km_bs, km_hs, vd_bs, vd_hs, vm_bs, vm_hs;
  int64_t tok_stride;
};

struct DecodeParams {
  int B, Hq, Hkv, hd, G;
  int HS;             // query heads per workgroup (head slab)
  int nslab;          // slabs per kv head
  int tile;           // tokens per LDS tile (generic kernel)
  float scale;        // 1 / sqrt(hd)
  const uint16_t* q;
  int64_t q_bs, q_hs;
  float* ws_m;        // [B*Hq][C]
  float* ws_l;        // [B*Hq][C]
  float* ws_acc;      // [B*Hq][C][hd]
  int C;              // chunks per (batch, kv head) over all segments
  int nseg;
  int stage_lds;      // MFMA kernel: LDS bytes of one stage buffer (two are used)
  int order;          // MFMA kernel: 1 = chunk-major workgroup order, 0 = grouped by XCD
  SegDev seg[kMaxSeg];
};

// MFMA fast path (pk_decode_mfma.hip): same parameters and partial layout.  waves: 4, or 8
// for a launch whose segments all take the wave-private group path (no device table,
// codes up to 4 bits).
// wave_only: every segment takes the wave-private group path (no workgroup stages, no
// device table), so the smaller wave-path-only variant serves the launch.
int launch_decode_mfma(const DecodeParams& dp, int lchunks, int max_kbits, int max_vbits,
                       int waves, bool wave_only, hipStream_t stream);

}  // namespace pk
