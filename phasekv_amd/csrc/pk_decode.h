// Device-side descriptors of the decode work list (shared by the decode kernels).
#pragma once

#include "pk_common.h"

namespace pk {

constexpr int kThreads = 256;                 // threads per decode workgroup
constexpr int kMaxSeg = PK_MAX_SEGMENTS_PER_LAUNCH;
constexpr int kCombineMaxHd = 256;            // largest head_dim handled by the combine
constexpr int kCombineLoads = 8;             // partials in flight per combine thread
constexpr int kCombineTarget = 4;            // partials per combine thread the host aims at
constexpr int kMinChunk = 64;                 // auto chunk lengths are multiples of this

// One segment as the kernels see it (element strides, see pk_segment).
struct SegDev {
  int kind, length, kbits, vbits, kgs, vgs;
  int chunk_len;      // tokens per chunk (work item)
  int n_chunks;       // chunks of this segment
  int gbegin;         // index of its first chunk among all chunks of a (batch, kv head)
  int lbegin;         // index of its first chunk within this launch (blockIdx.x)
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
  int wave_lds;       // MFMA kernel: LDS bytes of one wave's tile staging
  SegDev seg[kMaxSeg];
};

// MFMA fast path (pk_decode_mfma.hip): same parameters and partial layout.
int launch_decode_mfma(const DecodeParams& dp, int lchunks, int max_kbits, int max_vbits,
                       hipStream_t stream);

}  // namespace pk
