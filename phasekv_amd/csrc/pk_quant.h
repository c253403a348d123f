// Per-element arithmetic of the grouped min/max quantization, shared by the pack
// kernels and the fused cooling kernel so both give the same bits.  Follows
// src/phasekv/kernels/packing.py:123-155 of the reference: IEEE float32 with
// explicit round-to-nearest intrinsics, min/max propagating NaN.
#pragma once

#include "pk_common.h"

namespace pk {

// min / max with NaN propagation (torch.amin / amax semantics).
__device__ __forceinline__ float nan_min(float a, float b) { return (b < a || b != b) ? b : a; }
__device__ __forceinline__ float nan_max(float a, float b) { return (b > a || b != b) ? b : a; }

struct GroupStats {
  float mn;
  float scale;   // float32 scale used for the codes (the fp16 copy is what is stored)
};

// scale = max(max - min, 1e-8) / qmax (clamp_(min=1e-8) keeps NaN)
__device__ __forceinline__ GroupStats group_stats_from(float mn, float mx, int bits) {
  float range = __fsub_rn(mx, mn);
  range = (range < 1e-8f) ? 1e-8f : range;
  return GroupStats{mn, __fdiv_rn(range, static_cast<float>((1 << bits) - 1))};
}

// code = clamp(round_half_even((v - min) / scale), 0, qmax)
__device__ __forceinline__ uint32_t quant_code(float v, const GroupStats& s, int bits) {
  const float qmax = static_cast<float>((1 << bits) - 1);
  float q = rintf(__fdiv_rn(__fsub_rn(v, s.mn), s.scale));
  q = fminf(fmaxf(q, 0.0f), qmax);
  return static_cast<uint32_t>(q);
}

}  // namespace pk
