// Shared helpers of the PhaseKV HIP library (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include <string>

#include "phasekv_hip.h"

namespace pk {

// Thread-local error message behind pk_last_error().
void set_error(const std::string& msg);
void clear_error();

inline int fail(const std::string& msg) {
  set_error(msg);
  return PK_ERR_INVALID;
}

inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error(std::string(what) + ": " + hipGetErrorString(e));
    return PK_ERR_RUNTIME;
  }
  return PK_OK;
}

inline bool valid_bits(int bits) { return bits == 2 || bits == 4 || bits == 8; }

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Number of compute units of the current device (cached per device).
int device_cu_count();

}  // namespace pk

// fp16 bit pattern <-> float on the device.
__device__ __forceinline__ float pk_h2f(uint16_t h) {
  return __half2float(__ushort_as_half(h));
}
__device__ __forceinline__ uint16_t pk_f2h(float f) {
  return __half_as_ushort(__float2half_rn(f));
}
__device__ __forceinline__ float pk_bf2f(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}
