// Shared helpers of the PhaseKV HIP library (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include <new>
#include <string>

#include "phasekv_hip.h"

namespace pk {

// Thread-local error message behind pk_last_error(): a fixed buffer, so that
// recording an error never allocates or throws (longer messages are cut).
void set_error(const std::string& msg);
void set_error_text(const char* a, const char* b) noexcept;
void clear_error() noexcept;

// Body of every extern "C" entry point: no C++ exception crosses the ABI.  A
// failed host allocation or any other exception becomes PK_ERR_RUNTIME with a
// message naming the entry point.
template <class F>
inline int guarded(const char* what, F&& body) noexcept {
  try {
    return body();
  } catch (const std::bad_alloc&) {
    set_error_text(what, ": out of host memory");
  } catch (...) {
    set_error_text(what, ": unexpected C++ exception");
  }
  return PK_ERR_RUNTIME;
}

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
