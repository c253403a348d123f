// Library-level C entry points: errors, version, device info.
#include "pk_common.h"

#include <mutex>
#include <vector>

namespace pk {

static thread_local char g_last_error[512];

static void copy_text(size_t at, const char* text) noexcept {
  if (!text) return;
  while (*text && at + 1 < sizeof(g_last_error)) g_last_error[at++] = *text++;
  g_last_error[at] = 0;
}

void set_error(const std::string& msg) {
  g_last_error[0] = 0;
  copy_text(0, msg.c_str());
}

void set_error_text(const char* a, const char* b) noexcept {
  g_last_error[0] = 0;
  copy_text(0, a);
  size_t n = 0;
  while (n < sizeof(g_last_error) && g_last_error[n]) ++n;
  copy_text(n, b);
}

void clear_error() noexcept { g_last_error[0] = 0; }

int device_cu_count() {
  static std::mutex mu;
  static std::vector<int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  std::lock_guard<std::mutex> lock(mu);
  if (dev >= static_cast<int>(cache.size())) cache.resize(dev + 1, 0);
  if (cache[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    cache[dev] = cus;
  }
  return cache[dev];
}

}  // namespace pk

extern "C" const char* pk_last_error(void) { return pk::g_last_error; }

extern "C" const char* pk_version(void) { return "phasekv_hip 0.1 gfx950"; }

extern "C" int pk_device_info(int device, int* cu_count, int* lds_bytes_per_cu, int* wave_size,
                              int* l2_bytes) {
  return pk::guarded("pk_device_info", [&]() -> int {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
      return pk::fail("hipDeviceGetAttribute(MultiprocessorCount) failed"), PK_ERR_RUNTIME;
    if (cu_count) *cu_count = v;
    if (lds_bytes_per_cu) {
      v = 0;
      hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, device);
      *lds_bytes_per_cu = v;
    }
    if (wave_size) {
      v = 0;
      hipDeviceGetAttribute(&v, hipDeviceAttributeWarpSize, device);
      *wave_size = v;
    }
    if (l2_bytes) {
      v = 0;
      hipDeviceGetAttribute(&v, hipDeviceAttributeL2CacheSize, device);
      *l2_bytes = v;
    }
    return PK_OK;
  });
}
