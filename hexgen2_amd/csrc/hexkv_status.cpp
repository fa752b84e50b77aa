// Per-thread error reporting, version, the per-device symbol lookup and the
// device queries of the hexkv C ABI (host code only).
#include <stdarg.h>
#include <stdio.h>

#include <mutex>

#include "hexkv_common.h"

namespace hexkv {

static thread_local char g_last_error[512] = "";

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_last_error[0] = '\0'; }

int check_launch(const char *what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(HEXKV_EHIP, "%s: %s", what, hipGetErrorString(err));
  return HEXKV_OK;
}

int stream_device(hexkv_stream_t stream, int *dev, const char *what) {
  const hipError_t e = stream ? hipStreamGetDevice(static_cast<hipStream_t>(stream), dev) : hipGetDevice(dev);
  if (e != hipSuccess) return fail(HEXKV_EHIP, "%s: cannot tell the stream's device: %s", what, hipGetErrorString(e));
  if (*dev < 0 || *dev >= kMaxDevices)
    return fail(HEXKV_EUNSUPPORTED, "%s: device %d beyond the %d the library tracks", what, *dev, kMaxDevices);
  return HEXKV_OK;
}

int stream_xcds(hexkv_stream_t stream, int *xcds, const char *what) {
  static std::atomic<int> cache[kMaxDevices];
  int dev = 0;
  int rc = stream_device(stream, &dev, what);
  if (rc != HEXKV_OK) return rc;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    const hipError_t e = hipDeviceGetAttribute(&n, hipDeviceAttributeNumberOfXccs, dev);
    if (e != hipSuccess) return fail(HEXKV_EHIP, "%s: XCD count of device %d: %s", what, dev, hipGetErrorString(e));
    n = n > 0 ? n : 1;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  *xcds = n;
  return HEXKV_OK;
}

static std::mutex g_symbol_mu;

int symbol_address(const void *symbol, std::atomic<void *> *cache, hexkv_stream_t stream, void **addr,
                   const char *what) {
  int dev = 0;
  int rc = stream_device(stream, &dev, what);
  if (rc != HEXKV_OK) return rc;
  void *ptr = cache[dev].load(std::memory_order_acquire);
  if (ptr) {
    *addr = ptr;
    return HEXKV_OK;
  }
  std::lock_guard<std::mutex> lock(g_symbol_mu);
  ptr = cache[dev].load(std::memory_order_relaxed);
  if (!ptr) {
    int current = 0;
    hipError_t e = hipGetDevice(&current);
    if (e != hipSuccess) return fail(HEXKV_EHIP, "%s: hipGetDevice: %s", what, hipGetErrorString(e));
    if (current != dev && (e = hipSetDevice(dev)) != hipSuccess)
      return fail(HEXKV_EHIP, "%s: hipSetDevice(%d): %s", what, dev, hipGetErrorString(e));
    e = hipGetSymbolAddress(&ptr, symbol);
    const hipError_t back = current != dev ? hipSetDevice(current) : hipSuccess;
    if (e != hipSuccess || !ptr)
      return fail(HEXKV_EHIP, "%s: hipGetSymbolAddress on device %d: %s", what, dev, hipGetErrorString(e));
    if (back != hipSuccess)
      return fail(HEXKV_EHIP, "%s: restoring device %d: %s", what, current, hipGetErrorString(back));
    cache[dev].store(ptr, std::memory_order_release);
  }
  *addr = ptr;
  return HEXKV_OK;
}

}  // namespace hexkv

extern "C" int hexkv_version(void) { return 200; /* 0.2.0 */ }

extern "C" const char *hexkv_last_error(void) { return hexkv::g_last_error; }

extern "C" int hexkv_device_xcds(int32_t *xcds) {
  using namespace hexkv;
  clear_error();
  if (!xcds) return fail(HEXKV_EINVAL, "hexkv_device_xcds: null argument");
  int dev = 0, n = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&n, hipDeviceAttributeNumberOfXccs, dev);
  if (e != hipSuccess) return fail(HEXKV_EHIP, "hexkv_device_xcds: %s", hipGetErrorString(e));
  *xcds = n > 0 ? n : 1;
  return HEXKV_OK;
}
