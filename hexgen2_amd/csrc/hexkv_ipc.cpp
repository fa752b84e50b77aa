// Same-GPU, cross-process handoff of device buffers (hexkv_ipc_* in hexkv.h):
// HIP IPC memory handles for the sender's allocations, process-wide
// refcounted mappings on the receiver, and DLPack wrappers so a receiving
// framework can alias the mapped bytes without a copy.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <map>
#include <mutex>
#include <new>
#include <string>

#include "hexkv_common.h"

namespace hexkv {

static_assert(sizeof(hexkv_ipc_handle) == sizeof(hipIpcMemHandle_t), "IPC handle size");

// One mapping per exported allocation, shared by every tensor wrapped on it.
struct Mapping {
  void *base = nullptr;
  int refs = 0;
};

static std::mutex g_lock;
static std::map<std::string, Mapping> g_by_handle;  // handle bytes -> mapping
static std::map<void *, std::string> g_by_base;     // base -> handle bytes

static int release_base(void *base) {
  std::lock_guard<std::mutex> guard(g_lock);
  auto it = g_by_base.find(base);
  if (it == g_by_base.end()) return fail(HEXKV_EINVAL, "hexkv_ipc_close: %p is not an open mapping", base);
  Mapping &m = g_by_handle[it->second];
  if (--m.refs > 0) return HEXKV_OK;
  // Work enqueued on any stream may still read the mapping: drain the device
  // before it goes away.
  hipError_t err = hipDeviceSynchronize();
  hipError_t err2 = hipIpcCloseMemHandle(base);
  g_by_handle.erase(it->second);
  g_by_base.erase(it);
  if (err != hipSuccess) return fail(HEXKV_EHIP, "hexkv_ipc_close: %s", hipGetErrorString(err));
  if (err2 != hipSuccess) return fail(HEXKV_EHIP, "hexkv_ipc_close: %s", hipGetErrorString(err2));
  return HEXKV_OK;
}

// DLPack v0.8 ABI (dlpack.h, the framework-neutral tensor exchange format):
// only the fields this library fills.
struct DLDevice {
  int32_t device_type;  // kDLROCM = 10
  int32_t device_id;
};
struct DLDataType {
  uint8_t code;  // kDLInt 0, kDLUInt 1, kDLFloat 2, kDLBfloat 4, kDLBool 6
  uint8_t bits;
  uint16_t lanes;
};
struct DLTensor {
  void *data;
  DLDevice device;
  int32_t ndim;
  DLDataType dtype;
  int64_t *shape;
  int64_t *strides;
  uint64_t byte_offset;
};
struct DLManagedTensor {
  DLTensor dl_tensor;
  void *manager_ctx;
  void (*deleter)(DLManagedTensor *self);
};

constexpr int kMaxDims = 8;
constexpr size_t kMaxIpcBytes = size_t(1) << 31;

struct Wrapped {
  DLManagedTensor managed;
  int64_t shape[kMaxDims];
  void *base;  // mapping released on delete
};

static void delete_wrapped(DLManagedTensor *self) {
  Wrapped *w = static_cast<Wrapped *>(self->manager_ctx);
  release_base(w->base);
  delete w;
}

}  // namespace hexkv

extern "C" int hexkv_ipc_export(const void *ptr, hexkv_ipc_handle *handle, uint64_t *offset,
                                uint64_t *alloc_bytes) {
  using namespace hexkv;
  clear_error();
  if (!ptr || !handle || !offset || !alloc_bytes) return fail(HEXKV_EINVAL, "hexkv_ipc_export: null argument");
  hipDeviceptr_t base = nullptr;
  size_t size = 0;
  hipError_t err = hipMemGetAddressRange(&base, &size, const_cast<void *>(ptr));
  if (err != hipSuccess) return fail(HEXKV_EHIP, "hexkv_ipc_export: %s", hipGetErrorString(err));
  // Mapping an allocation of 2 GiB or more in another process has not
  // returned on this platform: refuse to hand out a handle for one.
  if (size >= kMaxIpcBytes)
    return fail(HEXKV_ERANGE, "hexkv_ipc_export: allocation of %zu bytes; exported allocations must be below 2 GiB",
                size);
  hipIpcMemHandle_t h;
  err = hipIpcGetMemHandle(&h, base);
  if (err != hipSuccess) return fail(HEXKV_EHIP, "hexkv_ipc_export: %s", hipGetErrorString(err));
  memcpy(handle->bytes, &h, sizeof(h));
  *offset = static_cast<uint64_t>(static_cast<const char *>(ptr) - static_cast<const char *>(base));
  *alloc_bytes = size;
  return HEXKV_OK;
}

extern "C" int hexkv_ipc_open(const hexkv_ipc_handle *handle, void **base) {
  using namespace hexkv;
  clear_error();
  if (!handle || !base) return fail(HEXKV_EINVAL, "hexkv_ipc_open: null argument");
  std::lock_guard<std::mutex> guard(g_lock);
  const std::string key(reinterpret_cast<const char *>(handle->bytes), sizeof(handle->bytes));
  auto it = g_by_handle.find(key);
  if (it != g_by_handle.end()) {
    ++it->second.refs;
    *base = it->second.base;
    return HEXKV_OK;
  }
  hipIpcMemHandle_t h;
  memcpy(&h, handle->bytes, sizeof(h));
  void *p = nullptr;
  hipError_t err = hipIpcOpenMemHandle(&p, h, hipIpcMemLazyEnablePeerAccess);
  if (err != hipSuccess) return fail(HEXKV_EHIP, "hexkv_ipc_open: %s", hipGetErrorString(err));
  Mapping m;
  m.base = p;
  m.refs = 1;
  g_by_handle[key] = m;
  g_by_base[p] = key;
  *base = p;
  return HEXKV_OK;
}

extern "C" int hexkv_ipc_close(void *base) {
  hexkv::clear_error();
  return hexkv::release_base(base);
}

extern "C" void *hexkv_ipc_dlpack(void *base, uint64_t offset, int ndim, const int64_t *shape,
                                  int dtype_code, int dtype_bits, int device_id) {
  using namespace hexkv;
  clear_error();
  if (!base || ndim < 0 || ndim > kMaxDims || (ndim > 0 && !shape) || dtype_bits <= 0) {
    fail(HEXKV_EINVAL, "hexkv_ipc_dlpack: bad arguments");
    return nullptr;
  }
  Wrapped *w = new (std::nothrow) Wrapped();
  if (!w) {
    fail(HEXKV_EINVAL, "hexkv_ipc_dlpack: out of host memory");
    return nullptr;
  }
  for (int i = 0; i < ndim; ++i) w->shape[i] = shape[i];
  w->base = base;
  DLTensor &t = w->managed.dl_tensor;
  t.data = static_cast<char *>(base) + offset;
  t.device.device_type = 10;  // kDLROCM
  t.device.device_id = device_id;
  t.ndim = ndim;
  t.dtype.code = static_cast<uint8_t>(dtype_code);
  t.dtype.bits = static_cast<uint8_t>(dtype_bits);
  t.dtype.lanes = 1;
  t.shape = w->shape;
  t.strides = nullptr;  // compact row-major
  t.byte_offset = 0;
  w->managed.manager_ctx = w;
  w->managed.deleter = delete_wrapped;
  return &w->managed;
}
