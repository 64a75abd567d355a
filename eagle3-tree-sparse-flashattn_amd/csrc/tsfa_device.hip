// Per-device cache of the attributes the forward planner needs (compute
// units, LDS per workgroup).

#include <atomic>

#include "tsfa_internal.h"

namespace tsfa {
namespace {

constexpr int kMaxDevices = 64;
std::atomic<int> g_cu_count[kMaxDevices];
std::atomic<int> g_max_lds[kMaxDevices];

int current_device(int* dev) {
  if (hipGetDevice(dev) != hipSuccess || *dev < 0 || *dev >= kMaxDevices) return TSFA_ERR_DEVICE;
  return TSFA_OK;
}

int cached_attr(std::atomic<int>* cache, hipDeviceAttribute_t attr, int* out) {
  int dev = 0;
  if (current_device(&dev) != TSFA_OK) return TSFA_ERR_DEVICE;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v <= 0) {
    if (hipDeviceGetAttribute(&v, attr, dev) != hipSuccess || v <= 0) return TSFA_ERR_DEVICE;
    cache[dev].store(v, std::memory_order_relaxed);
  }
  *out = v;
  return TSFA_OK;
}

}  // namespace

int device_cu_count(int* out) { return cached_attr(g_cu_count, hipDeviceAttributeMultiprocessorCount, out); }

int device_max_lds_per_block(int* out) {
  return cached_attr(g_max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, out);
}

}  // namespace tsfa

extern "C" int tsfa_device_limits(int32_t* out2) {
  if (out2 == nullptr) return TSFA_ERR_INVALID_ARGUMENT;
  int cus = 0, lds = 0;
  if (tsfa::device_cu_count(&cus) != TSFA_OK || tsfa::device_max_lds_per_block(&lds) != TSFA_OK)
    return TSFA_ERR_DEVICE;
  out2[0] = cus;
  out2[1] = lds;
  return TSFA_OK;
}
