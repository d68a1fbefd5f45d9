#include "device_memory.h"

#include <hip/hip_runtime_api.h>

#include <atomic>
#include <cstring>
#include <string>

namespace kvx {
namespace {

AddressInfo HipQuery(uint64_t addr) {
  AddressInfo out;
  hipPointerAttribute_t a;
  std::memset(&a, 0, sizeof(a));
  if (hipPointerGetAttributes(&a, reinterpret_cast<const void*>(addr)) != hipSuccess) {
    // An address the runtime does not know: it also records the failure as
    // this thread's last error, which must not surface in a later call.
    (void)hipGetLastError();
    return out;
  }
  switch (a.type) {
    case hipMemoryTypeDevice:
      out.kind = MemKind::kDevice;
      break;
    case hipMemoryTypeHost:
      out.kind = MemKind::kHost;
      break;
    case hipMemoryTypeUnregistered:
      return out;
    default:
      out.kind = MemKind::kOther;
      break;
  }
  out.device = a.device;
  if (out.kind == MemKind::kDevice) {
    hipDeviceptr_t base = nullptr;
    size_t size = 0;
    if (hipMemGetAddressRange(&base, &size, reinterpret_cast<hipDeviceptr_t>(addr)) ==
        hipSuccess) {
      out.base = reinterpret_cast<uint64_t>(base);
      out.size = size;
    } else {
      (void)hipGetLastError();
    }
  }
  return out;
}

std::atomic<AddressQuery> g_query{nullptr};

AddressInfo Lookup(uint64_t addr) {
  AddressQuery q = g_query.load(std::memory_order_acquire);
  return q != nullptr ? q(addr) : HipQuery(addr);
}

}  // namespace

void SetAddressQueryForTesting(AddressQuery q) { g_query.store(q, std::memory_order_release); }

Status DeviceRangeChecker::Check(uint64_t addr, uint64_t bytes, const char* what) {
  if (bytes == 0) return OkStatus();
  const std::string name(what);
  if (addr == 0) return InvalidArgumentError(name + ": null device address");
  uint64_t end = 0;
  if (__builtin_add_overflow(addr, bytes, &end)) {
    return InvalidArgumentError(name + ": address range overflows");
  }
  for (const auto& k : known_) {
    if (addr >= k.first && end <= k.second) return OkStatus();
  }
  const AddressInfo a = Lookup(addr);
  switch (a.kind) {
    case MemKind::kDevice:
      break;
    case MemKind::kHost:
      return InvalidArgumentError(name + ": host memory where a device buffer is required");
    case MemKind::kOther:
      return InvalidArgumentError(name + ": managed or other non-device memory where a "
                                         "device buffer is required");
    default:
      return InvalidArgumentError(name + ": not a device allocation (host or unknown "
                                         "address) where a device buffer is required");
  }
  if (device_ < 0) device_ = a.device;
  if (a.device != device_) {
    return InvalidArgumentError(name + ": memory of device " + std::to_string(a.device) +
                                ", not of device " + std::to_string(device_));
  }
  if (a.size > 0) {
    if (addr < a.base || end > a.base + a.size) {
      return InvalidArgumentError(name + ": range runs past the end of its device allocation");
    }
    known_.emplace_back(a.base, a.base + a.size);
  }
  return OkStatus();
}

bool StridedExtent(int64_t size, int64_t count, int64_t stride, uint64_t* bytes) {
  if (size <= 0 || count <= 0 || stride < 0) return false;
  int64_t last = 0;
  if (__builtin_mul_overflow(count - 1, stride, &last) ||
      __builtin_add_overflow(last, size, &last)) {
    return false;
  }
  *bytes = static_cast<uint64_t>(last);
  return true;
}

}  // namespace kvx
