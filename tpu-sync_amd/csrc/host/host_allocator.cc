#include "host_allocator.h"

#include <hip/hip_runtime_api.h>

#include <cstdlib>
#include <cstring>
#include <string>

#include "hip_util.h"

namespace kvx {

StatusOr<HostBufferAllocation> AllocateMallocHost(size_t bytes) {
  HostBufferAllocation a;
  if (bytes == 0) return a;
  void* p = nullptr;
  if (posix_memalign(&p, 64, bytes) != 0) {
    return ResourceExhaustedError("Failed to allocate host buffer of size: " +
                                  std::to_string(bytes));
  }
  std::memset(p, 0, bytes);
  a.ptr = static_cast<uint8_t*>(p);
  a.size = bytes;
  a.owner = std::shared_ptr<void>(p, [](void* q) { free(q); });
  return a;
}

StatusOr<HostBufferAllocation> AllocatePinnedHost(size_t bytes, int device) {
  HostBufferAllocation a;
  if (bytes == 0) return a;
  DeviceGuard g(device);
  void* p = nullptr;
  hipError_t e = hipHostMalloc(&p, bytes, hipHostMallocDefault);
  if (e != hipSuccess) {
    return ResourceExhaustedError("hipHostMalloc of " + std::to_string(bytes) +
                                  " bytes failed: " + hipGetErrorString(e));
  }
  std::memset(p, 0, bytes);
  a.ptr = static_cast<uint8_t*>(p);
  a.size = bytes;
  a.owner = std::shared_ptr<void>(p, [](void* q) { (void)hipHostFree(q); });
  return a;
}

}  // namespace kvx
