// Host memory for the host tier of the KV manager.
//
// Counterpart of the reference's HostBufferAllocator family
// (tpu_sync/core/host_memory_allocator.h:31-137): an allocation is a
// pointer, a size and an owner whose destruction frees it.
//   * kMalloc: 64-byte aligned, zeroed (the reference's posix_memalign
//     fallback, tpu_sync/kv_cache/kv_cache_manager_base.cc:329-345);
//   * kPinned: hipHostMalloc page-locked memory, zeroed, which the DMA
//     engines read and write directly (the reference's DmaMap'd host memory).
#ifndef KVX_HOST_HOST_ALLOCATOR_H_
#define KVX_HOST_HOST_ALLOCATOR_H_

#include <cstddef>
#include <cstdint>
#include <functional>
#include <memory>

#include "status.h"

namespace kvx {

struct HostBufferAllocation {
  uint8_t* ptr = nullptr;
  size_t size = 0;
  std::shared_ptr<void> owner;
};

enum class HostAllocKind : int { kMalloc = 0, kPinned = 1, kShm = 2 };

using HostBufferAllocator =
    std::function<StatusOr<HostBufferAllocation>(size_t bytes)>;

StatusOr<HostBufferAllocation> AllocateMallocHost(size_t bytes);
StatusOr<HostBufferAllocation> AllocatePinnedHost(size_t bytes, int device);

}  // namespace kvx

#endif  // KVX_HOST_HOST_ALLOCATOR_H_
