// Host memory for the host tier of the KV manager.
//
// Counterpart of the reference's HostBufferAllocator family
// (tpu_sync/core/host_memory_allocator.h:31-137): an allocation is a
// pointer, a size and an owner whose destruction frees it.
//   * kMalloc: 64-byte aligned, zeroed (the reference's posix_memalign
//     fallback, tpu_sync/kv_cache/kv_cache_manager_base.cc:329-345);
//   * kPinned: hipHostMalloc page-locked memory, zeroed, which the DMA
//     engines read and write directly (the reference's DmaMap'd host memory);
//   * kShm: a POSIX shared-memory segment that outlives the process, headed
//     by a schema record checked on warm boot (the reference's
//     SharedMemoryHostMemoryAllocator, host_memory_allocator.cc:245-411).
#ifndef KVX_HOST_HOST_ALLOCATOR_H_
#define KVX_HOST_HOST_ALLOCATOR_H_

#include <cstddef>
#include <cstdint>
#include <functional>
#include <memory>
#include <string>

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

// numa_node >= 0: the pages are allocated and first touched (zeroed) while
// the calling thread prefers that node; pinned memory then follows the
// thread's policy (hipHostMallocNumaUser).
StatusOr<HostBufferAllocation> AllocateMallocHost(size_t bytes, int numa_node = -1);
StatusOr<HostBufferAllocation> AllocatePinnedHost(size_t bytes, int device,
                                                  int numa_node = -1);

// Schema record at offset 0 of a shared-memory host pool. The layout is the
// reference's (tpu_sync/core/host_memory_allocator.h:95-108), so a segment
// left by either side is recognised (or rejected) by the other.
struct alignas(64) SharedMemoryHeader {
  uint64_t magic = 0x52414944454E5348ull;  // "RAIDENSH"
  uint32_t version = 1;
  char model_uid[256] = {0};
  uint32_t global_mesh_shape[5] = {0};
  uint32_t shard_layout[5] = {0};
  uint32_t num_blocks = 0;
  uint32_t block_size = 0;
  uint32_t num_heads = 0;
  uint32_t head_dim = 0;
  uint32_t itemsize = 0;
  uint64_t total_payload_bytes = 0;
  uint32_t reference_count = 0;
};
static_assert(sizeof(SharedMemoryHeader) == 384, "on-memory format");

// Name of the segment: "/<key>[_<server_name>][_dev_<device>]" (device < 0:
// no suffix), as the reference composes it (host_memory_allocator.cc:266-278).
std::string ShmSegmentName(const std::string& key, const std::string& server_name,
                           int device);

// Maps the segment `name` with `bytes` of payload after the header. Warm
// boot: an existing segment whose header matches `expected` (magic, version,
// model_uid, num_blocks, block_size, num_heads, head_dim, itemsize) and
// whose payload size is `bytes` is attached with its contents and its
// reference count incremented; anything else is unlinked and re-created
// zero-filled. The allocation points at the payload; releasing the owner
// decrements the reference count and unmaps, never unlinks. *warm reports
// which path was taken. numa_node >= 0: pages of the mapping not yet
// present prefer that node.
StatusOr<HostBufferAllocation> AllocateShmHost(const std::string& name,
                                               const SharedMemoryHeader& expected,
                                               size_t bytes, bool* warm,
                                               int numa_node = -1);

}  // namespace kvx

#endif  // KVX_HOST_HOST_ALLOCATOR_H_
