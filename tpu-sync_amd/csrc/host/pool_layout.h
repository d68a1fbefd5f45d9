// Byte-level block pool geometry over a wrapped storage: the reference's
// pool layout (tpu_sync/kv_cache/pool_layout.h:31-164), same rules and
// answers.
//
// A pool is num_blocks equally strided blocks starting at base_offset_bytes
// of one storage; every block carries the same regions of live bytes. A
// region is num_units strided runs of units_per_stride * unit_bytes live
// bytes. Host mirrors share the storage layout, so one byte offset addresses
// both sides of a device<->host copy; ComputePoolBlockCopyExtents returns
// the coalesced live extents of a block-id list (padding never copied).
#ifndef KVX_HOST_POOL_LAYOUT_H_
#define KVX_HOST_POOL_LAYOUT_H_

#include <cstddef>
#include <cstdint>
#include <string>
#include <utility>
#include <vector>

#include "status.h"

namespace kvx {

struct RegionSpec {
  std::string name;
  int64_t offset_bytes = 0;
  int64_t stride_bytes = 0;
  int64_t unit_bytes = 0;
  int64_t num_units = 0;
  int64_t units_per_stride = 1;
  // Saturate at INT64_MAX on overflow (as the reference does).
  int64_t live_bytes() const;
  int64_t extent_end_bytes() const;
  Status Validate(int64_t slot_bytes) const;
};

struct PoolSpec {
  std::string tag;
  size_t storage_index = 0;
  int64_t base_offset_bytes = 0;
  int64_t block_stride_bytes = 0;
  int64_t num_blocks = 0;
  std::vector<RegionSpec> regions;
  std::string dtype_tag;
  // End of the last live byte of the last block in the storage.
  int64_t storage_extent_end_bytes() const;
  // storage_bytes < 0 skips the storage-size check.
  Status Validate(int64_t storage_bytes) const;
};

struct PoolBlockCopyExtent {
  int64_t offset_bytes = 0;
  int64_t size_bytes = 0;
};

struct PoolLiveSegment {
  int64_t logical_offset = 0;
  int64_t physical_offset = 0;
  int64_t size = 0;
};

struct LiveCopyChunk {
  int64_t src_physical = 0;
  int64_t dst_physical = 0;
  int64_t size = 0;
};

bool RegionsCoverRange(const std::vector<RegionSpec>& regions, size_t start, size_t end);

// Sorted, coalesced live extents of `block_ids` (OutOfRange for a bad id).
StatusOr<std::vector<PoolBlockCopyExtent>> ComputePoolBlockCopyExtents(
    const PoolSpec& pool, const std::vector<int64_t>& block_ids);

// Physical live runs of one block with compact (logical) offsets.
StatusOr<std::vector<PoolLiveSegment>> ExpandPoolLiveSegments(const PoolSpec& pool);

StatusOr<std::pair<int64_t, int64_t>> PhysicalLiveRangeToLogical(
    const std::vector<PoolLiveSegment>& segments, int64_t physical_offset, int64_t size);

// Splits a compact-live copy at every source or destination run boundary.
StatusOr<std::vector<LiveCopyChunk>> TranslateLiveCopy(
    const std::vector<PoolLiveSegment>& src_segments,
    const std::vector<PoolLiveSegment>& dst_segments, int64_t src_offset,
    int64_t dst_offset, int64_t size);

}  // namespace kvx

#endif  // KVX_HOST_POOL_LAYOUT_H_
