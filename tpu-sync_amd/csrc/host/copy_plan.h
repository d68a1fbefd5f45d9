// Block-id lists to run-coalesced copy specs, and the receive-side load plan
// (tpu_sync/core/kv_cache_manager_with_transfer.cc:294-426).
//
// A spec is parallel (src, dst, size) vectors in blocks. OffsetsImpl pairs a
// block-id list with the compact positions 0..n-1 (the contiguous staging
// side), splitting where ids stop being consecutive; BuildCoalescedCopySpec
// pairs two id lists and splits where either side stops. BuildLoadCopyPlan
// orders the transport by remote id and the host-to-device copy by local id,
// dropping repeated local ids (which must name the same host id).
#ifndef KVX_HOST_COPY_PLAN_H_
#define KVX_HOST_COPY_PLAN_H_

#include <cstdint>
#include <vector>

#include "status.h"

namespace kvx {

struct CopySpec {
  std::vector<int64_t> src_offsets;
  std::vector<int64_t> dst_offsets;
  std::vector<int64_t> sizes;
};

struct CopyPlan {
  int64_t num_blocks = 0;
  std::vector<int64_t> requested_remote_block_ids;
  std::vector<int64_t> requested_local_block_ids;
  // Transport order: sorted (stably) by remote id.
  std::vector<int64_t> producer_remote_block_ids;
  std::vector<int64_t> transport_host_block_ids;
  // Host-to-device order: sorted (stably) by local id, duplicates dropped.
  std::vector<int64_t> h2d_local_block_ids;
  std::vector<int64_t> h2d_host_block_ids;
  CopySpec h2d_copy;  // host ids -> local ids, coalesced
};

CopySpec OffsetsImpl(const std::vector<int64_t>& block_ids, bool source_is_compact);
StatusOr<CopySpec> BuildCoalescedCopySpec(const std::vector<int64_t>& src_block_ids,
                                          const std::vector<int64_t>& dst_block_ids);
StatusOr<CopyPlan> BuildLoadCopyPlan(const std::vector<int64_t>& remote_block_ids,
                                     const std::vector<int64_t>& local_block_ids,
                                     const std::vector<int64_t>& local_host_block_ids);

}  // namespace kvx

#endif  // KVX_HOST_COPY_PLAN_H_
