#include "copy_plan.h"

#include <algorithm>
#include <numeric>

namespace kvx {
namespace {

// Calls emit(start, end) for each maximal run of positions [start, end) in
// [0, n) such that consecutive(i) holds for every i in (start, end).
template <typename Step, typename Emit>
void ForEachRun(int64_t n, Step consecutive, Emit emit) {
  for (int64_t start = 0; start < n;) {
    int64_t end = start + 1;
    while (end < n && consecutive(end)) ++end;
    emit(start, end);
    start = end;
  }
}

std::vector<size_t> StableOrder(const std::vector<int64_t>& keys) {
  std::vector<size_t> order(keys.size());
  std::iota(order.begin(), order.end(), size_t{0});
  std::stable_sort(order.begin(), order.end(),
                   [&](size_t a, size_t b) { return keys[a] < keys[b]; });
  return order;
}

}  // namespace

CopySpec OffsetsImpl(const std::vector<int64_t>& ids, bool source_is_compact) {
  CopySpec spec;
  const int64_t n = static_cast<int64_t>(ids.size());
  ForEachRun(
      n, [&](int64_t i) { return ids[i] == ids[i - 1] + 1; },
      [&](int64_t s, int64_t e) {
        spec.src_offsets.push_back(source_is_compact ? s : ids[s]);
        spec.dst_offsets.push_back(source_is_compact ? ids[s] : s);
        spec.sizes.push_back(e - s);
      });
  return spec;
}

StatusOr<CopySpec> BuildCoalescedCopySpec(const std::vector<int64_t>& src,
                                          const std::vector<int64_t>& dst) {
  if (src.size() != dst.size()) {
    return InvalidArgumentError("src and dst block lists must have same length");
  }
  CopySpec spec;
  ForEachRun(
      static_cast<int64_t>(src.size()),
      [&](int64_t i) { return src[i] == src[i - 1] + 1 && dst[i] == dst[i - 1] + 1; },
      [&](int64_t s, int64_t e) {
        spec.src_offsets.push_back(src[s]);
        spec.dst_offsets.push_back(dst[s]);
        spec.sizes.push_back(e - s);
      });
  return spec;
}

StatusOr<CopyPlan> BuildLoadCopyPlan(const std::vector<int64_t>& remote,
                                     const std::vector<int64_t>& local,
                                     const std::vector<int64_t>& host) {
  if (remote.size() != local.size() || local.size() != host.size()) {
    return InvalidArgumentError(
        "remote_block_ids, local_block_ids, and local_host_block_ids must have same length");
  }
  CopyPlan plan;
  plan.num_blocks = static_cast<int64_t>(remote.size());
  plan.requested_remote_block_ids = remote;
  plan.requested_local_block_ids = local;
  if (remote.empty()) return plan;
  for (size_t i : StableOrder(remote)) {
    plan.producer_remote_block_ids.push_back(remote[i]);
    plan.transport_host_block_ids.push_back(host[i]);
  }
  for (size_t i : StableOrder(local)) {
    if (!plan.h2d_local_block_ids.empty() && plan.h2d_local_block_ids.back() == local[i]) {
      if (plan.h2d_host_block_ids.back() != host[i]) {
        return InvalidArgumentError(
            "Duplicate local block IDs must map to the same host block ID");
      }
      continue;
    }
    plan.h2d_local_block_ids.push_back(local[i]);
    plan.h2d_host_block_ids.push_back(host[i]);
  }
  KVX_ASSIGN_OR_RETURN(plan.h2d_copy,
                       BuildCoalescedCopySpec(plan.h2d_host_block_ids, plan.h2d_local_block_ids));
  return plan;
}

}  // namespace kvx
