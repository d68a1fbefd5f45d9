#include "arg_ring.h"

#include <algorithm>
#include <cstring>

#include "hip_util.h"

namespace kvx {
namespace {
constexpr int64_t kAlign = 256;
int64_t AlignUp(int64_t v) { return (v + kAlign - 1) / kAlign * kAlign; }
}  // namespace

ArgRing::~ArgRing() {
  for (Slice& s : inflight_) {
    (void)hipEventSynchronize(s.done);
    (void)hipEventDestroy(s.done);
  }
  if (host_ != nullptr) (void)hipHostFree(host_);
  if (dev_ != 0) (void)hipFree(reinterpret_cast<void*>(dev_));
}

Status ArgRing::Init(int64_t bytes) { return Grow(bytes); }

Status ArgRing::Grow(int64_t bytes) {
  for (Slice& s : inflight_) {
    KVX_HIP_RETURN_IF_ERROR(hipEventSynchronize(s.done));
    (void)hipEventDestroy(s.done);
  }
  inflight_.clear();
  if (host_ != nullptr) (void)hipHostFree(host_);
  if (dev_ != 0) (void)hipFree(reinterpret_cast<void*>(dev_));
  host_ = nullptr;
  dev_ = 0;
  const int64_t size = AlignUp(std::max(bytes, size_ * 2));
  void* h = nullptr;
  void* d = nullptr;
  KVX_HIP_RETURN_IF_ERROR(hipHostMalloc(&h, size, hipHostMallocDefault));
  KVX_HIP_RETURN_IF_ERROR(hipMalloc(&d, size));
  host_ = static_cast<uint8_t*>(h);
  dev_ = reinterpret_cast<uint64_t>(d);
  size_ = size;
  head_ = 0;
  return OkStatus();
}

StatusOr<int64_t> ArgRing::Alloc(int64_t bytes) {
  bytes = AlignUp(std::max<int64_t>(bytes, 1));
  // Room for several requests of this size, so a launch can be prepared
  // while the previous ones still read their tables.
  if (bytes > size_) KVX_RETURN_IF_ERROR(Grow(4 * bytes));
  int64_t start = head_;
  if (start + bytes > size_) start = 0;
  const int64_t end = start + bytes;
  for (auto it = inflight_.begin(); it != inflight_.end();) {
    const bool overlap = it->begin < end && start < it->end;
    hipError_t q = hipEventQuery(it->done);
    if (q == hipErrorNotReady && overlap) {
      KVX_HIP_RETURN_IF_ERROR(hipEventSynchronize(it->done));
      q = hipSuccess;
    }
    if (q == hipErrorNotReady) {
      ++it;
      continue;
    }
    (void)hipEventDestroy(it->done);
    it = inflight_.erase(it);
  }
  head_ = end;
  return start;
}

Status ArgRing::Upload(int64_t off, int64_t bytes, hipStream_t stream) {
  KVX_HIP_RETURN_IF_ERROR(hipMemcpyAsync(reinterpret_cast<void*>(dev_ + off), host_ + off,
                                         bytes, hipMemcpyHostToDevice, stream));
  return OkStatus();
}

Status ArgRing::Commit(int64_t off, int64_t bytes, hipStream_t stream) {
  hipEvent_t e = nullptr;
  KVX_HIP_RETURN_IF_ERROR(hipEventCreateWithFlags(&e, hipEventDisableTiming));
  Status st = HipStatus(hipEventRecord(e, stream), "hipEventRecord(arg ring)");
  if (!st.ok()) {
    (void)hipEventDestroy(e);
    return st;
  }
  inflight_.push_back(Slice{off, off + AlignUp(bytes), e});
  return OkStatus();
}

void WriteStridedImage(const std::vector<StridedEntryDev>& table, uint32_t grid, uint8_t* out) {
  const size_t tbytes = table.size() * sizeof(StridedEntryDev);
  std::memcpy(out, table.data(), tbytes);
  uint32_t* map = reinterpret_cast<uint32_t*>(out + tbytes);
  for (size_t e = 0; e < table.size(); ++e) {
    const uint32_t end = e + 1 < table.size() ? table[e + 1].tile_begin : grid;
    for (uint32_t t = table[e].tile_begin; t < end; ++t) map[t] = static_cast<uint32_t>(e);
  }
}

Status LaunchStridedThroughRing(ArgRing& ring, const std::vector<StridedCopy>& copies,
                                hipStream_t stream, uint32_t max_workgroups,
                                hipEvent_t kernel_start) {
  if (copies.empty()) return OkStatus();
  const int vec = StridedVectorBytes(copies);
  std::vector<StridedEntryDev> table;
  uint32_t grid = 0, long_tiles = 0;
  if (!BuildStridedTable(copies, vec, &table, &grid, &long_tiles)) {
    return InvalidArgumentError("strided copy entry out of the kernel's limits");
  }
  const int64_t bytes = StridedImageBytes(table.size(), grid);
  KVX_ASSIGN_OR_RETURN(int64_t off, ring.Alloc(bytes));
  ArgSliceGuard keep([&ring, off, bytes, stream] { return ring.Commit(off, bytes, stream); },
                     stream);
  WriteStridedImage(table, grid, ring.host(off));
  KVX_RETURN_IF_ERROR(ring.Upload(off, bytes, stream));
  if (kernel_start != nullptr) KVX_HIP_RETURN_IF_ERROR(hipEventRecord(kernel_start, stream));
  KVX_HIP_RETURN_IF_ERROR(LaunchStridedCopy(
      reinterpret_cast<const StridedEntryDev*>(ring.dev(off)),
      static_cast<uint32_t>(table.size()), grid, vec, stream, max_workgroups, long_tiles));
  return keep.Commit();
}

}  // namespace kvx
