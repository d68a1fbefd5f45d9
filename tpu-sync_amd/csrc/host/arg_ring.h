// Pinned-host + device ring for kernel argument tables.
//
// A launch writes its table into the pinned half, uploads it with one
// hipMemcpyAsync on the launching stream (no stream of its own, which would
// take a share of the process's hardware queues) and records an event after
// the launch; a region is handed out again only once the event that last read it
// has completed (the host waits only when the ring wraps onto unfinished
// work). Not thread-safe: the owner serialises calls.
#ifndef KVX_HOST_ARG_RING_H_
#define KVX_HOST_ARG_RING_H_

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <deque>
#include <functional>
#include <vector>

#include "../kernels/strided_copy.h"
#include "status.h"

namespace kvx {

class ArgRing {
 public:
  ArgRing() = default;
  ~ArgRing();
  ArgRing(const ArgRing&) = delete;
  ArgRing& operator=(const ArgRing&) = delete;

  Status Init(int64_t bytes);
  // Reserves `bytes` (256-aligned); returns the offset. Grows the ring to
  // four such requests (after draining it) when one is larger than the ring.
  StatusOr<int64_t> Alloc(int64_t bytes);
  uint8_t* host(int64_t off) const { return host_ + off; }
  uint64_t dev(int64_t off) const { return dev_ + static_cast<uint64_t>(off); }
  // Uploads [off, off + bytes) on `stream`, ahead of the launch that reads it.
  Status Upload(int64_t off, int64_t bytes, hipStream_t stream);
  // Marks [off, off + bytes) in use until the work now enqueued on `stream`
  // finishes.
  Status Commit(int64_t off, int64_t bytes, hipStream_t stream);

 private:
  struct Slice {
    int64_t begin;
    int64_t end;
    hipEvent_t done;
  };
  Status Grow(int64_t bytes);
  uint8_t* host_ = nullptr;
  uint64_t dev_ = 0;
  int64_t size_ = 0;
  int64_t head_ = 0;
  std::deque<Slice> inflight_;
};

// Keeps an argument-table slice reserved on every return path. A slice whose
// upload has been queued may be read by that upload and by the launches
// after it, so it must be committed (its completion event recorded on the
// launching stream) even when a later step fails: Commit() does it on the
// success path, the destructor on an early return. If recording the event
// fails, the stream is drained instead, so nothing in flight can still read
// the slice when the ring hands it out again.
class ArgSliceGuard {
 public:
  ArgSliceGuard(std::function<Status()> commit, hipStream_t stream)
      : commit_(std::move(commit)), stream_(stream) {}
  ~ArgSliceGuard() {
    if (!done_) (void)Commit();
  }
  ArgSliceGuard(const ArgSliceGuard&) = delete;
  ArgSliceGuard& operator=(const ArgSliceGuard&) = delete;
  Status Commit() {
    done_ = true;
    Status st = commit_();
    if (!st.ok()) (void)hipStreamSynchronize(stream_);
    return st;
  }

 private:
  std::function<Status()> commit_;
  hipStream_t stream_;
  bool done_ = false;
};

// The device image a strided launch reads: the entry table followed by the
// tile -> entry map (one uint32 per workgroup of `grid`).
inline int64_t StridedImageBytes(size_t entries, uint32_t grid) {
  return static_cast<int64_t>(entries * sizeof(StridedEntryDev)) + static_cast<int64_t>(grid) * 4;
}
// Writes that image to `out` (StridedImageBytes(table.size(), grid) bytes).
void WriteStridedImage(const std::vector<StridedEntryDev>& table, uint32_t grid, uint8_t* out);

// Uploads the table and tile map of `copies` through `ring` and launches the
// strided-copy kernel on `stream` (at most max_workgroups workgroups when
// > 0); the ring region stays reserved until the launch ends. A non-null
// `kernel_start` is recorded on `stream` after the upload, right before the
// launch (to time the kernel alone).
Status LaunchStridedThroughRing(ArgRing& ring, const std::vector<StridedCopy>& copies,
                                hipStream_t stream, uint32_t max_workgroups = 0,
                                hipEvent_t kernel_start = nullptr);

}  // namespace kvx

#endif  // KVX_HOST_ARG_RING_H_
