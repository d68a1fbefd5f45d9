// Small HIP helpers shared by the host-side library.
#ifndef KVX_HOST_HIP_UTIL_H_
#define KVX_HOST_HIP_UTIL_H_

#include <hip/hip_runtime_api.h>

#include <cstdlib>
#include <initializer_list>
#include <string>
#include <vector>

#include "status.h"

namespace kvx {

inline Status HipStatus(hipError_t e, const char* what) {
  if (e == hipSuccess) return OkStatus();
  return InternalError(std::string(what) + ": " + hipGetErrorName(e) + " (" +
                       hipGetErrorString(e) + ")");
}

#define KVX_HIP_RETURN_IF_ERROR(expr) \
  KVX_RETURN_IF_ERROR(::kvx::HipStatus((expr), #expr))

// Makes `device` current for the scope and restores the caller's device, so
// calls into the library never change the device a framework thread uses.
class DeviceGuard {
 public:
  explicit DeviceGuard(int device) {
    if (hipGetDevice(&prev_) != hipSuccess) prev_ = -1;
    if (prev_ != device) {
      ok_ = hipSetDevice(device) == hipSuccess;
      restore_ = ok_ && prev_ >= 0;
    }
  }
  ~DeviceGuard() {
    if (restore_) (void)hipSetDevice(prev_);
  }
  bool ok() const { return ok_; }
  DeviceGuard(const DeviceGuard&) = delete;
  DeviceGuard& operator=(const DeviceGuard&) = delete;

 private:
  int prev_ = -1;
  bool ok_ = true;
  bool restore_ = false;
};

// Hardware queues per process the HIP runtime uses: GPU_MAX_HW_QUEUES, or
// its default of 4.
inline int HwQueuesPerProcess() {
  const char* v = std::getenv("GPU_MAX_HW_QUEUES");
  const int n = v != nullptr ? std::atoi(v) : 0;
  return n >= 1 && n <= 64 ? n : 4;
}

// Creates non-blocking streams meant to land on distinct hardware queues
// (best effort: the placement rests on the runtime's observed policy, not on
// a documented guarantee).
//
// The HIP runtime backs a process's streams with at most GPU_MAX_HW_QUEUES
// hardware queues (4 by default): the first streams get new queues, later
// ones join the queue with the fewest streams, ties going to the same queue
// each time. Streams created one after another can therefore share a queue
// when the pool fills between them, and streams on one queue run in order:
// an offload's DMA and a reload's DMA on one queue serialize (measured:
// offload+reload of Llama-3-8B batches at 54 instead of 96 GB/s when one
// stream existed before the engine's). One short-lived spacer stream per
// hardware queue, created first, fills the pool and evens out counts that
// differ by at most one, so the streams created next each join a different
// queue. Counts that differ by more (many streams created elsewhere on one
// queue) can still put two of them on one queue; more spacers (`spacers`,
// default one per hardware queue) even out larger differences.
// CreateStreamsOnDistinctQueuesChecked (queue_check.h) checks the result.
inline Status CreateStreamsOnDistinctQueues(const std::vector<hipStream_t*>& out,
                                            int spacers = 0) {
  std::vector<hipStream_t> sp(static_cast<size_t>(spacers > 0 ? spacers : HwQueuesPerProcess()),
                              nullptr);
  Status st = OkStatus();
  for (hipStream_t& s : sp) {
    if (st.ok()) st = HipStatus(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "spacer stream");
  }
  for (hipStream_t* s : out) {
    if (st.ok()) st = HipStatus(hipStreamCreateWithFlags(s, hipStreamNonBlocking), "stream");
  }
  for (hipStream_t s : sp) {
    if (s != nullptr) (void)hipStreamDestroy(s);
  }
  return st;
}

inline Status CreateStreamsOnDistinctQueues(std::initializer_list<hipStream_t*> out) {
  return CreateStreamsOnDistinctQueues(std::vector<hipStream_t*>(out));
}

}  // namespace kvx

#endif  // KVX_HOST_HIP_UTIL_H_
