// Async completion handle of a copy: the HIP counterpart of the reference's
// raiden::PjRtCopyFuture / RaidenFuture (tpu_sync/core/raw_transfer_core.h:379-621,
// tpu_sync/core/raiden_future.h:25-36). IsReady never blocks, PollError is a
// non-blocking error probe, Await blocks and returns the final status,
// OnReady runs a callback once the copy is done. A future keeps the buffers
// its copy touches alive until completion (the reference's buffer holds).
//
// Completion is a set of hipEvent_t recorded at the tail of the streams the
// copy used; WaitOnStream lets a consumer stream wait on the copy without
// blocking the host (no reference counterpart: PJRT has no streams).
#ifndef KVX_HOST_COPY_FUTURE_H_
#define KVX_HOST_COPY_FUTURE_H_

#include <hip/hip_runtime_api.h>

#include <condition_variable>
#include <functional>
#include <memory>
#include <mutex>
#include <vector>

#include "status.h"

namespace kvx {

class CopyFuture {
 public:
  // An already-completed future carrying `status`.
  explicit CopyFuture(Status status = OkStatus());

  // Takes ownership of `events` (destroyed with the last copy of the future).
  static CopyFuture FromEvents(std::vector<hipEvent_t> events,
                               std::vector<std::shared_ptr<void>> keep_alive);

  // Joins futures: ready when all are, first error wins.
  static CopyFuture Join(const std::vector<CopyFuture>& futures);

  // A future whose copy is issued later (queued dispatch): not ready until
  // Fulfill hands it the issued copy's future or Reject an error. Await and
  // WaitOnStream block until then.
  static CopyFuture Pending();
  void Fulfill(const CopyFuture& issued) const;
  void Reject(Status status) const;

  bool IsValid() const { return state_ != nullptr; }
  bool IsReady() const;
  Status PollError() const;
  Status Await() const;
  Status WaitOnStream(hipStream_t stream) const;
  void OnReady(std::function<void(Status)> cb) const;

 private:
  struct State {
    std::vector<hipEvent_t> events;
    std::vector<std::shared_ptr<void>> keep_alive;
    std::vector<std::shared_ptr<State>> children;
    Status status;
    mutable std::mutex mu;
    mutable std::condition_variable cv;
    bool pending = false;  // a queued dispatch has not issued the copy yet
    bool done = false;
    ~State();
  };
  friend class ReadyPoller;
  static void WaitIssued(const State& s);
  static bool StateReady(const State& s);
  static Status StatePoll(const State& s);
  static Status StateAwait(State& s);
  std::shared_ptr<State> state_;
};

}  // namespace kvx

#endif  // KVX_HOST_COPY_FUTURE_H_
