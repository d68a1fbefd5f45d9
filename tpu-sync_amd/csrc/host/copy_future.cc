#include "copy_future.h"

#include <chrono>
#include <list>
#include <thread>

#include "hip_util.h"

namespace kvx {

// One process-wide thread runs every OnReady callback whose copy was not yet
// done at registration: it polls the pending copies (never blocking on one
// while another may finish first) and calls each callback, outside its lock,
// once its copy is done. A callback that blocks delays the ones after it.
class ReadyPoller {
 public:
  static ReadyPoller& Get() {
    // Never destroyed: callbacks may still be pending at process exit.
    static ReadyPoller* p = new ReadyPoller();
    return *p;
  }
  void Add(std::shared_ptr<CopyFuture::State> s, std::function<void(Status)> cb) {
    {
      std::lock_guard<std::mutex> l(mu_);
      items_.push_back(Item{std::move(s), std::move(cb)});
    }
    cv_.notify_one();
  }

 private:
  struct Item {
    std::shared_ptr<CopyFuture::State> state;
    std::function<void(Status)> cb;
  };
  ReadyPoller() {
    std::thread([this] { Loop(); }).detach();
  }
  void Loop() {
    while (true) {
      std::list<Item> ready;
      {
        std::unique_lock<std::mutex> l(mu_);
        cv_.wait(l, [this] { return !items_.empty(); });
        for (auto it = items_.begin(); it != items_.end();) {
          auto next = std::next(it);
          if (CopyFuture::StateReady(*it->state)) ready.splice(ready.end(), items_, it);
          it = next;
        }
      }
      for (Item& r : ready) r.cb(CopyFuture::StateAwait(*r.state));
      if (ready.empty()) std::this_thread::sleep_for(std::chrono::microseconds(20));
    }
  }
  std::mutex mu_;
  std::condition_variable cv_;
  std::list<Item> items_;
};

CopyFuture::State::~State() {
  for (hipEvent_t e : events) {
    if (e != nullptr) (void)hipEventDestroy(e);
  }
}

CopyFuture::CopyFuture(Status status) : state_(std::make_shared<State>()) {
  state_->status = std::move(status);
  state_->done = true;
}

CopyFuture CopyFuture::FromEvents(std::vector<hipEvent_t> events,
                                  std::vector<std::shared_ptr<void>> keep_alive) {
  CopyFuture f;
  f.state_->events = std::move(events);
  f.state_->keep_alive = std::move(keep_alive);
  f.state_->done = f.state_->events.empty();
  return f;
}

CopyFuture CopyFuture::Join(const std::vector<CopyFuture>& futures) {
  CopyFuture f;
  f.state_->done = false;
  for (const CopyFuture& c : futures) {
    if (c.state_) f.state_->children.push_back(c.state_);
  }
  return f;
}

CopyFuture CopyFuture::Pending() {
  CopyFuture f;
  f.state_->done = false;
  f.state_->pending = true;
  return f;
}

void CopyFuture::Fulfill(const CopyFuture& issued) const {
  std::lock_guard<std::mutex> l(state_->mu);
  if (!state_->pending) return;
  if (issued.state_) state_->children.push_back(issued.state_);
  state_->pending = false;
  state_->cv.notify_all();
}

void CopyFuture::Reject(Status status) const {
  std::lock_guard<std::mutex> l(state_->mu);
  if (!state_->pending) return;
  state_->status = std::move(status);
  state_->pending = false;
  state_->done = true;
  state_->cv.notify_all();
}

void CopyFuture::WaitIssued(const State& s) {
  std::unique_lock<std::mutex> l(s.mu);
  s.cv.wait(l, [&s] { return !s.pending; });
}

bool CopyFuture::StateReady(const State& s) {
  {
    std::lock_guard<std::mutex> l(s.mu);
    if (s.pending) return false;
    if (s.done) return true;
  }
  for (const auto& c : s.children) {
    if (!StateReady(*c)) return false;
  }
  for (hipEvent_t e : s.events) {
    hipError_t q = hipEventQuery(e);
    if (q == hipErrorNotReady) return false;
  }
  return true;
}

Status CopyFuture::StatePoll(const State& s) {
  {
    std::lock_guard<std::mutex> l(s.mu);
    if (!s.status.ok()) return s.status;
    if (s.done || s.pending) return OkStatus();
  }
  for (const auto& c : s.children) {
    Status st = StatePoll(*c);
    if (!st.ok()) return st;
  }
  for (hipEvent_t e : s.events) {
    hipError_t q = hipEventQuery(e);
    if (q != hipSuccess && q != hipErrorNotReady) {
      return HipStatus(q, "copy completion event");
    }
  }
  return OkStatus();
}

Status CopyFuture::StateAwait(State& s) {
  WaitIssued(s);
  {
    std::lock_guard<std::mutex> l(s.mu);
    if (s.done) return s.status;
  }
  Status result = OkStatus();
  for (const auto& c : s.children) {
    Status st = StateAwait(*c);
    if (result.ok() && !st.ok()) result = st;
  }
  for (hipEvent_t e : s.events) {
    Status st = HipStatus(hipEventSynchronize(e), "copy completion event");
    if (result.ok() && !st.ok()) result = st;
  }
  std::lock_guard<std::mutex> l(s.mu);
  if (!s.done) {
    if (s.status.ok()) s.status = result;
    s.done = true;
    s.keep_alive.clear();
  }
  return s.status;
}

bool CopyFuture::IsReady() const { return StateReady(*state_); }

Status CopyFuture::PollError() const { return StatePoll(*state_); }

Status CopyFuture::Await() const { return StateAwait(*state_); }

Status CopyFuture::WaitOnStream(hipStream_t stream) const {
  std::vector<const State*> stack{state_.get()};
  while (!stack.empty()) {
    const State* s = stack.back();
    stack.pop_back();
    WaitIssued(*s);
    for (const auto& c : s->children) stack.push_back(c.get());
    for (hipEvent_t e : s->events) {
      KVX_HIP_RETURN_IF_ERROR(hipStreamWaitEvent(stream, e, 0));
    }
  }
  return OkStatus();
}

void CopyFuture::OnReady(std::function<void(Status)> cb) const {
  if (StateReady(*state_)) {
    cb(Await());
    return;
  }
  ReadyPoller::Get().Add(state_, std::move(cb));
}

}  // namespace kvx
