#include "host_copy_pool.h"

#include <algorithm>

#include "stream_copy.h"

namespace kvx {

HostCopyPool::HostCopyPool(int threads) {
  for (int t = 0; t < threads; ++t) workers_.emplace_back([this] { Work(); });
}

HostCopyPool::~HostCopyPool() {
  {
    std::lock_guard<std::mutex> l(mu_);
    stop_ = true;
  }
  cv_.notify_all();
  for (std::thread& t : workers_) t.join();
}

void HostCopyPool::Copy(const std::vector<Segment>& segs) {
  constexpr size_t kPiece = 4u << 20;
  std::vector<Segment> pieces;
  for (const Segment& s : segs) {
    for (size_t o = 0; o < s.bytes; o += kPiece) {
      pieces.push_back(Segment{s.dst + o, s.src + o, std::min(kPiece, s.bytes - o)});
    }
  }
  if (pieces.empty()) return;
  std::lock_guard<std::mutex> call(call_mu_);
  {
    std::lock_guard<std::mutex> l(mu_);
    batch_ = &pieces;
    next_.store(0);
    left_ = pieces.size();
    ++generation_;
  }
  cv_.notify_all();
  Drain(&pieces);
  std::unique_lock<std::mutex> l(mu_);
  done_cv_.wait(l, [this] { return left_ == 0 && active_ == 0; });
  batch_ = nullptr;
}

void HostCopyPool::Drain(const std::vector<Segment>* p) {
  const size_t n = p->size();
  // Many small pieces (random blocks of a pageable tier: each crosses
  // several 4 KiB pages) are taken four at a time, so a thread knows its
  // next piece and prefetches it while it copies the current one; few
  // pieces are taken one at a time to keep every thread busy.
  const size_t take = n >= 64 * (workers_.size() + 1) ? 4 : 1;
  size_t finished = 0;
  for (size_t i = next_.fetch_add(take); i < n; i = next_.fetch_add(take)) {
    const size_t e = std::min(n, i + take);
    if (take > 1) PrefetchSource((*p)[i].src, (*p)[i].bytes);
    for (size_t j = i; j < e; ++j) {
      if (j + 1 < e) PrefetchSource((*p)[j + 1].src, (*p)[j + 1].bytes);
      // Streaming stores: the DMA engines read and write the same host
      // memory meanwhile, and the bytes are not read again by this CPU.
      StreamCopy((*p)[j].dst, (*p)[j].src, (*p)[j].bytes);
      ++finished;
    }
  }
  // Completion is published under mu_ below; whoever reads these bytes
  // (a DMA issued afterwards, the caller) comes after it.
  StreamFence();
  if (finished > 0) {
    std::lock_guard<std::mutex> l(mu_);
    left_ -= finished;
    if (left_ == 0 && active_ == 0) done_cv_.notify_all();
  }
}

void HostCopyPool::Work() {
  uint64_t seen = 0;
  while (true) {
    const std::vector<Segment>* p = nullptr;
    {
      std::unique_lock<std::mutex> l(mu_);
      cv_.wait(l, [&] { return stop_ || (generation_ != seen && batch_ != nullptr); });
      if (stop_) return;
      seen = generation_;
      p = batch_;
      ++active_;
    }
    Drain(p);
    std::lock_guard<std::mutex> l(mu_);
    if (--active_ == 0 && left_ == 0) done_cv_.notify_all();
  }
}

}  // namespace kvx
