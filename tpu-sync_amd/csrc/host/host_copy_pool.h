// A fixed pool of host threads that copy batches of segments in parallel with
// the calling thread. The pageable lanes use it to move bytes between their
// pinned bounce buffers and pageable host memory (malloc, /dev/shm).
#ifndef KVX_HOST_HOST_COPY_POOL_H_
#define KVX_HOST_HOST_COPY_POOL_H_

#include <atomic>
#include <condition_variable>
#include <cstddef>
#include <cstdint>
#include <mutex>
#include <thread>
#include <vector>

namespace kvx {

class HostCopyPool {
 public:
  struct Segment {
    uint8_t* dst;
    const uint8_t* src;
    size_t bytes;
  };

  // `threads` workers besides the calling thread (0: the caller copies alone).
  explicit HostCopyPool(int threads);
  ~HostCopyPool();
  HostCopyPool(const HostCopyPool&) = delete;
  HostCopyPool& operator=(const HostCopyPool&) = delete;

  // Copies every segment (segments do not overlap one another). Segments are
  // split into pieces of at most 4 MiB that the workers and the caller take
  // from a shared counter; many small pieces are taken four at a time, the
  // next one prefetched while the current one is copied. Copies of at least
  // 4 KiB use streaming stores. Returns when every byte is in place and
  // globally visible. Calls from several threads run one after another.
  void Copy(const std::vector<Segment>& segs);

  int threads() const { return static_cast<int>(workers_.size()); }

 private:
  void Drain(const std::vector<Segment>* p);
  void Work();

  std::mutex call_mu_;  // one batch at a time
  std::vector<std::thread> workers_;
  std::mutex mu_;
  std::condition_variable cv_, done_cv_;
  const std::vector<Segment>* batch_ = nullptr;
  std::atomic<size_t> next_{0};
  size_t left_ = 0;
  int active_ = 0;  // workers inside Drain of the current batch
  uint64_t generation_ = 0;
  bool stop_ = false;
};

}  // namespace kvx

#endif  // KVX_HOST_HOST_COPY_POOL_H_
