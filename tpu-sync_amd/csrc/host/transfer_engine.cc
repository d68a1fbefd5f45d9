#include "transfer_engine.h"

#include <algorithm>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <cstring>
#include <numeric>
#include <thread>

#include "../kernels/block_copy.h"
#include "../kernels/strided_copy.h"
#include "hip_util.h"
#include "host_copy_pool.h"

namespace kvx {
namespace {

constexpr int64_t kArgAlign = 256;

int64_t AlignUp(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

// Capacity of chunk `index` of a copy planned on a bounce lane, with `left`
// bytes not yet planned. The first chunk's host fill (H2D) comes before any
// DMA and the last chunk's host copy (D2H) after the last one, so chunks
// grow from cap/8 to cap over the first three and take at most half of what
// is left towards the end (down to cap/8).
int64_t LaneChunkCap(int64_t cap, size_t index, int64_t left) {
  int64_t c = index < 3 ? cap >> (3 - index) : cap;
  c = std::min(c, std::max(cap / 8, (left + 1) / 2));
  return std::max<int64_t>(c, 1);
}

// A run of compact indices whose host ids are consecutive.
struct HostRun {
  int64_t i0;
  int64_t len;
  int64_t host0;
};

// One piece of a staging chunk: flat blocks [f0, f0 + nb) of one group,
// placed at byte offset buf_off of the chunk buffer.
struct PiecePlan {
  int group;
  int64_t f0;
  int64_t nb;
  int64_t buf_off;
};

}  // namespace

StatusOr<StagingLayout> DeviceStagingLayout(const std::vector<int64_t>& block_bytes, int64_t n,
                                            bool block_major) {
  if (n < 0) return InvalidArgumentError("negative block count");
  const size_t S = block_bytes.size();
  StagingLayout out;
  out.base.assign(S, 0);
  out.stride_k.assign(S, 0);
  if (block_major) {
    for (size_t s = 1; s < S; ++s) {
      if (block_bytes[s] != block_bytes[0]) {
        return InvalidArgumentError("block-major staging needs one block size");
      }
    }
    const int64_t B = S > 0 ? block_bytes[0] : 0;
    for (size_t s = 0; s < S; ++s) {
      out.base[s] = static_cast<int64_t>(s) * B;
      out.stride_k[s] = static_cast<int64_t>(S) * B;
    }
    out.total_bytes = static_cast<int64_t>(S) * B * n;
    return out;
  }
  // Groups of equal block size in first-appearance order (as MakeGroups).
  std::vector<int64_t> sizes;
  std::vector<std::vector<size_t>> members;
  for (size_t s = 0; s < S; ++s) {
    size_t g = 0;
    while (g < sizes.size() && sizes[g] != block_bytes[s]) ++g;
    if (g == sizes.size()) {
      sizes.push_back(block_bytes[s]);
      members.emplace_back();
    }
    members[g].push_back(s);
  }
  int64_t off = 0;
  for (size_t g = 0; g < sizes.size(); ++g) {
    for (size_t m = 0; m < members[g].size(); ++m) {
      out.base[members[g][m]] = off + static_cast<int64_t>(m) * n * sizes[g];
      out.stride_k[members[g][m]] = sizes[g];
    }
    off += static_cast<int64_t>(members[g].size()) * n * sizes[g];
  }
  out.total_bytes = off;
  return out;
}

// Pinned bounce buffers of a pageable lane (one per staging-ring slot) and
// the host threads that move bytes between them and pageable host memory.
struct TransferEngine::Bounce {
  using Segment = HostCopyPool::Segment;
  std::vector<uint8_t*> bufs;
  std::vector<hipEvent_t> dma_done;  // last DMA into (D2H) or out of (H2D) bufs[k]
  // With fixed SDMA engines (sdma != null) the DMAs are ROCr copies and
  // dma_sig[k] stands in for dma_done[k].
  const SdmaEngines* sdma = nullptr;
  std::vector<hsa_signal_t> dma_sig;
  // The slot's last DMA was a stream-ordered hipMemcpyAsync recorded in
  // dma_done[k] even with SDMA engines (the last chunk of an H2D copy).
  std::vector<bool> event_dma;
  std::vector<bool> used;
  std::vector<std::vector<Segment>> owed;  // D2H: host copies still due from bufs[k]
  std::vector<std::vector<CopyFuture>> waiters;  // D2H: copies complete once bufs[k] drains
  std::deque<size_t> order;                // D2H: slots with copies owed, oldest first
  HostCopyPool pool;                       // the lane's host copy threads

  explicit Bounce(int threads) : pool(threads) {}
  ~Bounce() {
    WaitAllDma();
    for (hsa_signal_t s : dma_sig) SdmaEngines::DestroySignal(s);
    for (uint8_t* b : bufs) (void)hipHostFree(b);
    for (hipEvent_t e : dma_done) (void)hipEventDestroy(e);
  }

  Status WaitDma(size_t k) {
    if (sdma != nullptr && !event_dma[k]) return SdmaEngines::Wait(dma_sig[k]);
    return HipStatus(hipEventSynchronize(dma_done[k]), "bounce buffer DMA");
  }
  // Waits for every DMA still in flight (SDMA copies are on no stream, so a
  // stream synchronisation does not cover them).
  void WaitAllDma() {
    for (size_t k = 0; k < dma_sig.size(); ++k) {
      if (event_dma[k]) {
        (void)hipEventSynchronize(dma_done[k]);
      } else {
        (void)SdmaEngines::Wait(dma_sig[k]);
      }
    }
  }
  // Moves the segments' bytes with the pool and the calling thread.
  void Copy(const std::vector<Segment>& segs) { pool.Copy(segs); }

  // D2H: waits for the oldest slot's DMA, moves its bytes into place and
  // completes the copies waiting on it.
  Status DrainOldest() {
    const size_t k = order.front();
    order.pop_front();
    Status st = WaitDma(k);
    if (st.ok()) Copy(owed[k]);
    owed[k].clear();
    used[k] = false;
    for (const CopyFuture& f : waiters[k]) {
      if (st.ok()) {
        f.Fulfill(CopyFuture());
      } else {
        f.Reject(st);
      }
    }
    waiters[k].clear();
    return st;
  }
  Status DrainAll() {
    Status first = OkStatus();
    while (!order.empty()) {
      Status st = DrainOldest();
      if (first.ok() && !st.ok()) first = st;
    }
    return first;
  }
};

// One direction of pageable-host copies: a worker thread runs queued copies
// in order on the lane's own streams, staging ring, argument ring and bounce
// buffers, so a save and a load through /dev/shm overlap.
struct TransferEngine::PageableLane {
  struct Job {
    Direction dir;
    std::vector<StorageView> storages;
    std::vector<int64_t> cdev, chost;
    std::vector<ByteExtent> extents;  // non-empty: a pool-extent copy
    hipEvent_t dep_event = nullptr;
    CopyFuture future;
  };
  std::thread worker;
  std::mutex mu;
  std::condition_variable cv, idle_cv;
  std::deque<Job> jobs;
  bool stop = false;
  bool running = false;
  hipStream_t ks = nullptr, cs = nullptr;
  Ring ring;
  ArgRing args;
  std::unique_ptr<Bounce> bounce;

  // Releases whatever was created (also after a failed set-up). The worker
  // has been joined; the owner's device is current.
  ~PageableLane() {
    for (hipStream_t s : {ks, cs}) {
      if (s != nullptr) (void)hipStreamSynchronize(s);
    }
    if (bounce) bounce->WaitAllDma();  // before the staging buffers go
    for (uint64_t b : ring.bufs) (void)hipFree(reinterpret_cast<void*>(b));
    for (hipEvent_t e : ring.ready) (void)hipEventDestroy(e);
    for (hipEvent_t e : ring.free) (void)hipEventDestroy(e);
    bounce.reset();
    for (hipStream_t s : {ks, cs}) {
      if (s != nullptr) (void)hipStreamDestroy(s);
    }
  }
};

TransferEngine::TransferEngine(const EngineOptions& opts) : opts_(opts) {}

StatusOr<std::unique_ptr<TransferEngine>> TransferEngine::Create(
    const EngineOptions& opts) {
  if (opts.staging_chunk_bytes <= 0 || opts.staging_chunks <= 0 ||
      opts.arg_ring_bytes <= 0) {
    return InvalidArgumentError("engine sizes must be positive");
  }
  std::unique_ptr<TransferEngine> e(new TransferEngine(opts));
  KVX_RETURN_IF_ERROR(e->Init());
  return e;
}

Status TransferEngine::Init() {
  DeviceGuard g(opts_.device);
  if (!g.ok()) return InvalidArgumentError("cannot select HIP device");
  KVX_RETURN_IF_ERROR(CreateStreamsOnDistinctQueuesChecked(
      {&gather_stream_, &d2h_stream_, &h2d_stream_, &scatter_stream_}, &placement_));
  return GrowArgRing(opts_.arg_ring_bytes);
}

Status TransferEngine::EnsureRing(Ring* r) {
  // Allocated on first use: a manager whose copies all go zero-copy or
  // through the pageable lanes never holds these chunks.
  if (!r->bufs.empty()) return OkStatus();
  for (int k = 0; k < opts_.staging_chunks; ++k) {
    void* p = nullptr;
    KVX_HIP_RETURN_IF_ERROR(hipMalloc(&p, opts_.staging_chunk_bytes));
    r->bufs.push_back(reinterpret_cast<uint64_t>(p));
    KVX_ASSIGN_OR_RETURN(hipEvent_t ready, NewEvent());
    KVX_ASSIGN_OR_RETURN(hipEvent_t free_ev, NewEvent());
    r->ready.push_back(ready);
    r->free.push_back(free_ev);
    r->used.push_back(false);
  }
  return OkStatus();
}

TransferEngine::~TransferEngine() {
  // Pageable lanes finish their queued copies, then release their memory.
  for (std::unique_ptr<PageableLane>& lane : lanes_) {
    if (!lane) continue;
    {
      std::lock_guard<std::mutex> l(lane->mu);
      lane->stop = true;
    }
    lane->cv.notify_all();
    lane->worker.join();
  }
  DeviceGuard g(opts_.device);
  for (std::unique_ptr<PageableLane>& lane : lanes_) lane.reset();
  for (hipStream_t s :
       {gather_stream_, d2h_stream_, h2d_stream_, scatter_stream_}) {
    if (s != nullptr) (void)hipStreamSynchronize(s);
  }
  for (ArgSlice& s : arg_inflight_) (void)hipEventDestroy(s.done);
  arg_inflight_.clear();
  for (std::deque<StagedInFlight>& q : staged_inflight_) {
    for (const StagedInFlight& s : q) (void)hipEventDestroy(s.done);
    q.clear();
  }
  for (hipEvent_t e : spare_events_) (void)hipEventDestroy(e);
  spare_events_.clear();
  extent_args_.reset();
  for (KernelSample& s : samples_) {
    (void)hipEventDestroy(s.start);
    (void)hipEventDestroy(s.stop);
  }
  samples_.clear();
  for (Ring* r : {&out_ring_, &in_ring_}) {
    for (uint64_t b : r->bufs) (void)hipFree(reinterpret_cast<void*>(b));
    for (hipEvent_t e : r->ready) (void)hipEventDestroy(e);
    for (hipEvent_t e : r->free) (void)hipEventDestroy(e);
  }
  if (arg_host_ != nullptr) (void)hipHostFree(arg_host_);
  if (arg_dev_ != 0) (void)hipFree(reinterpret_cast<void*>(arg_dev_));
  for (hipStream_t s :
       {gather_stream_, d2h_stream_, h2d_stream_, scatter_stream_}) {
    if (s != nullptr) (void)hipStreamDestroy(s);
  }
}

uint32_t TransferEngine::LaneDmaEngines() {
  std::lock_guard<std::mutex> l(lanes_mu_);
  if (!sdma_ || (!lanes_[0] && !lanes_[1])) return 0;
  return (sdma_->engine(/*d2h=*/true) << 16) | sdma_->engine(/*d2h=*/false);
}

EngineStats TransferEngine::stats() const {
  std::lock_guard<std::mutex> l(const_cast<std::mutex&>(mu_));
  return stats_;
}

Status TransferEngine::Synchronize() {
  {
    std::lock_guard<std::mutex> l(lanes_mu_);
    for (std::unique_ptr<PageableLane>& lane : lanes_) {
      if (!lane) continue;
      std::unique_lock<std::mutex> ll(lane->mu);
      lane->idle_cv.wait(ll, [&] { return lane->jobs.empty() && !lane->running; });
    }
  }
  DeviceGuard g(opts_.device);
  for (std::unique_ptr<PageableLane>& lane : lanes_) {
    if (!lane) continue;
    KVX_HIP_RETURN_IF_ERROR(hipStreamSynchronize(lane->ks));
    KVX_HIP_RETURN_IF_ERROR(hipStreamSynchronize(lane->cs));
  }
  for (hipStream_t s :
       {gather_stream_, d2h_stream_, h2d_stream_, scatter_stream_}) {
    KVX_HIP_RETURN_IF_ERROR(hipStreamSynchronize(s));
  }
  return OkStatus();
}

Status TransferEngine::LaunchCopy(const CopyLaunch& l, bool gather, int vec,
                                  hipStream_t stream) {
  KernelSample s;
  if (opts_.profile_kernels) {
    KVX_HIP_RETURN_IF_ERROR(hipEventCreate(&s.start));
    KVX_HIP_RETURN_IF_ERROR(hipEventCreate(&s.stop));
    KVX_HIP_RETURN_IF_ERROR(hipEventRecord(s.start, stream));
  }
  CopyLaunch cl = l;
  cl.gather_workgroups_per_cu = opts_.gather_workgroups_per_cu;
  KVX_HIP_RETURN_IF_ERROR(LaunchBlockCopy(
      cl, gather ? CopyDir::kGather : CopyDir::kScatter, vec, stream));
  ++stats_.kernel_launches;
  if (opts_.profile_kernels) {
    KVX_HIP_RETURN_IF_ERROR(hipEventRecord(s.stop, stream));
    for (int k = 0; k < l.npieces; ++k) {
      s.bytes += 2 * l.pieces[k].nblocks * l.pieces[k].block_bytes;
    }
    s.gather = gather;
    samples_.push_back(s);
  }
  return OkStatus();
}

StatusOr<KernelTimes> TransferEngine::ProfiledKernelTimes(bool gather,
                                                          bool reset) {
  std::lock_guard<std::mutex> l(mu_);
  KernelTimes t;
  for (const KernelSample& s : samples_) {
    if (s.gather != gather) continue;
    KVX_HIP_RETURN_IF_ERROR(hipEventSynchronize(s.stop));
    float ms = 0;
    KVX_HIP_RETURN_IF_ERROR(hipEventElapsedTime(&ms, s.start, s.stop));
    ++t.launches;
    t.total_ms += ms;
    t.bytes += s.bytes;
  }
  if (reset) {
    std::vector<KernelSample> keep;
    for (KernelSample& s : samples_) {
      if (s.gather == gather) {
        (void)hipEventDestroy(s.start);
        (void)hipEventDestroy(s.stop);
      } else {
        keep.push_back(s);
      }
    }
    samples_.swap(keep);
  }
  return t;
}

StatusOr<hipEvent_t> TransferEngine::NewEvent() {
  hipEvent_t e = nullptr;
  KVX_HIP_RETURN_IF_ERROR(hipEventCreateWithFlags(&e, hipEventDisableTiming));
  return e;
}

Status TransferEngine::GrowArgRing(int64_t bytes) {
  for (ArgSlice& s : arg_inflight_) {
    KVX_HIP_RETURN_IF_ERROR(hipEventSynchronize(s.done));
    (void)hipEventDestroy(s.done);
  }
  arg_inflight_.clear();
  if (arg_host_ != nullptr) (void)hipHostFree(arg_host_);
  if (arg_dev_ != 0) (void)hipFree(reinterpret_cast<void*>(arg_dev_));
  arg_host_ = nullptr;
  arg_dev_ = 0;
  const int64_t size = AlignUp(std::max(bytes, arg_bytes_ * 2), kArgAlign);
  void* h = nullptr;
  void* d = nullptr;
  KVX_HIP_RETURN_IF_ERROR(hipHostMalloc(&h, size, hipHostMallocDefault));
  KVX_HIP_RETURN_IF_ERROR(hipMalloc(&d, size));
  arg_host_ = static_cast<uint8_t*>(h);
  arg_dev_ = reinterpret_cast<uint64_t>(d);
  arg_bytes_ = size;
  arg_head_ = 0;
  return OkStatus();
}

StatusOr<int64_t> TransferEngine::ArgAlloc(int64_t bytes) {
  bytes = AlignUp(std::max<int64_t>(bytes, 1), kArgAlign);
  if (bytes > arg_bytes_) KVX_RETURN_IF_ERROR(GrowArgRing(bytes));
  int64_t start = arg_head_;
  if (start + bytes > arg_bytes_) start = 0;
  const int64_t end = start + bytes;
  // Retire finished slices; wait for any unfinished one that overlaps.
  for (auto it = arg_inflight_.begin(); it != arg_inflight_.end();) {
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
    it = arg_inflight_.erase(it);
  }
  arg_head_ = end;
  return start;
}

Status TransferEngine::ArgCommit(int64_t begin, int64_t end,
                                 hipStream_t stream) {
  KVX_ASSIGN_OR_RETURN(hipEvent_t ev, NewEvent());
  KVX_HIP_RETURN_IF_ERROR(hipEventRecord(ev, stream));
  arg_inflight_.push_back(ArgSlice{begin, end, ev});
  return OkStatus();
}

std::vector<TransferEngine::Group> TransferEngine::MakeGroups(
    const std::vector<StorageView>& s) {
  std::vector<Group> groups;
  for (size_t w = 0; w < s.size(); ++w) {
    const int64_t pool = s[w].block_bytes > 0 ? s[w].dev_bytes / s[w].block_bytes : 0;
    Group* g = nullptr;
    for (Group& c : groups) {
      if (c.block_bytes == s[w].block_bytes) g = &c;
    }
    if (g == nullptr) {
      groups.push_back(Group{});
      g = &groups.back();
      g->block_bytes = s[w].block_bytes;
      g->pool_blocks = pool;
    }
    g->pool_blocks = std::min(g->pool_blocks, pool);
    g->members.push_back(static_cast<int>(w));
  }
  return groups;
}

Status TransferEngine::WaitDep(hipStream_t dep, hipStream_t on) {
  if (dep == nullptr) return OkStatus();
  KVX_ASSIGN_OR_RETURN(hipEvent_t ev, NewEvent());
  Status st = HipStatus(hipEventRecord(ev, dep), "hipEventRecord(dep)");
  if (st.ok()) st = HipStatus(hipStreamWaitEvent(on, ev, 0), "hipStreamWaitEvent");
  (void)hipEventDestroy(ev);
  return st;
}

namespace {

int64_t NowUs() {
  return std::chrono::duration_cast<std::chrono::microseconds>(
             std::chrono::steady_clock::now().time_since_epoch())
      .count();
}

}  // namespace

bool TransferEngine::DuplexNow(Direction dir) {
  if (opts_.auto_duplex_window_us <= 0) return false;
  std::lock_guard<std::mutex> l(duplex_mu_);
  std::deque<CopyFuture>& other = recent_[1 - static_cast<int>(dir)];
  while (!other.empty() && other.front().IsReady()) other.pop_front();
  const int64_t now = NowUs();
  if (!other.empty()) last_duplex_us_ = now;
  return now - last_duplex_us_ < opts_.auto_duplex_window_us;
}

void TransferEngine::NoteIssued(Direction dir, const CopyFuture& f) {
  if (opts_.auto_duplex_window_us <= 0) return;
  std::lock_guard<std::mutex> l(duplex_mu_);
  std::deque<CopyFuture>& q = recent_[static_cast<int>(dir)];
  while (!q.empty() && q.front().IsReady()) q.pop_front();
  q.push_back(f);
  constexpr size_t kMaxRemembered = 256;
  if (q.size() > kMaxRemembered) q.pop_front();
}

StatusOr<CopyFuture> TransferEngine::Copy(
    Direction dir, const std::vector<StorageView>& storages,
    const std::vector<int64_t>& src, const std::vector<int64_t>& dst,
    const std::vector<int64_t>& sizes, hipStream_t dep) {
  if (opts_.mode != TransferMode::kAuto) {
    return CopyPath(dir, storages, src, dst, sizes, dep, /*duplex=*/false);
  }
  const bool duplex = DuplexNow(dir);
  StatusOr<CopyFuture> r = CopyPath(dir, storages, src, dst, sizes, dep, duplex);
  if (r.ok()) NoteIssued(dir, r.value());
  return r;
}

StatusOr<CopyFuture> TransferEngine::CopyPath(
    Direction dir, const std::vector<StorageView>& storages,
    const std::vector<int64_t>& src, const std::vector<int64_t>& dst,
    const std::vector<int64_t>& sizes, hipStream_t dep, bool duplex) {
  if (src.size() != dst.size() || src.size() != sizes.size()) {
    return InvalidArgumentError("src, dst and sizes must have the same length");
  }
  int64_t total = 0;
  int64_t min_run = INT64_MAX;
  for (int64_t s : sizes) {
    total += s;
    if (s > 0) min_run = std::min(min_run, s);
  }
  if (total == 0 || storages.empty()) return CopyFuture();
  int64_t min_block = INT64_MAX, max_block = 0;
  bool host_ok = true;
  for (const StorageView& s : storages) {
    min_block = std::min(min_block, s.block_bytes);
    max_block = std::max(max_block, s.block_bytes);
    host_ok = host_ok && s.host_kernel_access;
  }
  if (!host_ok && opts_.host_copy_threads > 0 && opts_.mode != TransferMode::kZeroCopy &&
      max_block <= opts_.staging_chunk_bytes) {
    // Pageable host memory: the runtime would bounce every run through its
    // own small pinned buffers one call at a time; the lane moves whole
    // staging chunks with one DMA each and spreads the host side over
    // several threads.
    std::vector<int64_t> cdev, chost;
    KVX_RETURN_IF_ERROR(PlanPairs(dir, src, dst, sizes, &cdev, &chost));
    return CopyPageable(dir, storages, cdev, chost, {}, dep);
  }
  if ((min_run != INT64_MAX && min_run * min_block >= opts_.direct_min_bytes) ||
      max_block > opts_.staging_chunk_bytes) {
    // Long runs, or blocks that do not fit a staging chunk: one DMA per run;
    // in auto mode, runs of a pinned mirror that average under
    // auto_direct_min_run_bytes with the other direction idle: one
    // zero-copy launch (see EngineOptions::auto_direct_min_run_bytes).
    if (opts_.mode == TransferMode::kAuto && host_ok && !duplex &&
        max_block <= (int64_t{1} << 32)) {
      int64_t runs = 0;
      for (int64_t s : sizes) runs += s > 0 ? 1 : 0;
      int64_t sum_block = 0;
      for (const StorageView& s : storages) sum_block += s.block_bytes;
      // Mean bytes of a (storage, run): total blocks x the sum of the
      // storages' block bytes over (runs x storages).
      const double mean_run = static_cast<double>(total) * static_cast<double>(sum_block) /
                              (static_cast<double>(runs) * static_cast<double>(storages.size()));
      if (mean_run < static_cast<double>(opts_.auto_direct_min_run_bytes)) {
        std::vector<int64_t> cdev, chost;
        KVX_RETURN_IF_ERROR(PlanPairs(dir, src, dst, sizes, &cdev, &chost));
        // One launch addresses fewer than 2^32 (block, storage) pairs.
        if (static_cast<uint64_t>(cdev.size()) * storages.size() <= UINT32_MAX) {
          return CopyZeroCopy(dir, storages, cdev, chost, dep);
        }
      }
    }
    return CopyDirect(dir, storages, src, dst, sizes, dep);
  }
  std::vector<int64_t> cdev, chost;
  KVX_RETURN_IF_ERROR(PlanPairs(dir, src, dst, sizes, &cdev, &chost));
  if (opts_.mode == TransferMode::kLanes && opts_.host_copy_threads > 0) {
    return CopyPageable(dir, storages, cdev, chost, {}, dep);
  }
  bool zero_copy = opts_.mode == TransferMode::kZeroCopy;
  if (opts_.mode == TransferMode::kAuto && host_ok) {
    // The staged path costs one hipMemcpyAsync per (storage, host run) and
    // lets SDMA carry H2D next to a D2H in flight; the zero-copy kernel costs
    // the same for any host layout. Short host runs go zero-copy.
    int64_t runs = 0;
    for (size_t i = 0; i < chost.size(); ++i) {
      if (i == 0 || chost[i] != chost[i - 1] + 1) ++runs;
    }
    zero_copy = static_cast<int64_t>(chost.size()) * max_block <
                opts_.auto_staged_min_run_bytes * runs;
  }
  if (opts_.mode == TransferMode::kAuto && opts_.host_copy_threads > 0) {
    // A copy of more than auto_lanes_min_chunks staging chunks goes through
    // the lanes, which issue one chunk at a time; so does a staged copy that
    // would leave more than that many staged chunks of its direction in
    // flight together with the copies before it.
    int64_t per_block = 0;  // bytes of one block over every storage
    for (const StorageView& s : storages) per_block += s.block_bytes;
    const int64_t n = static_cast<int64_t>(cdev.size());
    const int64_t chunk = opts_.staging_chunk_bytes;
    bool lanes = per_block > 0 && n > opts_.auto_lanes_min_chunks * chunk / per_block;
    // Short runs while both directions are at work: the lanes, in both
    // directions (see EngineOptions::auto_duplex_window_us).
    if (!lanes && zero_copy && duplex) lanes = true;
    if (!lanes && !zero_copy) {
      const int64_t own = (n * per_block + chunk - 1) / chunk;
      std::lock_guard<std::mutex> l(mu_);
      lanes = own + StagedChunksInFlightLocked(dir) > opts_.auto_lanes_min_chunks;
    }
    if (lanes) return CopyPageable(dir, storages, cdev, chost, {}, dep);
  }
  if (zero_copy) {
    if (!host_ok) {
      return FailedPreconditionError(
          "zero-copy transfers need a pinned host mirror the GPU can access");
    }
    return CopyZeroCopy(dir, storages, cdev, chost, dep);
  }
  return CopyStaged(dir, storages, cdev, chost, dep);
}

StatusOr<CopyFuture> TransferEngine::CopyDirect(
    Direction dir, const std::vector<StorageView>& storages,
    const std::vector<int64_t>& src, const std::vector<int64_t>& dst,
    const std::vector<int64_t>& sizes, hipStream_t dep) {
  std::lock_guard<std::mutex> l(mu_);
  DeviceGuard g(opts_.device);
  hipStream_t cs = dir == Direction::kD2H ? d2h_stream_ : h2d_stream_;
  KVX_RETURN_IF_ERROR(WaitDep(dep, cs));
  for (const StorageView& s : storages) {
    const int64_t B = s.block_bytes;
    for (size_t r = 0; r < sizes.size(); ++r) {
      if (sizes[r] == 0) continue;
      const size_t bytes = static_cast<size_t>(sizes[r] * B);
      if (dir == Direction::kD2H) {
        KVX_HIP_RETURN_IF_ERROR(hipMemcpyAsync(
            s.host + dst[r] * B, reinterpret_cast<void*>(s.dev + src[r] * B),
            bytes, hipMemcpyDeviceToHost, cs));
      } else {
        KVX_HIP_RETURN_IF_ERROR(hipMemcpyAsync(
            reinterpret_cast<void*>(s.dev + dst[r] * B), s.host + src[r] * B,
            bytes, hipMemcpyHostToDevice, cs));
      }
      ++stats_.memcpy_calls;
    }
  }
  KVX_ASSIGN_OR_RETURN(hipEvent_t done, NewEvent());
  KVX_HIP_RETURN_IF_ERROR(hipEventRecord(done, cs));
  ++stats_.direct_copies;
  return CopyFuture::FromEvents({done}, {});
}

StatusOr<CopyFuture> TransferEngine::CopyFull(
    Direction dir, const std::vector<StorageView>& storages,
    const std::vector<int64_t>& bytes, hipStream_t dep) {
  bool host_ok = true;
  for (const StorageView& s : storages) host_ok = host_ok && s.host_kernel_access;
  if (!host_ok && opts_.host_copy_threads > 0) {
    // Pageable host memory: each storage's leading bytes as one extent
    // through a bounce lane, one lane copy per distinct length.
    std::vector<CopyFuture> parts;
    std::vector<bool> taken(storages.size(), false);
    for (size_t w = 0; w < storages.size(); ++w) {
      if (taken[w] || bytes[w] == 0) continue;
      std::vector<StorageView> group;
      for (size_t v = w; v < storages.size(); ++v) {
        if (!taken[v] && bytes[v] == bytes[w]) {
          group.push_back(storages[v]);
          taken[v] = true;
        }
      }
      KVX_ASSIGN_OR_RETURN(CopyFuture f,
                           CopyPageable(dir, group, {}, {}, {ByteExtent{0, bytes[w]}}, dep));
      parts.push_back(f);
    }
    return CopyFuture::Join(parts);
  }
  std::lock_guard<std::mutex> l(mu_);
  DeviceGuard g(opts_.device);
  hipStream_t cs = dir == Direction::kD2H ? d2h_stream_ : h2d_stream_;
  KVX_RETURN_IF_ERROR(WaitDep(dep, cs));
  for (size_t w = 0; w < storages.size(); ++w) {
    const StorageView& s = storages[w];
    if (bytes[w] == 0) continue;
    if (dir == Direction::kD2H) {
      KVX_HIP_RETURN_IF_ERROR(hipMemcpyAsync(s.host,
                                             reinterpret_cast<void*>(s.dev),
                                             bytes[w], hipMemcpyDeviceToHost, cs));
    } else {
      KVX_HIP_RETURN_IF_ERROR(hipMemcpyAsync(reinterpret_cast<void*>(s.dev),
                                             s.host, bytes[w],
                                             hipMemcpyHostToDevice, cs));
    }
    ++stats_.memcpy_calls;
  }
  KVX_ASSIGN_OR_RETURN(hipEvent_t done, NewEvent());
  KVX_HIP_RETURN_IF_ERROR(hipEventRecord(done, cs));
  ++stats_.direct_copies;
  return CopyFuture::FromEvents({done}, {});
}

Status TransferEngine::PlanPairs(Direction dir, const std::vector<int64_t>& src,
                                 const std::vector<int64_t>& dst,
                                 const std::vector<int64_t>& sizes,
                                 std::vector<int64_t>* dev_ids,
                                 std::vector<int64_t>* host_ids) {
  const bool d2h = dir == Direction::kD2H;
  // Expand runs into (device id, host id) pairs.
  int64_t N = 0;
  for (int64_t s : sizes) N += s;
  std::vector<int64_t> dev_id(N), host_id(N);
  {
    int64_t k = 0;
    for (size_t r = 0; r < sizes.size(); ++r) {
      for (int64_t j = 0; j < sizes[r]; ++j, ++k) {
        dev_id[k] = d2h ? src[r] + j : dst[r] + j;
        host_id[k] = d2h ? dst[r] + j : src[r] + j;
      }
    }
  }
  // One writer per destination block: the last pair naming it wins, as when
  // the copies are issued in order.
  const std::vector<int64_t>& dest = d2h ? host_id : dev_id;
  std::vector<int64_t> order(N);
  std::iota(order.begin(), order.end(), 0);
  std::stable_sort(order.begin(), order.end(),
                   [&](int64_t a, int64_t b) { return dest[a] < dest[b]; });
  std::vector<int64_t> kept;
  kept.reserve(N);
  for (int64_t k = 0; k < N; ++k) {
    if (k + 1 < N && dest[order[k + 1]] == dest[order[k]]) continue;
    kept.push_back(order[k]);
  }
  // Compact order: by host id, so every host run is contiguous in staging.
  if (!d2h) {
    std::stable_sort(kept.begin(), kept.end(), [&](int64_t a, int64_t b) {
      return host_id[a] < host_id[b];
    });
  }
  const int64_t n = static_cast<int64_t>(kept.size());
  if (n > INT32_MAX) return InvalidArgumentError("too many blocks in one copy");
  dev_ids->resize(n);
  host_ids->resize(n);
  for (int64_t i = 0; i < n; ++i) {
    (*dev_ids)[i] = dev_id[kept[i]];
    (*host_ids)[i] = host_id[kept[i]];
  }
  return OkStatus();
}

StatusOr<CopyFuture> TransferEngine::CopyExtents(
    Direction dir, const std::vector<StorageView>& storages,
    const std::vector<ByteExtent>& extents, hipStream_t dep) {
  const bool d2h = dir == Direction::kD2H;
  bool kernel = opts_.mode != TransferMode::kStaged;
  bool any_short = false;
  int64_t total = 0;
  for (const ByteExtent& e : extents) {
    any_short |= e.bytes < opts_.direct_min_bytes;
    total += e.bytes;
  }
  bool host_ok = true;
  for (const StorageView& s : storages) host_ok = host_ok && s.host_kernel_access;
  if (total == 0 || storages.empty()) return CopyFuture();
  if ((!host_ok || opts_.mode == TransferMode::kLanes) && opts_.host_copy_threads > 0) {
    // Pageable host memory (or lanes mode): live bytes packed into staging
    // chunks and moved through a bounce lane.
    return CopyPageable(dir, storages, {}, {}, extents, dep);
  }
  kernel &= host_ok && any_short;
  std::lock_guard<std::mutex> l(mu_);
  DeviceGuard g(opts_.device);
  if (!kernel) {
    hipStream_t cs = d2h ? d2h_stream_ : h2d_stream_;
    KVX_RETURN_IF_ERROR(WaitDep(dep, cs));
    for (const StorageView& s : storages) {
      for (const ByteExtent& e : extents) {
        if (e.bytes == 0) continue;
        void* dev = reinterpret_cast<void*>(s.dev + static_cast<uint64_t>(e.offset));
        if (d2h) {
          KVX_HIP_RETURN_IF_ERROR(hipMemcpyAsync(s.host + e.offset, dev, e.bytes,
                                                 hipMemcpyDeviceToHost, cs));
        } else {
          KVX_HIP_RETURN_IF_ERROR(hipMemcpyAsync(dev, s.host + e.offset, e.bytes,
                                                 hipMemcpyHostToDevice, cs));
        }
        ++stats_.memcpy_calls;
      }
    }
    KVX_ASSIGN_OR_RETURN(hipEvent_t done, NewEvent());
    KVX_HIP_RETURN_IF_ERROR(hipEventRecord(done, cs));
    ++stats_.direct_copies;
    return CopyFuture::FromEvents({done}, {});
  }
  // One launch for every (storage, extent): the kernel moves the live bytes
  // between HBM and the mapped host region itself.
  std::vector<StridedCopy> copies;
  copies.reserve(storages.size() * extents.size());
  for (const StorageView& s : storages) {
    const uint64_t host = reinterpret_cast<uint64_t>(s.host);
    for (const ByteExtent& e : extents) {
      if (e.bytes == 0) continue;
      StridedCopy c;
      c.src = (d2h ? s.dev : host) + static_cast<uint64_t>(e.offset);
      c.dst = (d2h ? host : s.dev) + static_cast<uint64_t>(e.offset);
      c.size = e.bytes;
      copies.push_back(c);
    }
  }
  hipStream_t ks = d2h ? gather_stream_ : scatter_stream_;
  if (!extent_args_) {
    auto ring = std::make_unique<ArgRing>();
    KVX_RETURN_IF_ERROR(ring->Init(1 << 20));
    extent_args_ = std::move(ring);
  }
  KVX_RETURN_IF_ERROR(WaitDep(dep, ks));
  // PCIe-bound: a few dozen workgroups keep the link busy (see the
  // zero-copy caps).
  const int64_t cap = d2h ? opts_.zero_copy_d2h_workgroups : opts_.zero_copy_h2d_workgroups;
  KVX_RETURN_IF_ERROR(LaunchStridedThroughRing(*extent_args_, copies, ks,
                                               static_cast<uint32_t>(cap > 0 ? cap : 0)));
  KVX_ASSIGN_OR_RETURN(hipEvent_t done, NewEvent());
  KVX_HIP_RETURN_IF_ERROR(hipEventRecord(done, ks));
  ++stats_.kernel_launches;
  ++stats_.extent_kernel_copies;
  return CopyFuture::FromEvents({done}, {});
}

StatusOr<CopyFuture> TransferEngine::CopyZeroCopy(
    Direction dir, const std::vector<StorageView>& storages,
    const std::vector<int64_t>& cdev, const std::vector<int64_t>& chost,
    hipStream_t dep) {
  const bool d2h = dir == Direction::kD2H;
  const int64_t n = static_cast<int64_t>(cdev.size());
  std::vector<Group> groups = MakeGroups(storages);
  for (const Group& gr : groups) {
    if (static_cast<int64_t>(gr.members.size()) * n > UINT32_MAX) {
      return InvalidArgumentError("copy too large for one launch");
    }
  }
  std::lock_guard<std::mutex> l(mu_);
  DeviceGuard dg(opts_.device);
  hipStream_t ks = d2h ? gather_stream_ : scatter_stream_;
  // Arguments: device ids, host ids, then a device and a host base-address
  // table per group.
  int64_t arg_bytes = 2 * AlignUp(n * 8, kArgAlign);
  std::vector<int64_t> dev_tab(groups.size()), host_tab(groups.size());
  for (size_t gi = 0; gi < groups.size(); ++gi) {
    const int64_t tb = AlignUp(static_cast<int64_t>(groups[gi].members.size()) * 8, kArgAlign);
    dev_tab[gi] = arg_bytes;
    host_tab[gi] = arg_bytes + tb;
    arg_bytes += 2 * tb;
  }
  KVX_ASSIGN_OR_RETURN(int64_t aoff, ArgAlloc(arg_bytes));
  ArgSliceGuard keep([this, aoff, arg_bytes, ks] { return ArgCommit(aoff, aoff + arg_bytes, ks); },
                     ks);
  const int64_t ids2_off = AlignUp(n * 8, kArgAlign);
  std::memcpy(arg_host_ + aoff, cdev.data(), n * 8);
  std::memcpy(arg_host_ + aoff + ids2_off, chost.data(), n * 8);
  uint64_t acc = 0;
  std::vector<int64_t> other_blocks(groups.size(), INT64_MAX);
  for (size_t gi = 0; gi < groups.size(); ++gi) {
    uint64_t* dt = reinterpret_cast<uint64_t*>(arg_host_ + aoff + dev_tab[gi]);
    uint64_t* ht = reinterpret_cast<uint64_t*>(arg_host_ + aoff + host_tab[gi]);
    for (size_t m = 0; m < groups[gi].members.size(); ++m) {
      const StorageView& sv = storages[groups[gi].members[m]];
      dt[m] = sv.dev;
      ht[m] = reinterpret_cast<uint64_t>(sv.host);
      acc |= dt[m] | ht[m];
      other_blocks[gi] = std::min(other_blocks[gi], sv.host_bytes / sv.block_bytes);
    }
  }
  KVX_HIP_RETURN_IF_ERROR(hipMemcpyAsync(reinterpret_cast<void*>(arg_dev_ + aoff),
                                         arg_host_ + aoff, arg_bytes,
                                         hipMemcpyHostToDevice, ks));
  KVX_RETURN_IF_ERROR(WaitDep(dep, ks));
  for (size_t g0 = 0; g0 < groups.size(); g0 += kMaxPieces) {
    CopyLaunch cl;
    cl.ids = reinterpret_cast<const int64_t*>(arg_dev_ + aoff);
    cl.ids2 = reinterpret_cast<const int64_t*>(arg_dev_ + aoff + ids2_off);
    cl.n = n;
    cl.max_workgroups = d2h ? opts_.zero_copy_d2h_workgroups
                            : opts_.zero_copy_h2d_workgroups;
    for (size_t gi = g0; gi < groups.size() && gi < g0 + kMaxPieces; ++gi) {
      const Group& gr = groups[gi];
      CopyPiece& c = cl.pieces[cl.npieces++];
      c.storages = arg_dev_ + aoff + dev_tab[gi];
      c.others = arg_dev_ + aoff + host_tab[gi];
      c.other_blocks = other_blocks[gi];
      c.f0 = 0;
      c.nblocks = static_cast<int64_t>(gr.members.size()) * n;
      c.block_bytes = gr.block_bytes;
      c.pool_blocks = gr.pool_blocks;
    }
    const int vec = LaunchVectorBytes(cl, acc);
    KVX_RETURN_IF_ERROR(LaunchCopy(cl, d2h, vec, ks));
  }
  KVX_RETURN_IF_ERROR(keep.Commit());
  KVX_ASSIGN_OR_RETURN(hipEvent_t done, NewEvent());
  KVX_HIP_RETURN_IF_ERROR(hipEventRecord(done, ks));
  ++stats_.zero_copy_copies;
  return CopyFuture::FromEvents({done}, {});
}

StatusOr<CopyFuture> TransferEngine::CopyStaged(
    Direction dir, const std::vector<StorageView>& storages,
    const std::vector<int64_t>& cdev, const std::vector<int64_t>& chost,
    hipStream_t dep) {
  const bool d2h = dir == Direction::kD2H;
  std::lock_guard<std::mutex> l(mu_);
  DeviceGuard dg(opts_.device);
  LaneView lane;
  lane.ks = d2h ? gather_stream_ : scatter_stream_;
  lane.cs = d2h ? d2h_stream_ : h2d_stream_;
  lane.ring = d2h ? &out_ring_ : &in_ring_;
  KVX_RETURN_IF_ERROR(EnsureRing(lane.ring));
  hipEvent_t done = nullptr;
  const int64_t chunks_before = stats_.chunks;
  KVX_RETURN_IF_ERROR(StagedOnLane(lane, dir, storages, cdev, chost, dep, &done));
  ++stats_.staged_copies;
  // Track the chunks this copy keeps in flight (in auto mode Copy() keeps the
  // total bounded; see EngineOptions::auto_lanes_min_chunks). Finished copies
  // leave the list first, so it holds only copies still in flight. The copy
  // is already enqueued: if no event can be had it goes untracked rather than
  // failing.
  if (opts_.mode != TransferMode::kAuto) return CopyFuture::FromEvents({done}, {});
  (void)StagedChunksInFlightLocked(dir);
  hipEvent_t track = nullptr;
  if (!spare_events_.empty()) {
    track = spare_events_.back();
    spare_events_.pop_back();
  } else {
    StatusOr<hipEvent_t> e = NewEvent();
    if (e.ok()) track = e.value();
  }
  if (track != nullptr) {
    if (hipEventRecord(track, d2h ? lane.cs : lane.ks) == hipSuccess) {
      staged_inflight_[static_cast<int>(dir)].push_back(
          StagedInFlight{track, stats_.chunks - chunks_before});
    } else {
      (void)hipEventDestroy(track);
    }
  }
  return CopyFuture::FromEvents({done}, {});
}

int64_t TransferEngine::StagedChunksInFlightLocked(Direction dir) {
  std::deque<StagedInFlight>& q = staged_inflight_[static_cast<int>(dir)];
  // Copies finish in order on their streams: drop finished ones from the
  // front.
  while (!q.empty() && hipEventQuery(q.front().done) == hipSuccess) {
    spare_events_.push_back(q.front().done);
    q.pop_front();
  }
  int64_t chunks = 0;
  for (const StagedInFlight& s : q) chunks += s.chunks;
  return chunks;
}

Status TransferEngine::PipelineBounceSdma(const LaneView& lane, Direction dir,
                                          const std::vector<ChunkWork>& chunks,
                                          int64_t* memcpys) {
  const bool d2h = dir == Direction::kD2H;
  Ring& ring = *lane.ring;
  Bounce* b = lane.bounce;
  const SdmaEngines& dma = *b->sdma;
  // The host orders each DMA against the lane's kernels, since a ROCr copy
  // waits on no stream: a D2H chunk's DMA starts once its gather has run; an
  // H2D chunk's scatter is launched once its DMA has landed, one chunk
  // later, so the next chunk's host fill and DMA overlap that wait.
  auto segments = [&](const ChunkWork& ch, uint8_t* bb, std::vector<Bounce::Segment>* out) {
    for (const HostSegment& s : ch.segs) {
      const size_t bytes = static_cast<size_t>(s.bytes);
      if (d2h) {
        out->push_back(Bounce::Segment{s.host, bb + s.off, bytes});
      } else {
        out->push_back(Bounce::Segment{bb + s.off, s.host, bytes});
      }
    }
  };
  if (d2h) {
    for (const ChunkWork& ch : chunks) {
      const size_t k = ring.next;
      ring.next = (ring.next + 1) % ring.bufs.size();
      const uint64_t buf = ring.bufs[k];
      // Staging slot k is free once bounce slot k has drained: its last DMA
      // read the staging buffer.
      while (b->used[k]) KVX_RETURN_IF_ERROR(b->DrainOldest());
      KVX_RETURN_IF_ERROR(ch.kernel(buf));
      KVX_HIP_RETURN_IF_ERROR(hipEventRecord(ring.ready[k], lane.ks));
      KVX_HIP_RETURN_IF_ERROR(hipEventSynchronize(ring.ready[k]));
      KVX_RETURN_IF_ERROR(dma.Start(/*d2h=*/true, b->bufs[k], reinterpret_cast<void*>(buf),
                                    static_cast<size_t>(ch.bytes), b->dma_sig[k]));
      ++*memcpys;
      segments(ch, b->bufs[k], &b->owed[k]);
      b->used[k] = true;
      b->order.push_back(k);
      ring.used[k] = true;
    }
    return OkStatus();
  }
  // H2D. On an error return no DMA of this call may still be in flight: the
  // next call refills the bounce buffers.
  struct DrainOnError {
    Bounce* b;
    bool armed = true;
    ~DrainOnError() {
      if (armed) b->WaitAllDma();
    }
  } guard{b};
  const ChunkWork* prev = nullptr;
  size_t prev_k = 0;
  auto scatter = [&](const ChunkWork& ch, size_t j) -> Status {
    KVX_RETURN_IF_ERROR(b->WaitDma(j));
    KVX_RETURN_IF_ERROR(ch.kernel(ring.bufs[j]));
    KVX_HIP_RETURN_IF_ERROR(hipEventRecord(ring.free[j], lane.ks));
    return OkStatus();
  };
  for (const ChunkWork& ch : chunks) {
    const size_t k = ring.next;
    ring.next = (ring.next + 1) % ring.bufs.size();
    if (prev != nullptr && prev_k == k) {
      // A one-slot ring: the previous chunk still owns this slot, so its
      // scatter goes first (after its DMA has landed), and the wait below
      // then covers that scatter before the slot is refilled.
      KVX_RETURN_IF_ERROR(scatter(*prev, prev_k));
      prev = nullptr;
    }
    // The slot's last scatter has read the staging buffer (its DMA landed
    // before that scatter was launched).
    if (ring.used[k]) KVX_HIP_RETURN_IF_ERROR(hipEventSynchronize(ring.free[k]));
    std::vector<Bounce::Segment> segs;
    segments(ch, b->bufs[k], &segs);
    b->Copy(segs);
    const bool last = &ch == &chunks.back();
    if (last) {
      // The last chunk crosses on the lane's copy stream and its scatter
      // follows on the kernel stream, so this thread need not wait for it:
      // the next copy's first host fill and DMA overlap this one's end.
      KVX_HIP_RETURN_IF_ERROR(hipMemcpyAsync(reinterpret_cast<void*>(ring.bufs[k]), b->bufs[k],
                                             static_cast<size_t>(ch.bytes),
                                             hipMemcpyHostToDevice, lane.cs));
      KVX_HIP_RETURN_IF_ERROR(hipEventRecord(b->dma_done[k], lane.cs));
      b->event_dma[k] = true;
    } else {
      KVX_RETURN_IF_ERROR(dma.Start(/*d2h=*/false, reinterpret_cast<void*>(ring.bufs[k]),
                                    b->bufs[k], static_cast<size_t>(ch.bytes), b->dma_sig[k]));
      b->event_dma[k] = false;
    }
    ++*memcpys;
    b->used[k] = true;
    ring.used[k] = true;
    if (prev != nullptr) KVX_RETURN_IF_ERROR(scatter(*prev, prev_k));
    prev = &ch;
    prev_k = k;
  }
  if (prev != nullptr) {
    KVX_HIP_RETURN_IF_ERROR(hipStreamWaitEvent(lane.ks, b->dma_done[prev_k], 0));
    KVX_RETURN_IF_ERROR(prev->kernel(ring.bufs[prev_k]));
    KVX_HIP_RETURN_IF_ERROR(hipEventRecord(ring.free[prev_k], lane.ks));
  }
  guard.armed = false;
  return OkStatus();
}

Status TransferEngine::PipelineChunks(const LaneView& lane, Direction dir,
                                      const std::vector<ChunkWork>& chunks, int64_t* memcpys) {
  if (lane.bounce != nullptr && lane.bounce->sdma != nullptr) {
    return PipelineBounceSdma(lane, dir, chunks, memcpys);
  }
  const bool d2h = dir == Direction::kD2H;
  hipStream_t ks = lane.ks;
  hipStream_t cs = lane.cs;
  Ring& ring = *lane.ring;
  Bounce* bounce = lane.bounce;

  // Pinned host: one DMA per segment straight between staging and host.
  auto issue_memcpys = [&](const ChunkWork& ch, uint64_t buf) -> Status {
    for (const HostSegment& s : ch.segs) {
      void* stg = reinterpret_cast<void*>(buf + static_cast<uint64_t>(s.off));
      const size_t bytes = static_cast<size_t>(s.bytes);
      if (d2h) {
        KVX_HIP_RETURN_IF_ERROR(hipMemcpyAsync(s.host, stg, bytes, hipMemcpyDeviceToHost, cs));
      } else {
        KVX_HIP_RETURN_IF_ERROR(hipMemcpyAsync(stg, s.host, bytes, hipMemcpyHostToDevice, cs));
      }
      ++*memcpys;
    }
    return OkStatus();
  };
  // Host copies between pageable host memory and bounce buffer `bb`.
  auto bounce_segments = [&](const ChunkWork& ch, uint8_t* bb,
                             std::vector<Bounce::Segment>* out) {
    for (const HostSegment& s : ch.segs) {
      const size_t bytes = static_cast<size_t>(s.bytes);
      if (d2h) {
        out->push_back(Bounce::Segment{s.host, bb + s.off, bytes});
      } else {
        out->push_back(Bounce::Segment{bb + s.off, s.host, bytes});
      }
    }
  };
  for (const ChunkWork& ch : chunks) {
    const size_t k = ring.next;
    ring.next = (ring.next + 1) % ring.bufs.size();
    const uint64_t buf = ring.bufs[k];
    if (d2h) {
      if (ring.used[k]) KVX_HIP_RETURN_IF_ERROR(hipStreamWaitEvent(ks, ring.free[k], 0));
      KVX_RETURN_IF_ERROR(ch.kernel(buf));
      KVX_HIP_RETURN_IF_ERROR(hipEventRecord(ring.ready[k], ks));
      KVX_HIP_RETURN_IF_ERROR(hipStreamWaitEvent(cs, ring.ready[k], 0));
      if (bounce != nullptr) {
        // One DMA of the whole chunk into pinned memory; host threads move
        // the segments into place once it lands (a few chunks later).
        while (bounce->used[k]) KVX_RETURN_IF_ERROR(bounce->DrainOldest());
        KVX_HIP_RETURN_IF_ERROR(hipMemcpyAsync(bounce->bufs[k], reinterpret_cast<void*>(buf),
                                               static_cast<size_t>(ch.bytes),
                                               hipMemcpyDeviceToHost, cs));
        KVX_HIP_RETURN_IF_ERROR(hipEventRecord(bounce->dma_done[k], cs));
        ++*memcpys;
        bounce_segments(ch, bounce->bufs[k], &bounce->owed[k]);
        bounce->used[k] = true;
        bounce->order.push_back(k);
      } else {
        KVX_RETURN_IF_ERROR(issue_memcpys(ch, buf));
      }
      KVX_HIP_RETURN_IF_ERROR(hipEventRecord(ring.free[k], cs));
    } else {
      if (bounce != nullptr) {
        // Host threads fill the pinned slot (once its last DMA is done),
        // then one DMA moves the whole chunk.
        if (bounce->used[k]) KVX_HIP_RETURN_IF_ERROR(hipEventSynchronize(bounce->dma_done[k]));
        std::vector<Bounce::Segment> segs;
        bounce_segments(ch, bounce->bufs[k], &segs);
        bounce->Copy(segs);
      }
      if (ring.used[k]) KVX_HIP_RETURN_IF_ERROR(hipStreamWaitEvent(cs, ring.free[k], 0));
      if (bounce != nullptr) {
        KVX_HIP_RETURN_IF_ERROR(hipMemcpyAsync(reinterpret_cast<void*>(buf), bounce->bufs[k],
                                               static_cast<size_t>(ch.bytes),
                                               hipMemcpyHostToDevice, cs));
        KVX_HIP_RETURN_IF_ERROR(hipEventRecord(bounce->dma_done[k], cs));
        ++*memcpys;
        bounce->used[k] = true;
      } else {
        KVX_RETURN_IF_ERROR(issue_memcpys(ch, buf));
      }
      KVX_HIP_RETURN_IF_ERROR(hipEventRecord(ring.ready[k], cs));
      KVX_HIP_RETURN_IF_ERROR(hipStreamWaitEvent(ks, ring.ready[k], 0));
      KVX_RETURN_IF_ERROR(ch.kernel(buf));
      KVX_HIP_RETURN_IF_ERROR(hipEventRecord(ring.free[k], ks));
    }
    ring.used[k] = true;
  }
  return OkStatus();
}

Status TransferEngine::StagedOnLane(const LaneView& lane, Direction dir,
                                    const std::vector<StorageView>& storages,
                                    const std::vector<int64_t>& cdev,
                                    const std::vector<int64_t>& chost, hipStream_t dep,
                                    hipEvent_t* done) {
  const bool d2h = dir == Direction::kD2H;
  const int64_t n = static_cast<int64_t>(cdev.size());
  std::vector<HostRun> runs;
  for (int64_t i = 0; i < n;) {
    int64_t e = i + 1;
    while (e < n && chost[e] == chost[e - 1] + 1) ++e;
    runs.push_back(HostRun{i, e - i, chost[i]});
    i = e;
  }
  if (n > INT32_MAX) return InvalidArgumentError("too many blocks in one copy");

  std::vector<Group> groups = MakeGroups(storages);
  for (const Group& gr : groups) {
    if (gr.block_bytes > opts_.staging_chunk_bytes) {
      return InvalidArgumentError("block larger than a staging chunk");
    }
    if (static_cast<int64_t>(gr.members.size()) * n > UINT32_MAX) {
      return InvalidArgumentError("copy too large for one plan");
    }
  }
  hipStream_t ks = lane.ks;
  hipStream_t cs = lane.cs;

  // Counters, folded into stats_ at the end (under mu_ for a pageable lane).
  int64_t memcpys = 0, launches = 0;

  // Arguments: compact device ids, then one base-address table per group.
  int64_t arg_bytes = AlignUp(n * 8, kArgAlign);
  std::vector<int64_t> table_off(groups.size());
  for (size_t gi = 0; gi < groups.size(); ++gi) {
    table_off[gi] = arg_bytes;
    arg_bytes += AlignUp(static_cast<int64_t>(groups[gi].members.size()) * 8, kArgAlign);
  }
  int64_t aoff = 0;
  uint8_t* arg_host = nullptr;
  uint64_t arg_dev = 0;
  if (lane.args != nullptr) {
    KVX_ASSIGN_OR_RETURN(aoff, lane.args->Alloc(arg_bytes));
    arg_host = lane.args->host(aoff);
    arg_dev = lane.args->dev(aoff);
  } else {
    KVX_ASSIGN_OR_RETURN(aoff, ArgAlloc(arg_bytes));
    arg_host = arg_host_ + aoff;
    arg_dev = arg_dev_ + aoff;
  }
  ArgSliceGuard keep(
      [this, &lane, aoff, arg_bytes, ks] {
        return lane.args != nullptr ? lane.args->Commit(aoff, arg_bytes, ks)
                                    : ArgCommit(aoff, aoff + arg_bytes, ks);
      },
      ks);
  std::memcpy(arg_host, cdev.data(), n * 8);
  uint64_t align_acc = 0;
  for (size_t gi = 0; gi < groups.size(); ++gi) {
    uint64_t* t = reinterpret_cast<uint64_t*>(arg_host + table_off[gi]);
    for (size_t m = 0; m < groups[gi].members.size(); ++m) {
      t[m] = storages[groups[gi].members[m]].dev;
      align_acc |= t[m];
    }
    groups[gi].table_dev = arg_dev + table_off[gi];
  }
  if (lane.args != nullptr) {
    KVX_RETURN_IF_ERROR(lane.args->Upload(aoff, arg_bytes, ks));
  } else {
    KVX_HIP_RETURN_IF_ERROR(hipMemcpyAsync(reinterpret_cast<void*>(arg_dev), arg_host,
                                           arg_bytes, hipMemcpyHostToDevice, ks));
  }
  KVX_RETURN_IF_ERROR(WaitDep(dep, ks));
  const int64_t* ids_dev = reinterpret_cast<const int64_t*>(arg_dev);

  // Chunk plan over the layer-major staging layout of all groups.
  const int64_t cap = opts_.staging_chunk_bytes;
  // A bounce lane ramps its chunks (LaneChunkCap); stream-ordered copies
  // keep full ones, their kernels being short next to a chunk's DMA.
  const bool ramp = lane.bounce != nullptr;
  int64_t left = 0;  // bytes not yet planned
  for (const Group& gr : groups) {
    left += static_cast<int64_t>(gr.members.size()) * n * gr.block_bytes;
  }
  auto chunk_cap = [&](size_t index) -> int64_t {
    return ramp ? LaneChunkCap(cap, index, left) : cap;
  };
  std::vector<std::vector<PiecePlan>> plans;
  {
    std::vector<PiecePlan> cur;
    int64_t used = 0;
    int64_t cur_cap = chunk_cap(0);
    for (size_t gi = 0; gi < groups.size(); ++gi) {
      const int64_t B = groups[gi].block_bytes;
      const int64_t F = static_cast<int64_t>(groups[gi].members.size()) * n;
      int64_t f = 0;
      while (f < F) {
        int64_t fit = (cur_cap - used) / B;
        // A chunk holds at least one block (B <= cap: the ring's buffers).
        if (fit == 0 && used == 0) fit = 1;
        if (fit == 0) {
          plans.push_back(std::move(cur));
          cur.clear();
          left -= used;
          used = 0;
          cur_cap = chunk_cap(plans.size());
          continue;
        }
        const int64_t take = std::min(fit, F - f);
        cur.push_back(PiecePlan{static_cast<int>(gi), f, take, used});
        used += take * B;
        f += take;
      }
    }
    if (!cur.empty()) plans.push_back(std::move(cur));
  }

  // Host-run segments of piece p: (host pointer, offset in the chunk, bytes).
  auto add_segments = [&](const PiecePlan& p, std::vector<HostSegment>* out) {
    const Group& gr = groups[p.group];
    const int64_t B = gr.block_bytes;
    const int64_t wlo = p.f0 / n;
    const int64_t whi = (p.f0 + p.nb - 1) / n;
    for (int64_t w = wlo; w <= whi; ++w) {
      const StorageView& s = storages[gr.members[w]];
      const int64_t ilo = std::max<int64_t>(p.f0 - w * n, 0);
      const int64_t ihi = std::min<int64_t>(p.f0 + p.nb - w * n, n);
      // First run that ends after ilo.
      auto it = std::upper_bound(runs.begin(), runs.end(), ilo,
                                 [](int64_t v, const HostRun& r) { return v < r.i0; });
      if (it != runs.begin()) --it;
      for (; it != runs.end() && it->i0 < ihi; ++it) {
        const int64_t a = std::max(it->i0, ilo);
        const int64_t b = std::min(it->i0 + it->len, ihi);
        if (a >= b) continue;
        out->push_back(HostSegment{s.host + (it->host0 + (a - it->i0)) * B,
                                   p.buf_off + (w * n + a - p.f0) * B, (b - a) * B});
      }
    }
  };

  auto launch = [&](const std::vector<PiecePlan>& ps, uint64_t buf) -> Status {
    for (size_t p0 = 0; p0 < ps.size(); p0 += kMaxPieces) {
      CopyLaunch cl;
      cl.ids = ids_dev;
      cl.n = n;
      uint64_t acc = align_acc | buf;
      for (size_t k = p0; k < ps.size() && k < p0 + kMaxPieces; ++k) {
        const PiecePlan& p = ps[k];
        const Group& gr = groups[p.group];
        CopyPiece& c = cl.pieces[cl.npieces++];
        c.storages = gr.table_dev;
        c.staging = buf + static_cast<uint64_t>(p.buf_off) -
                    static_cast<uint64_t>(p.f0) * static_cast<uint64_t>(gr.block_bytes);
        c.stride_w = n * gr.block_bytes;
        c.stride_i = gr.block_bytes;
        c.f0 = p.f0;
        c.nblocks = p.nb;
        c.block_bytes = gr.block_bytes;
        c.pool_blocks = gr.pool_blocks;
        acc |= static_cast<uint64_t>(p.buf_off);
      }
      const int vec = LaunchVectorBytes(cl, acc);
      if (lane.args != nullptr) {
        // A pageable lane runs outside mu_: launch without profiling samples.
        KVX_HIP_RETURN_IF_ERROR(LaunchBlockCopy(
            cl, d2h ? CopyDir::kGather : CopyDir::kScatter, vec, ks));
        ++launches;
      } else {
        KVX_RETURN_IF_ERROR(LaunchCopy(cl, d2h, vec, ks));
      }
    }
    return OkStatus();
  };

  std::vector<ChunkWork> chunks(plans.size());
  for (size_t k = 0; k < plans.size(); ++k) {
    ChunkWork& ch = chunks[k];
    for (const PiecePlan& p : plans[k]) {
      ch.bytes = std::max(ch.bytes, p.buf_off + p.nb * groups[p.group].block_bytes);
      add_segments(p, &ch.segs);
    }
    const std::vector<PiecePlan>* plan = &plans[k];
    ch.kernel = [&launch, plan](uint64_t buf) { return launch(*plan, buf); };
  }
  KVX_RETURN_IF_ERROR(PipelineChunks(lane, dir, chunks, &memcpys));

  const int64_t nchunks = static_cast<int64_t>(chunks.size());
  KVX_RETURN_IF_ERROR(keep.Commit());
  if (lane.args != nullptr) {
    std::lock_guard<std::mutex> l(mu_);
    stats_.memcpy_calls += memcpys;
    stats_.chunks += nchunks;
    stats_.kernel_launches += launches;
  } else {
    stats_.memcpy_calls += memcpys;
    stats_.chunks += nchunks;
  }
  if (d2h && lane.bounce != nullptr) {
    *done = nullptr;  // complete once its bounce slots drain
    return OkStatus();
  }
  KVX_ASSIGN_OR_RETURN(*done, NewEvent());
  KVX_HIP_RETURN_IF_ERROR(hipEventRecord(*done, d2h ? cs : ks));
  return OkStatus();
}

Status TransferEngine::ExtentsOnLane(const LaneView& lane, Direction dir,
                                     const std::vector<StorageView>& storages,
                                     const std::vector<ByteExtent>& extents, hipEvent_t* done) {
  const bool d2h = dir == Direction::kD2H;
  // Pieces start at 16-byte offsets, so a chunk holds at most the largest
  // multiple of 16 that fits the staging and bounce buffers.
  const int64_t cap = opts_.staging_chunk_bytes / 16 * 16;
  if (cap == 0) {
    return InvalidArgumentError("pool extents through a lane need staging chunks of 16 bytes or more");
  }
  // Every (storage, extent) piece packed into staging chunks at 16-byte
  // aligned offsets, split where a chunk fills. The strided kernel packs
  // (D2H) or unpacks (H2D) a chunk; staging offsets are relative until the
  // chunk's buffer is known.
  std::vector<ChunkWork> chunks;
  std::vector<std::vector<StridedCopy>> tables;
  ChunkWork cur;
  std::vector<StridedCopy> tab;
  int64_t used = 0;
  // H2D ramps its chunks (LaneChunkCap): a pool copy is often one chunk,
  // whose host fill would otherwise come whole before its DMA (a 16 MiB
  // pool load 31.8 -> 37.7 GB/s). D2H keeps full chunks: its host copies
  // already overlap the next copy's DMA, and the extra chunks cost it
  // (53.7 -> 48.2 GB/s).
  int64_t unplanned = 0;  // bytes not yet planned
  for (const ByteExtent& e : extents) unplanned += e.bytes;
  unplanned *= static_cast<int64_t>(storages.size());
  auto chunk_cap = [&](size_t index) -> int64_t {
    return d2h ? cap : LaneChunkCap(cap, index, unplanned);
  };
  int64_t cur_cap = chunk_cap(0);
  auto flush = [&]() {
    if (!cur.segs.empty()) {
      cur.bytes = used;
      chunks.push_back(std::move(cur));
      tables.push_back(std::move(tab));
    }
    cur = ChunkWork();
    tab.clear();
    used = 0;
    cur_cap = chunk_cap(chunks.size());
  };
  for (const StorageView& s : storages) {
    for (const ByteExtent& e : extents) {
      int64_t off = e.offset;
      int64_t left = e.bytes;
      while (left > 0) {
        if (used >= cur_cap) {
          flush();
          continue;
        }
        const int64_t take = std::min(left, cur_cap - used);
        cur.segs.push_back(HostSegment{s.host + off, used, take});
        StridedCopy c;
        const uint64_t dev = s.dev + static_cast<uint64_t>(off);
        c.src = d2h ? dev : static_cast<uint64_t>(used);
        c.dst = d2h ? static_cast<uint64_t>(used) : dev;
        c.size = take;
        tab.push_back(c);
        used = AlignUp(used + take, 16);
        off += take;
        left -= take;
        unplanned -= take;
      }
    }
  }
  flush();
  for (size_t k = 0; k < chunks.size(); ++k) {
    const std::vector<StridedCopy>* t = &tables[k];
    chunks[k].kernel = [&lane, d2h, t](uint64_t buf) -> Status {
      std::vector<StridedCopy> copies = *t;
      for (StridedCopy& c : copies) (d2h ? c.dst : c.src) += buf;
      return LaunchStridedThroughRing(*lane.args, copies, lane.ks);
    };
  }
  int64_t memcpys = 0;
  KVX_RETURN_IF_ERROR(PipelineChunks(lane, dir, chunks, &memcpys));
  {
    std::lock_guard<std::mutex> l(mu_);
    stats_.memcpy_calls += memcpys;
    stats_.chunks += static_cast<int64_t>(chunks.size());
    stats_.kernel_launches += static_cast<int64_t>(chunks.size());
  }
  if (d2h) {
    *done = nullptr;  // complete once its bounce slots drain
    return OkStatus();
  }
  KVX_ASSIGN_OR_RETURN(*done, NewEvent());
  KVX_HIP_RETURN_IF_ERROR(hipEventRecord(*done, lane.ks));
  return OkStatus();
}

StatusOr<TransferEngine::PageableLane*> TransferEngine::Lane(Direction dir) {
  std::lock_guard<std::mutex> l(lanes_mu_);
  std::unique_ptr<PageableLane>& slot = lanes_[static_cast<int>(dir)];
  if (slot) return slot.get();
  DeviceGuard g(opts_.device);
  auto lane = std::make_unique<PageableLane>();
  KVX_RETURN_IF_ERROR(CreateStreamsOnDistinctQueues({&lane->ks, &lane->cs}));
  KVX_RETURN_IF_ERROR(lane->args.Init(1 << 20));
  // The thread that issues the lane's copies takes part in every host copy.
  lane->bounce = std::make_unique<Bounce>(opts_.host_copy_threads - 1);
  for (int k = 0; k < opts_.staging_chunks; ++k) {
    void* d = nullptr;
    KVX_HIP_RETURN_IF_ERROR(hipMalloc(&d, opts_.staging_chunk_bytes));
    lane->ring.bufs.push_back(reinterpret_cast<uint64_t>(d));
    KVX_ASSIGN_OR_RETURN(hipEvent_t ready, NewEvent());
    KVX_ASSIGN_OR_RETURN(hipEvent_t free_ev, NewEvent());
    lane->ring.ready.push_back(ready);
    lane->ring.free.push_back(free_ev);
    lane->ring.used.push_back(false);
    void* h = nullptr;
    KVX_HIP_RETURN_IF_ERROR(hipHostMalloc(&h, opts_.staging_chunk_bytes, hipHostMallocDefault));
    lane->bounce->bufs.push_back(static_cast<uint8_t*>(h));
    KVX_ASSIGN_OR_RETURN(hipEvent_t dma, NewEvent());
    lane->bounce->dma_done.push_back(dma);
    lane->bounce->event_dma.push_back(false);
    lane->bounce->used.push_back(false);
    lane->bounce->owed.emplace_back();
    lane->bounce->waiters.emplace_back();
  }
  if (!sdma_tried_) {
    // Fixed SDMA engines for the lanes' DMAs unless KVX_LANE_DMA=hip, or
    // ROCr cannot provide them (then hipMemcpyAsync).
    sdma_tried_ = true;
    const char* mode = std::getenv("KVX_LANE_DMA");
    if (mode == nullptr || std::string(mode) != "hip") {
      StatusOr<std::unique_ptr<SdmaEngines>> e = SdmaEngines::Create(opts_.device);
      if (e.ok()) sdma_ = std::move(e.value());
    }
  }
  if (sdma_) {
    for (int k = 0; k < opts_.staging_chunks; ++k) {
      KVX_ASSIGN_OR_RETURN(hsa_signal_t s, SdmaEngines::NewSignal());
      lane->bounce->dma_sig.push_back(s);
    }
    lane->bounce->sdma = sdma_.get();
  }
  PageableLane* raw = lane.get();
  lane->worker = std::thread([this, raw] { LaneLoop(raw); });
  slot = std::move(lane);
  return raw;
}

void TransferEngine::LaneLoop(PageableLane* lane) {
  Bounce* b = lane->bounce.get();
  while (true) {
    PageableLane::Job job;
    {
      std::unique_lock<std::mutex> l(lane->mu);
      lane->cv.wait(l, [lane] { return lane->stop || !lane->jobs.empty(); });
      if (lane->jobs.empty()) return;  // stopping, queue drained
      job = std::move(lane->jobs.front());
      lane->jobs.pop_front();
      lane->running = true;
    }
    Status st = OkStatus();
    hipEvent_t done = nullptr;
    {
      DeviceGuard g(opts_.device);
      if (job.dep_event != nullptr) {
        st = HipStatus(hipStreamWaitEvent(lane->ks, job.dep_event, 0), "dep wait");
        if (st.ok()) st = HipStatus(hipStreamWaitEvent(lane->cs, job.dep_event, 0), "dep wait");
        (void)hipEventDestroy(job.dep_event);
      }
      if (st.ok()) {
        LaneView v;
        v.ks = lane->ks;
        v.cs = lane->cs;
        v.ring = &lane->ring;
        v.args = &lane->args;
        v.bounce = b;
        st = job.extents.empty()
                 ? StagedOnLane(v, job.dir, job.storages, job.cdev, job.chost, nullptr, &done)
                 : ExtentsOnLane(v, job.dir, job.storages, job.extents, &done);
      }
    }
    if (!st.ok()) {
      job.future.Reject(st);
    } else {
      {
        std::lock_guard<std::mutex> l(mu_);
        ++stats_.staged_copies;
        ++stats_.bounce_copies;
      }
      if (done == nullptr && !b->order.empty()) {
        // D2H: the last bytes still sit in bounce buffers; the copy
        // completes when its newest slot drains (slots drain in order), so
        // the next copy's DMA overlaps these host copies.
        b->waiters[b->order.back()].push_back(job.future);
      } else {
        job.future.Fulfill(done != nullptr ? CopyFuture::FromEvents({done}, {}) : CopyFuture());
      }
    }
    bool idle;
    {
      std::lock_guard<std::mutex> l(lane->mu);
      idle = lane->jobs.empty();
    }
    if (idle) {
      // Nothing queued: finish every owed host copy now.
      DeviceGuard g(opts_.device);
      (void)b->DrainAll();  // failures reach the waiting copies' futures
    }
    {
      std::lock_guard<std::mutex> l(lane->mu);
      lane->running = false;
    }
    lane->idle_cv.notify_all();
  }
}

StatusOr<CopyFuture> TransferEngine::CopyPageable(Direction dir,
                                                  const std::vector<StorageView>& storages,
                                                  const std::vector<int64_t>& cdev,
                                                  const std::vector<int64_t>& chost,
                                                  const std::vector<ByteExtent>& extents,
                                                  hipStream_t dep) {
  KVX_ASSIGN_OR_RETURN(PageableLane * lane, Lane(dir));
  PageableLane::Job job{dir, storages, cdev, chost, extents, nullptr, CopyFuture::Pending()};
  if (dep != nullptr) {
    DeviceGuard g(opts_.device);
    KVX_ASSIGN_OR_RETURN(job.dep_event, NewEvent());
    KVX_HIP_RETURN_IF_ERROR(hipEventRecord(job.dep_event, dep));
  }
  CopyFuture f = job.future;
  {
    std::lock_guard<std::mutex> l(lane->mu);
    lane->jobs.push_back(std::move(job));
  }
  lane->cv.notify_one();
  return f;
}

StatusOr<CopyFuture> TransferEngine::DeviceCopy(
    bool gather, const std::vector<StorageView>& storages,
    const std::vector<int64_t>& ids, uint64_t staging, bool block_major,
    hipStream_t stream) {
  const int64_t n = static_cast<int64_t>(ids.size());
  if (n == 0 || storages.empty()) return CopyFuture();
  std::vector<Group> groups = MakeGroups(storages);
  if (block_major && groups.size() != 1) {
    return InvalidArgumentError("block-major staging needs one block size");
  }
  for (const Group& gr : groups) {
    if (static_cast<int64_t>(gr.members.size()) * n > UINT32_MAX) {
      return InvalidArgumentError("copy too large for one launch");
    }
  }
  std::lock_guard<std::mutex> l(mu_);
  DeviceGuard dg(opts_.device);
  int64_t arg_bytes = AlignUp(n * 8, kArgAlign);
  std::vector<int64_t> table_off(groups.size());
  for (size_t gi = 0; gi < groups.size(); ++gi) {
    table_off[gi] = arg_bytes;
    arg_bytes += AlignUp(static_cast<int64_t>(groups[gi].members.size()) * 8, kArgAlign);
  }
  KVX_ASSIGN_OR_RETURN(int64_t aoff, ArgAlloc(arg_bytes));
  ArgSliceGuard keep(
      [this, aoff, arg_bytes, stream] { return ArgCommit(aoff, aoff + arg_bytes, stream); },
      stream);
  std::memcpy(arg_host_ + aoff, ids.data(), n * 8);
  uint64_t acc = staging;
  for (size_t gi = 0; gi < groups.size(); ++gi) {
    uint64_t* t = reinterpret_cast<uint64_t*>(arg_host_ + aoff + table_off[gi]);
    for (size_t m = 0; m < groups[gi].members.size(); ++m) {
      t[m] = storages[groups[gi].members[m]].dev;
      acc |= t[m];
    }
    groups[gi].table_dev = arg_dev_ + aoff + table_off[gi];
  }
  KVX_HIP_RETURN_IF_ERROR(hipMemcpyAsync(reinterpret_cast<void*>(arg_dev_ + aoff),
                                         arg_host_ + aoff, arg_bytes,
                                         hipMemcpyHostToDevice, stream));
  int64_t off = 0;
  for (size_t g0 = 0; g0 < groups.size(); g0 += kMaxPieces) {
    CopyLaunch cl;
    cl.ids = reinterpret_cast<const int64_t*>(arg_dev_ + aoff);
    cl.n = n;
    for (size_t gi = g0; gi < groups.size() && gi < g0 + kMaxPieces; ++gi) {
      const Group& gr = groups[gi];
      const int64_t W = static_cast<int64_t>(gr.members.size());
      CopyPiece& c = cl.pieces[cl.npieces++];
      c.storages = gr.table_dev;
      c.staging = staging + static_cast<uint64_t>(off);
      c.stride_w = block_major ? gr.block_bytes : n * gr.block_bytes;
      c.stride_i = block_major ? W * gr.block_bytes : gr.block_bytes;
      c.f0 = 0;
      c.nblocks = W * n;
      c.block_bytes = gr.block_bytes;
      c.pool_blocks = gr.pool_blocks;
      acc |= static_cast<uint64_t>(off);
      off += W * n * gr.block_bytes;
    }
    const int vec = LaunchVectorBytes(cl, acc);
    KVX_RETURN_IF_ERROR(LaunchCopy(cl, gather, vec, stream));
  }
  KVX_RETURN_IF_ERROR(keep.Commit());
  KVX_ASSIGN_OR_RETURN(hipEvent_t done, NewEvent());
  KVX_HIP_RETURN_IF_ERROR(hipEventRecord(done, stream));
  return CopyFuture::FromEvents({done}, {});
}

}  // namespace kvx
