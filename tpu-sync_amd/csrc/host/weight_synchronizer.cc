#include "weight_synchronizer.h"

#include <algorithm>
#include <cstring>
#include <map>

#include "hip_util.h"
#include "numa.h"

namespace kvx {
namespace {

constexpr int64_t kTensorAlign = 256;

int64_t AlignUp(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

StatusOr<hipEvent_t> NewEvent() {
  hipEvent_t e = nullptr;
  KVX_HIP_RETURN_IF_ERROR(hipEventCreateWithFlags(&e, hipEventDisableTiming));
  return e;
}

}  // namespace

StatusOr<std::unique_ptr<WeightSynchronizer>> WeightSynchronizer::Create(
    WeightSyncConfig cfg) {
  std::unique_ptr<WeightSynchronizer> w(new WeightSynchronizer(std::move(cfg)));
  KVX_RETURN_IF_ERROR(w->Init());
  return w;
}

Status WeightSynchronizer::Init() {
  const int64_t n = cfg_.num_layers * cfg_.num_shards;
  if (cfg_.num_layers < 0 || cfg_.num_shards <= 0) {
    return InvalidArgumentError("num_layers must be >= 0 and num_shards >= 1");
  }
  if (static_cast<int64_t>(cfg_.device_ptrs.size()) != n ||
      static_cast<int64_t>(cfg_.device_bytes.size()) != n) {
    return InvalidArgumentError("device_ptrs and device_bytes need num_layers * num_shards entries");
  }
  if (cfg_.chunk_bytes <= 0 || cfg_.staging_chunks <= 0) {
    return InvalidArgumentError("staging chunk size and count must be positive");
  }
  if (!cfg_.tiled.empty() && static_cast<int64_t>(cfg_.tiled.size()) != n) {
    return InvalidArgumentError("tiled layouts need num_layers * num_shards entries (or none)");
  }
  off_.resize(n);
  host_bytes_.resize(n);
  int64_t pos = 0;
  for (int64_t k = 0; k < n; ++k) {
    if (cfg_.device_bytes[k] < 0 || (cfg_.device_bytes[k] > 0 && cfg_.device_ptrs[k] == 0)) {
      return InvalidArgumentError("null device pointer or negative size");
    }
    host_bytes_[k] = cfg_.device_bytes[k];
    if (const TiledPlan* tp = plan(k)) {
      if (cfg_.device_bytes[k] < tp->tiled_bytes) {
        return InvalidArgumentError("tensor " + std::to_string(k) +
                                    ": device buffer smaller than its tiled layout (" +
                                    std::to_string(tp->tiled_bytes) + " bytes)");
      }
      if (tp->tiled_bytes > 0 && cfg_.device_ptrs[k] == 0) {
        return InvalidArgumentError("null device pointer");
      }
      host_bytes_[k] = tp->logical_bytes;
    }
    off_[k] = pos;
    pos = AlignUp(pos + host_bytes_[k], kTensorAlign);
  }
  total_ = pos;
  DeviceGuard g(cfg_.device);
  if (!g.ok()) return InvalidArgumentError("cannot select HIP device");
  numa_node_ = cfg_.numa_local ? GpuNumaNode(cfg_.device) : -1;
  switch (cfg_.host_alloc) {
    case HostAllocKind::kPinned: {
      KVX_ASSIGN_OR_RETURN(host_, AllocatePinnedHost(static_cast<size_t>(total_), cfg_.device,
                                                     numa_node_));
      break;
    }
    case HostAllocKind::kMalloc: {
      KVX_ASSIGN_OR_RETURN(host_, AllocateMallocHost(static_cast<size_t>(total_), numa_node_));
      break;
    }
    default:
      return UnimplementedError("weight sync host memory must be pinned or malloc");
  }
  // Pack kernels and the two DMA directions on different hardware queues.
  KVX_RETURN_IF_ERROR(CreateStreamsOnDistinctQueues({&ks_, &d2h_, &h2d_}));
  const int64_t chunk = std::min<int64_t>(cfg_.chunk_bytes, std::max<int64_t>(total_, 1));
  cfg_.chunk_bytes = chunk;
  // A chunk must hold one tile row of every tiled tensor.
  for (int64_t k = 0; k < n; ++k) {
    const TiledPlan* tp = plan(k);
    if (tp == nullptr || !tp->standard) continue;
    const int64_t group =
        static_cast<int64_t>(std::min(tp->tH, tp->H) * tp->W) * tp->layout.itemsize;
    if (group > chunk) {
      return InvalidArgumentError("tensor " + std::to_string(k) + ": a tile row (" +
                                  std::to_string(group) +
                                  " bytes) does not fit a staging chunk");
    }
  }
  for (int k = 0; k < cfg_.staging_chunks; ++k) {
    // kTensorAlign spare bytes: a chunk sits at (lo mod kTensorAlign) in its
    // buffer (ChunkRange), so every tensor keeps its host alignment there.
    void* p = nullptr;
    KVX_HIP_RETURN_IF_ERROR(hipMalloc(&p, chunk + kTensorAlign));
    ring_.push_back(reinterpret_cast<uint64_t>(p));
    KVX_ASSIGN_OR_RETURN(hipEvent_t f, NewEvent());
    free_.push_back(f);
    slot_stream_.push_back(nullptr);
  }
  return args_.Init(1 << 20);
}

WeightSynchronizer::~WeightSynchronizer() {
  DeviceGuard g(cfg_.device);
  (void)Synchronize();
  for (Sample& s : samples_) {
    (void)hipEventDestroy(s.start);
    (void)hipEventDestroy(s.stop);
  }
  for (uint64_t b : ring_) (void)hipFree(reinterpret_cast<void*>(b));
  for (hipEvent_t e : free_) (void)hipEventDestroy(e);
  for (hipStream_t s : {ks_, d2h_, h2d_}) {
    if (s != nullptr) (void)hipStreamDestroy(s);
  }
}

Status WeightSynchronizer::Synchronize() {
  for (hipStream_t s : {ks_, d2h_, h2d_}) {
    if (s != nullptr) KVX_HIP_RETURN_IF_ERROR(hipStreamSynchronize(s));
  }
  return OkStatus();
}

Status WeightSynchronizer::WaitDep(hipStream_t dep, hipStream_t on) {
  if (dep == nullptr) return OkStatus();
  KVX_ASSIGN_OR_RETURN(hipEvent_t e, NewEvent());
  Status st = HipStatus(hipEventRecord(e, dep), "hipEventRecord(dep)");
  if (st.ok()) st = HipStatus(hipStreamWaitEvent(on, e, 0), "hipStreamWaitEvent");
  (void)hipEventDestroy(e);
  return st;
}

Status WeightSynchronizer::RangeEntries(int64_t lo, int64_t hi, uint64_t image, bool pack,
                                        std::vector<StridedCopy>* out,
                                        std::vector<TiledJob>* zero,
                                        std::vector<TiledJob>* tiled) const {
  out->clear();
  zero->clear();
  tiled->clear();
  // Tensors are laid out in ascending offset order: find the first one that
  // ends after lo.
  const int64_t n = static_cast<int64_t>(off_.size());
  int64_t k = std::upper_bound(off_.begin(), off_.end(), lo) - off_.begin() - 1;
  if (k < 0) k = 0;
  for (; k < n && off_[k] < hi; ++k) {
    const int64_t a = std::max(lo, off_[k]);
    const int64_t b = std::min(hi, off_[k] + host_bytes_[k]);
    if (a >= b) continue;
    if (const TiledPlan* tp = plan(k)) {
      // The linear image of tensor k starts (off_k - lo) bytes into `image`
      // (only its bytes in [a, b) are touched).
      const uint64_t origin = image + static_cast<uint64_t>(off_[k]) - static_cast<uint64_t>(lo);
      KVX_RETURN_IF_ERROR(AppendTiledJobs(*tp, cfg_.device_ptrs[k], origin, a - off_[k],
                                          b - off_[k], /*tile=*/!pack,
                                          /*zero_pass=*/a == off_[k], zero, tiled));
      continue;
    }
    StridedCopy c;
    const uint64_t dev = cfg_.device_ptrs[k] + static_cast<uint64_t>(a - off_[k]);
    const uint64_t img = image + static_cast<uint64_t>(a - lo);
    c.src = pack ? dev : img;
    c.dst = pack ? img : dev;
    c.size = b - a;
    c.count = 1;
    out->push_back(c);
  }
  return OkStatus();
}

Status WeightSynchronizer::Launch(const std::vector<StridedCopy>& copies,
                                  const std::vector<TiledJob>& zero,
                                  const std::vector<TiledJob>& tiled, bool pack,
                                  hipStream_t stream) {
  Sample s;
  if (cfg_.profile_kernels) {
    KVX_HIP_RETURN_IF_ERROR(hipEventCreate(&s.start));
    KVX_HIP_RETURN_IF_ERROR(hipEventCreate(&s.stop));
  }
  // The start event goes on the stream after the first table upload, so a
  // sample times the kernels alone. Padding is cleared before any data of
  // the same tensors is written.
  hipEvent_t start = s.start;
  if (!zero.empty()) {
    KVX_RETURN_IF_ERROR(LaunchTiledThroughRing(args_, zero, stream, start));
    start = nullptr;
  }
  if (!copies.empty()) {
    KVX_RETURN_IF_ERROR(LaunchStridedThroughRing(args_, copies, stream, 0, start));
    start = nullptr;
  }
  if (!tiled.empty()) {
    KVX_RETURN_IF_ERROR(LaunchTiledThroughRing(args_, tiled, stream, start));
    start = nullptr;
  }
  if (cfg_.profile_kernels) {
    if (start != nullptr) KVX_HIP_RETURN_IF_ERROR(hipEventRecord(start, stream));
    KVX_HIP_RETURN_IF_ERROR(hipEventRecord(s.stop, stream));
    for (const StridedCopy& c : copies) s.bytes += c.size * (c.count > 0 ? c.count : 1);
    for (const TiledJob& j : tiled) {
      const bool std_form = j.dev.mode == kDetileStd || j.dev.mode == kTileStd;
      s.bytes += static_cast<int64_t>(j.dev.count) *
                 (std_form ? static_cast<int64_t>(j.dev.P) * j.vec : j.dev.itemsize);
    }
    s.pack = pack;
    samples_.push_back(s);
  }
  return OkStatus();
}

Status WeightSynchronizer::KernelTimes(bool pack, bool reset, int64_t* launches, double* ms,
                                       int64_t* bytes) {
  std::lock_guard<std::mutex> l(mu_);
  *launches = 0;
  *ms = 0;
  *bytes = 0;
  std::vector<Sample> keep;
  for (Sample& s : samples_) {
    if (s.pack != pack) {
      keep.push_back(s);
      continue;
    }
    KVX_HIP_RETURN_IF_ERROR(hipEventSynchronize(s.stop));
    float t = 0;
    KVX_HIP_RETURN_IF_ERROR(hipEventElapsedTime(&t, s.start, s.stop));
    ++*launches;
    *ms += t;
    *bytes += s.bytes;
    if (reset) {
      (void)hipEventDestroy(s.start);
      (void)hipEventDestroy(s.stop);
    } else {
      keep.push_back(s);
    }
  }
  samples_.swap(keep);
  return OkStatus();
}

StatusOr<int64_t> WeightSynchronizer::CutBelow(int64_t lo, int64_t x) const {
  const int64_t n = static_cast<int64_t>(off_.size());
  const int64_t k = std::upper_bound(off_.begin(), off_.end(), x) - off_.begin() - 1;
  int64_t cut;
  const TiledPlan* tp = k >= 0 && k < n ? plan(k) : nullptr;
  if (tp != nullptr && x < off_[k] + host_bytes_[k]) {
    cut = off_[k] + tp->CutAtOrBelow(x - off_[k]);
  } else {
    // Elsewhere keep chunk starts 256-byte aligned, like the tensors.
    cut = x / kTensorAlign * kTensorAlign;
    if (cut <= lo) cut = x;
  }
  if (cut <= lo) {
    return InternalError("staging chunk holds no whole tile row of tensor " + std::to_string(k));
  }
  return cut;
}

Status WeightSynchronizer::ChunkRange(bool d2h, int64_t range_lo, int64_t range_hi) {
  hipStream_t cs = d2h ? d2h_ : h2d_;
  const int64_t C = cfg_.chunk_bytes;
  std::vector<StridedCopy> entries;
  std::vector<TiledJob> zero, tiled;
  int64_t hi = range_lo;
  for (int64_t lo = range_lo; lo < range_hi; lo = hi) {
    hi = std::min(range_hi, lo + C);
    if (hi < range_hi) {
      KVX_ASSIGN_OR_RETURN(hi, CutBelow(lo, hi));
    }
    const size_t k = next_;
    next_ = (next_ + 1) % ring_.size();
    // The chunk starts at lo's offset within a kTensorAlign span of its
    // buffer (hipMalloc returns kTensorAlign-aligned memory), so a tensor at
    // a kTensorAlign-aligned host offset is kTensorAlign-aligned in staging
    // too, wherever the previous cut fell (a tile row of an odd-width int8
    // tensor, say): the vector kernels keep their widest vectors and no
    // tensor origin drops below its element size.
    const uint64_t buf = ring_[k] + static_cast<uint64_t>(lo % kTensorAlign);
    KVX_RETURN_IF_ERROR(RangeEntries(lo, hi, buf, /*pack=*/d2h, &entries, &zero, &tiled));
    // Both directions share the ring: a slot last used by the other
    // direction's stream is reused once that use has finished.
    if (slot_stream_[k] != nullptr && slot_stream_[k] != cs) {
      KVX_HIP_RETURN_IF_ERROR(hipStreamWaitEvent(cs, free_[k], 0));
    }
    if (d2h) {
      KVX_RETURN_IF_ERROR(Launch(entries, zero, tiled, true, cs));
      KVX_HIP_RETURN_IF_ERROR(hipMemcpyAsync(host_.ptr + lo, reinterpret_cast<void*>(buf),
                                             static_cast<size_t>(hi - lo),
                                             hipMemcpyDeviceToHost, cs));
    } else {
      KVX_HIP_RETURN_IF_ERROR(hipMemcpyAsync(reinterpret_cast<void*>(buf), host_.ptr + lo,
                                             static_cast<size_t>(hi - lo),
                                             hipMemcpyHostToDevice, cs));
      KVX_RETURN_IF_ERROR(Launch(entries, zero, tiled, false, cs));
    }
    KVX_HIP_RETURN_IF_ERROR(hipEventRecord(free_[k], cs));
    slot_stream_[k] = cs;
  }
  return OkStatus();
}

StatusOr<CopyFuture> WeightSynchronizer::Chunked(bool d2h, hipStream_t dep) {
  std::lock_guard<std::mutex> l(mu_);
  DeviceGuard g(cfg_.device);
  if (total_ == 0) return CopyFuture();
  // Each chunk's kernel and DMA run in order on the direction's one stream.
  // With the kernels on a stream of their own, chained to the DMAs by
  // events, every chunk is enqueued at once and the runtime's copies slowed
  // down: the 16.06 GB Llama-3-8B set moved D2H at 33-39 GB/s in 256 MiB
  // chunks and 23-24 GB/s in 32 MiB chunks, against 55.6 / 53.4 on one
  // stream (H2D 53.6 / 48 against 55.8 / 53.6); the kernel then waits for
  // the previous chunk's DMA, a few percent of the DMA's time.
  hipStream_t cs = d2h ? d2h_ : h2d_;
  KVX_RETURN_IF_ERROR(WaitDep(dep, cs));
  KVX_RETURN_IF_ERROR(ChunkRange(d2h, 0, total_));
  KVX_ASSIGN_OR_RETURN(hipEvent_t done, NewEvent());
  KVX_HIP_RETURN_IF_ERROR(hipEventRecord(done, cs));
  return CopyFuture::FromEvents({done}, {host_.owner});
}

StatusOr<CopyFuture> WeightSynchronizer::D2h(hipStream_t dep) { return Chunked(true, dep); }
StatusOr<CopyFuture> WeightSynchronizer::H2d(hipStream_t dep) { return Chunked(false, dep); }

StatusOr<CopyFuture> WeightSynchronizer::D2hLayer(int64_t layer, hipStream_t dep) {
  if (layer < 0 || layer >= cfg_.num_layers) return CopyFuture();
  std::lock_guard<std::mutex> l(mu_);
  DeviceGuard g(cfg_.device);
  KVX_RETURN_IF_ERROR(WaitDep(dep, d2h_));
  for (int64_t s = 0; s < cfg_.num_shards; ++s) {
    const int64_t k = layer * cfg_.num_shards + s;
    if (host_bytes_[k] == 0) continue;
    if (plan(k) != nullptr) {
      // Detiled in HBM through the staging ring, as the whole set is.
      KVX_RETURN_IF_ERROR(ChunkRange(true, off_[k], off_[k] + host_bytes_[k]));
      continue;
    }
    KVX_HIP_RETURN_IF_ERROR(hipMemcpyAsync(host_.ptr + off_[k],
                                           reinterpret_cast<void*>(cfg_.device_ptrs[k]),
                                           static_cast<size_t>(cfg_.device_bytes[k]),
                                           hipMemcpyDeviceToHost, d2h_));
  }
  KVX_ASSIGN_OR_RETURN(hipEvent_t done, NewEvent());
  KVX_HIP_RETURN_IF_ERROR(hipEventRecord(done, d2h_));
  return CopyFuture::FromEvents({done}, {host_.owner});
}

StatusOr<CopyFuture> WeightSynchronizer::H2dLayer(int64_t layer, hipStream_t dep) {
  if (layer < 0 || layer >= cfg_.num_layers) return CopyFuture();
  std::lock_guard<std::mutex> l(mu_);
  DeviceGuard g(cfg_.device);
  KVX_RETURN_IF_ERROR(WaitDep(dep, h2d_));
  for (int64_t s = 0; s < cfg_.num_shards; ++s) {
    const int64_t k = layer * cfg_.num_shards + s;
    if (host_bytes_[k] == 0) continue;
    if (plan(k) != nullptr) {
      KVX_RETURN_IF_ERROR(ChunkRange(false, off_[k], off_[k] + host_bytes_[k]));
      continue;
    }
    KVX_HIP_RETURN_IF_ERROR(hipMemcpyAsync(reinterpret_cast<void*>(cfg_.device_ptrs[k]),
                                           host_.ptr + off_[k],
                                           static_cast<size_t>(cfg_.device_bytes[k]),
                                           hipMemcpyHostToDevice, h2d_));
  }
  KVX_ASSIGN_OR_RETURN(hipEvent_t done, NewEvent());
  KVX_HIP_RETURN_IF_ERROR(hipEventRecord(done, h2d_));
  return CopyFuture::FromEvents({done}, {host_.owner});
}

StatusOr<CopyFuture> WeightSynchronizer::WholeCopy(bool pack, uint64_t staging, int64_t bytes,
                                                   hipStream_t stream) {
  if (staging == 0 || bytes < total_) {
    return InvalidArgumentError("staging buffer smaller than the packed parameter set (" +
                                std::to_string(total_) + " bytes)");
  }
  std::lock_guard<std::mutex> l(mu_);
  DeviceGuard g(cfg_.device);
  std::vector<StridedCopy> entries;
  std::vector<TiledJob> zero, tiled;
  KVX_RETURN_IF_ERROR(RangeEntries(0, total_, staging, pack, &entries, &zero, &tiled));
  KVX_RETURN_IF_ERROR(Launch(entries, zero, tiled, pack, stream));
  KVX_ASSIGN_OR_RETURN(hipEvent_t done, NewEvent());
  KVX_HIP_RETURN_IF_ERROR(hipEventRecord(done, stream));
  return CopyFuture::FromEvents({done}, {});
}

StatusOr<CopyFuture> WeightSynchronizer::Pack(uint64_t staging, int64_t bytes,
                                              hipStream_t stream) {
  return WholeCopy(true, staging, bytes, stream);
}

StatusOr<CopyFuture> WeightSynchronizer::Unpack(uint64_t staging, int64_t bytes,
                                                hipStream_t stream) {
  return WholeCopy(false, staging, bytes, stream);
}

namespace {

// One argument ring per device for the stand-alone copies; callers hold
// RingMutex().
std::mutex& RingMutex() {
  static std::mutex* mu = new std::mutex();
  return *mu;
}

StatusOr<ArgRing*> DeviceRing(int device) {
  static std::map<int, ArgRing*>* rings = new std::map<int, ArgRing*>();
  ArgRing*& ring = (*rings)[device];
  if (ring == nullptr) {
    auto* r = new ArgRing();
    Status st = r->Init(1 << 20);
    if (!st.ok()) {
      delete r;
      return st;
    }
    ring = r;
  }
  return ring;
}

}  // namespace

StatusOr<CopyFuture> CopyStridedOnDevice(int device, const std::vector<StridedCopy>& copies,
                                         hipStream_t stream) {
  std::lock_guard<std::mutex> l(RingMutex());
  DeviceGuard g(device);
  if (!g.ok()) return InvalidArgumentError("cannot select HIP device");
  KVX_ASSIGN_OR_RETURN(ArgRing * ring, DeviceRing(device));
  KVX_RETURN_IF_ERROR(LaunchStridedThroughRing(*ring, copies, stream));
  KVX_ASSIGN_OR_RETURN(hipEvent_t done, NewEvent());
  KVX_HIP_RETURN_IF_ERROR(hipEventRecord(done, stream));
  return CopyFuture::FromEvents({done}, {});
}

StatusOr<CopyFuture> TileOnDevice(int device, const TiledPlan& plan, uint64_t linear,
                                  uint64_t tiled, bool tile, hipStream_t stream) {
  if (plan.logical_bytes > 0 && (linear == 0 || tiled == 0)) {
    return InvalidArgumentError("null buffer");
  }
  if (!plan.tiled) {
    // No tiles: the bytes as they are (tiling_utils.cc:959-964, 993-998).
    if (plan.logical_bytes == 0) return CopyStridedOnDevice(device, {}, stream);
    StridedCopy c;
    c.src = tile ? linear : tiled;
    c.dst = tile ? tiled : linear;
    c.size = plan.logical_bytes;
    return CopyStridedOnDevice(device, {c}, stream);
  }
  std::vector<TiledJob> zero, jobs;
  KVX_RETURN_IF_ERROR(AppendTiledJobs(plan, tiled, linear, 0, plan.logical_bytes, tile,
                                      /*zero_pass=*/true, &zero, &jobs));
  std::lock_guard<std::mutex> l(RingMutex());
  DeviceGuard g(device);
  if (!g.ok()) return InvalidArgumentError("cannot select HIP device");
  KVX_ASSIGN_OR_RETURN(ArgRing * ring, DeviceRing(device));
  KVX_RETURN_IF_ERROR(LaunchTiledThroughRing(*ring, zero, stream));
  KVX_RETURN_IF_ERROR(LaunchTiledThroughRing(*ring, jobs, stream));
  KVX_ASSIGN_OR_RETURN(hipEvent_t done, NewEvent());
  KVX_HIP_RETURN_IF_ERROR(hipEventRecord(done, stream));
  return CopyFuture::FromEvents({done}, {});
}

StatusOr<std::unique_ptr<StridedCopyPlan>> StridedCopyPlan::Create(
    int device, const std::vector<StridedCopy>& copies) {
  std::unique_ptr<StridedCopyPlan> p(new StridedCopyPlan());
  p->device_ = device;
  std::vector<StridedEntryDev> table;
  if (!copies.empty()) {
    p->vec_ = StridedVectorBytes(copies);
    if (!BuildStridedTable(copies, p->vec_, &table, &p->grid_, &p->long_tiles_)) {
      return InvalidArgumentError("strided copy entry out of the kernel's limits");
    }
  }
  p->n_ = static_cast<uint32_t>(table.size());
  for (const StridedCopy& c : copies) {
    p->bytes_ += c.size * (c.count <= 0 ? 1 : c.count);
  }
  if (p->grid_ == 0) return p;
  DeviceGuard g(device);
  if (!g.ok()) return InvalidArgumentError("cannot select HIP device");
  std::vector<uint8_t> image(static_cast<size_t>(StridedImageBytes(table.size(), p->grid_)));
  WriteStridedImage(table, p->grid_, image.data());
  KVX_HIP_RETURN_IF_ERROR(hipMalloc(&p->image_, image.size()));
  KVX_HIP_RETURN_IF_ERROR(
      hipMemcpy(p->image_, image.data(), image.size(), hipMemcpyHostToDevice));
  return p;
}

StridedCopyPlan::~StridedCopyPlan() {
  DeviceGuard g(device_);
  for (hipEvent_t e : runs_) {
    (void)hipEventSynchronize(e);
    (void)hipEventDestroy(e);
  }
  for (auto& s : samples_) {
    (void)hipEventSynchronize(s.second);
    (void)hipEventDestroy(s.first);
    (void)hipEventDestroy(s.second);
  }
  if (image_ != nullptr) (void)hipFree(image_);
}

void StridedCopyPlan::SetProfiling(bool on) {
  std::lock_guard<std::mutex> l(mu_);
  profile_ = on;
}

Status StridedCopyPlan::KernelTimes(bool reset, int64_t* launches, double* ms, int64_t* bytes) {
  DeviceGuard g(device_);
  if (!g.ok()) return InvalidArgumentError("cannot select HIP device");
  std::lock_guard<std::mutex> l(mu_);
  *launches = 0;
  *ms = 0;
  *bytes = 0;
  for (auto& s : samples_) {
    KVX_HIP_RETURN_IF_ERROR(hipEventSynchronize(s.second));
    float t = 0;
    KVX_HIP_RETURN_IF_ERROR(hipEventElapsedTime(&t, s.first, s.second));
    ++*launches;
    *ms += t;
    *bytes += 2 * bytes_;
  }
  if (reset) {
    for (auto& s : samples_) {
      (void)hipEventDestroy(s.first);
      (void)hipEventDestroy(s.second);
    }
    samples_.clear();
  }
  return OkStatus();
}

StatusOr<CopyFuture> StridedCopyPlan::Run(hipStream_t stream) {
  DeviceGuard g(device_);
  if (!g.ok()) return InvalidArgumentError("cannot select HIP device");
  std::lock_guard<std::mutex> l(mu_);
  // Both events exist before the launch, so a launched run is always
  // tracked and always has a future.
  KVX_ASSIGN_OR_RETURN(hipEvent_t done, NewEvent());
  if (grid_ > 0) {
    // Runs that have finished no longer read the image.
    for (auto it = runs_.begin(); it != runs_.end();) {
      if (hipEventQuery(*it) == hipSuccess) {
        (void)hipEventDestroy(*it);
        it = runs_.erase(it);
      } else {
        ++it;
      }
    }
    StatusOr<hipEvent_t> ran = NewEvent();
    if (!ran.ok()) {
      (void)hipEventDestroy(done);
      return ran.status();
    }
    runs_.push_back(ran.value());
    hipEvent_t t0 = nullptr, t1 = nullptr;
    if (profile_ && (hipEventCreate(&t0) != hipSuccess || hipEventCreate(&t1) != hipSuccess ||
                     hipEventRecord(t0, stream) != hipSuccess)) {
      // Profiling is best effort: this run goes unsampled.
      (void)hipGetLastError();
      if (t0 != nullptr) (void)hipEventDestroy(t0);
      if (t1 != nullptr) (void)hipEventDestroy(t1);
      t0 = t1 = nullptr;
    }
    const hipError_t e = LaunchStridedCopy(static_cast<const StridedEntryDev*>(image_), n_,
                                           grid_, vec_, stream, 0, long_tiles_);
    if (e != hipSuccess) {
      if (t0 != nullptr) (void)hipEventDestroy(t0);
      if (t1 != nullptr) (void)hipEventDestroy(t1);
      (void)hipEventDestroy(done);
      return HipStatus(e, "strided copy launch");
    }
    if (t0 != nullptr) {
      if (hipEventRecord(t1, stream) == hipSuccess) {
        samples_.emplace_back(t0, t1);
      } else {
        (void)hipGetLastError();
        (void)hipEventDestroy(t0);
        (void)hipEventDestroy(t1);
      }
    }
    // The image must outlive the launch: without its event, wait here.
    if (hipEventRecord(ran.value(), stream) != hipSuccess) (void)hipStreamSynchronize(stream);
  }
  const hipError_t rec = hipEventRecord(done, stream);
  if (rec != hipSuccess) {
    (void)hipEventDestroy(done);
    return HipStatus(rec, "hipEventRecord");
  }
  return CopyFuture::FromEvents({done}, {});
}

}  // namespace kvx
