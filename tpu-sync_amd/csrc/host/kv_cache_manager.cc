#include "kv_cache_manager.h"

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <string>

#include "hip_util.h"
#include "numa.h"

namespace kvx {

Status ValidateOffsetsAndSizes(const std::vector<int64_t>& src_offsets,
                               const std::vector<int64_t>& dst_offsets,
                               const std::vector<int64_t>& sizes) {
  if (!dst_offsets.empty() && src_offsets.size() != dst_offsets.size()) {
    return InvalidArgumentError(
        "src_offsets, dst_offsets, and sizes must have the same length");
  }
  if (!sizes.empty() && src_offsets.size() != sizes.size()) {
    return InvalidArgumentError(
        "src_offsets, dst_offsets, and sizes must have the same length");
  }
  for (const std::vector<int64_t>* v : {&src_offsets, &dst_offsets, &sizes}) {
    for (int64_t x : *v) {
      if (x < 0) {
        return InvalidArgumentError("copy offsets and sizes must be non-negative");
      }
    }
  }
  return OkStatus();
}

void CoalesceMajorDimCopies(const std::vector<int64_t>& src_offsets,
                            const std::vector<int64_t>& dst_offsets,
                            const std::vector<int64_t>& sizes,
                            std::vector<int64_t>& out_src,
                            std::vector<int64_t>& out_dst,
                            std::vector<int64_t>& out_sizes) {
  out_src.clear();
  out_dst.clear();
  out_sizes.clear();
  for (size_t i = 0; i < src_offsets.size(); ++i) {
    const bool extends = !out_src.empty() &&
                         src_offsets[i] == out_src.back() + out_sizes.back() &&
                         dst_offsets[i] == out_dst.back() + out_sizes.back();
    if (extends) {
      out_sizes.back() += sizes[i];
    } else {
      out_src.push_back(src_offsets[i]);
      out_dst.push_back(dst_offsets[i]);
      out_sizes.push_back(sizes[i]);
    }
  }
}

namespace {

// a * b + c <= limit without overflow, for non-negative operands.
bool RangeFits(int64_t a, int64_t b, int64_t c, int64_t limit) {
  int64_t prod = 0;
  int64_t sum = 0;
  if (__builtin_mul_overflow(a, b, &prod)) return false;
  if (__builtin_add_overflow(prod, c, &sum)) return false;
  return sum <= limit;
}

}  // namespace

StatusOr<std::unique_ptr<KVCacheManager>> KVCacheManager::Create(
    ManagerConfig cfg) {
  std::unique_ptr<KVCacheManager> m(new KVCacheManager(std::move(cfg)));
  KVX_RETURN_IF_ERROR(m->Init());
  return m;
}

Status KVCacheManager::Init() {
  num_layers_ = cfg_.num_layers;
  num_shards_ = cfg_.num_shards;
  if (num_layers_ < 0 || num_shards_ < 0) {
    return InvalidArgumentError("num_layers and num_shards must be non-negative");
  }
  if (cfg_.host_blocks < 0 || cfg_.host_blocks > std::numeric_limits<int>::max()) {
    return InvalidArgumentError("host_blocks out of range");
  }
  host_blocks_ = cfg_.host_blocks;
  const bool device_backed = !cfg_.device_ptrs.empty();
  const size_t nstor = static_cast<size_t>(num_layers_ * num_shards_);
  major_dim_ = cfg_.major_dim;
  layer_block_bytes_.assign(num_layers_, 0);
  layer_physical_bytes_.assign(num_layers_, 0);
  storages_.assign(nstor, StorageInfo{});

  if (device_backed) {
    if (cfg_.device_ptrs.size() != nstor || cfg_.device_bytes.size() != nstor) {
      return InvalidArgumentError(
          "device_ptrs and device_bytes need num_layers * num_shards entries");
    }
    if (major_dim_ <= 0) return InvalidArgumentError("major_dim must be positive");
    for (int64_t l = 0; l < num_layers_; ++l) {
      // The layer's on-device size is the size of its first shard
      // (kv_cache_manager_base.cc:287-296).
      const int64_t phys = cfg_.device_bytes[l * num_shards_];
      layer_physical_bytes_[l] = phys;
      layer_block_bytes_[l] = phys / major_dim_;
      for (int64_t s = 0; s < num_shards_; ++s) {
        const size_t k = l * num_shards_ + s;
        if (cfg_.device_bytes[k] < phys) {
          return InvalidArgumentError(
              "Device buffer shard size smaller than physical size");
        }
        if (cfg_.device_ptrs[k] == 0) {
          return InvalidArgumentError("null device pointer");
        }
        storages_[k].dev = cfg_.device_ptrs[k];
        storages_[k].dev_bytes = cfg_.device_bytes[k];
      }
    }
    slice_byte_size_ = cfg_.slice_byte_size > 0
                           ? cfg_.slice_byte_size
                           : (num_layers_ > 0 ? layer_block_bytes_[0] : 0);
  } else {
    slice_byte_size_ = cfg_.slice_byte_size;
    if (slice_byte_size_ < 0) return InvalidArgumentError("slice_byte_size < 0");
    for (int64_t l = 0; l < num_layers_; ++l) layer_block_bytes_[l] = slice_byte_size_;
  }

  lbm_ = std::make_unique<LogicalBlockManager>(static_cast<int>(host_blocks_));

  switch (cfg_.numa) {
    case ManagerConfig::Numa::kAuto:
      numa_node_ = device_backed ? GpuNumaNode(cfg_.device) : -1;
      break;
    case ManagerConfig::Numa::kNode:
      if (cfg_.numa_node < 0) return InvalidArgumentError("numa_node must be non-negative");
      numa_node_ = cfg_.numa_node;
      break;
    default:
      numa_node_ = -1;
  }

  // Shared-memory host tier: one segment holds every (layer, shard) mirror
  // back to back, [storage][host_blocks][layer block bytes]. (The
  // reference's shm allocator hands the same mapping to every mirror, which
  // aliases the layers of a multi-layer pool.)
  HostBufferAllocation shm;
  int64_t shm_off = 0;
  if (cfg_.host_alloc == HostAllocKind::kShm) {
    if (cfg_.shm_key.empty()) {
      return InvalidArgumentError("shared-memory host tier needs a shm_key");
    }
    int64_t total = 0;
    for (size_t k = 0; k < nstor; ++k) {
      const int64_t layer_bb = layer_block_bytes_[k / num_shards_];
      if (!RangeFits(host_blocks_, layer_bb, total, std::numeric_limits<int64_t>::max())) {
        return InvalidArgumentError("host mirror size overflows");
      }
      total += host_blocks_ * layer_bb;
    }
    SharedMemoryHeader want;
    const std::string uid = cfg_.model_uid.empty() ? "default_model" : cfg_.model_uid;
    if (uid.size() >= sizeof(want.model_uid)) {
      return InvalidArgumentError("model_uid too long");
    }
    std::memcpy(want.model_uid, uid.data(), uid.size());
    want.num_blocks = static_cast<uint32_t>(host_blocks_);
    want.block_size = static_cast<uint32_t>(slice_byte_size_);
    const std::string name = ShmSegmentName(cfg_.shm_key, cfg_.shm_server_name,
                                            device_backed ? cfg_.device : -1);
    KVX_ASSIGN_OR_RETURN(shm, AllocateShmHost(name, want, static_cast<size_t>(total),
                                              &shm_warm_, numa_node_));
  }

  for (size_t k = 0; k < nstor; ++k) {
    // Each (layer, shard) mirror holds host_blocks blocks of that layer's own
    // block size. The reference sizes every mirror by the first layer's
    // block; per-layer sizing is the same for uniform models and lets side
    // tables with small blocks (fp8 scales) keep small mirrors.
    const int64_t layer_bb = layer_block_bytes_[k / num_shards_];
    if (!RangeFits(host_blocks_, layer_bb, 0, std::numeric_limits<int64_t>::max())) {
      return InvalidArgumentError("host mirror size overflows");
    }
    const int64_t alloc_size = host_blocks_ * layer_bb;
    StatusOr<HostBufferAllocation> a = Status();
    switch (cfg_.host_alloc) {
      case HostAllocKind::kMalloc:
        a = AllocateMallocHost(static_cast<size_t>(alloc_size), numa_node_);
        break;
      case HostAllocKind::kPinned:
        a = device_backed ? AllocatePinnedHost(static_cast<size_t>(alloc_size), cfg_.device,
                                               numa_node_)
                          : AllocateMallocHost(static_cast<size_t>(alloc_size), numa_node_);
        break;
      case HostAllocKind::kShm: {
        HostBufferAllocation part;
        part.ptr = shm.ptr + shm_off;
        part.size = static_cast<size_t>(alloc_size);
        part.owner = shm.owner;
        shm_off += alloc_size;
        a = part;
        break;
      }
      default:
        return UnimplementedError("host allocator kind not supported");
    }
    if (!a.ok()) return a.status();
    if (alloc_size > 0 && a->ptr == nullptr) {
      return InternalError("Host allocator returned null buffer for size: " +
                           std::to_string(alloc_size));
    }
    storages_[k].host = a->ptr;
    storages_[k].host_bytes = static_cast<int64_t>(a->size);
    storages_[k].host_owner = a->owner;
    allocated_host_bytes_ += a->size;
  }

  if (device_backed) {
    EngineOptions eo = cfg_.engine;
    eo.device = cfg_.device;
    KVX_ASSIGN_OR_RETURN(engine_, TransferEngine::Create(eo));
    // hipHostMalloc memory is mapped into the GPU's address space, so the
    // copy kernels may read and write the mirror directly.
    host_kernel_access_ = cfg_.host_alloc == HostAllocKind::kPinned;
  }
  switch (cfg_.dispatch) {
    case ManagerConfig::Dispatch::kQueued:
      queued_ = true;
      break;
    case ManagerConfig::Dispatch::kEnv: {
      const char* env = std::getenv("RAIDEN_ENABLE_ASYNC_DISPATCH");
      queued_ = env != nullptr && std::string(env) == "1";
      break;
    }
    default:
      queued_ = false;
  }
  if (queued_) {
    if (engine_) {
      DeviceGuard g(cfg_.device);
      KVX_HIP_RETURN_IF_ERROR(hipStreamCreateWithFlags(&dep_proxy_, hipStreamNonBlocking));
    }
    worker_ = std::thread(&KVCacheManager::WorkerLoop, this);
  }
  return OkStatus();
}

KVCacheManager::~KVCacheManager() {
  StopWorker();
  (void)WaitForPendingWork();
  if (dep_proxy_ != nullptr) {
    DeviceGuard g(cfg_.device);
    (void)hipStreamDestroy(dep_proxy_);
  }
}

Status KVCacheManager::WaitForPendingWork() {
  if (!engine_) return OkStatus();
  // The engine's streams are private: waiting on them leaves unrelated
  // framework work on the device alone.
  return engine_->Synchronize();
}

StatusOr<std::vector<KVCacheManager::Work>> KVCacheManager::SelectWorks(
    std::optional<size_t> layer_idx, std::optional<size_t> shard_idx) const {
  if (layer_idx.has_value() && *layer_idx >= static_cast<size_t>(num_layers_)) {
    return OutOfRangeError("layer or shard index out of range");
  }
  if (shard_idx.has_value() && *shard_idx >= static_cast<size_t>(num_shards_)) {
    return OutOfRangeError("layer or shard index out of range");
  }
  std::vector<Work> works;
  for (int64_t l = 0; l < num_layers_; ++l) {
    if (layer_idx.has_value() && *layer_idx != static_cast<size_t>(l)) continue;
    for (int64_t s = 0; s < num_shards_; ++s) {
      if (shard_idx.has_value() && *shard_idx != static_cast<size_t>(s)) continue;
      works.push_back(Work{static_cast<size_t>(l), static_cast<size_t>(s)});
    }
  }
  return works;
}

StatusOr<CopyFuture> KVCacheManager::Transfer(
    Direction dir, const std::vector<int64_t>& src,
    const std::vector<int64_t>& dst, const std::vector<int64_t>& sizes_in,
    std::optional<int64_t> slot_idx, std::optional<size_t> layer_idx,
    std::optional<size_t> shard_idx, hipStream_t dep) {
  const bool d2h = dir == Direction::kD2H;
  {
    std::lock_guard<std::mutex> l(log_mu_);
    dispatch_log_.push_back(d2h ? 'D' : 'H');
    if (dispatch_log_.size() > 256) dispatch_log_.erase(0, dispatch_log_.size() - 256);
  }
  if (!engine_) {
    return FailedPreconditionError(
        d2h ? "D2h requires a device-backed KVCacheManagerBase"
            : "H2d requires a device-backed KVCacheManagerBase");
  }
  KVX_RETURN_IF_ERROR(ValidateOffsetsAndSizes(src, dst, sizes_in));
  // The reference coalesces src against dst and sizes element-wise; a list
  // with sources but without destinations has nothing to pair them with.
  if (!src.empty() && dst.empty()) {
    return InvalidArgumentError(
        "src_offsets, dst_offsets, and sizes must have the same length");
  }
  std::vector<int64_t> sizes = sizes_in;
  if (sizes.empty()) sizes.assign(src.size(), 1);
  KVX_ASSIGN_OR_RETURN(std::vector<Work> works, SelectWorks(layer_idx, shard_idx));
  std::vector<int64_t> src_c, dst_c, sizes_c;
  CoalesceMajorDimCopies(src, dst, sizes, src_c, dst_c, sizes_c);
  const bool is_partial = !src_c.empty();

  std::vector<StorageView> views;
  std::vector<int64_t> full_bytes;
  views.reserve(works.size());
  for (const Work& w : works) {
    const StorageInfo& si = storage(w.layer, w.shard);
    uint8_t* host = si.host;
    int64_t host_size = si.host_bytes;
    if (slot_idx.has_value()) {
      KVX_ASSIGN_OR_RETURN(KVCacheHostSpan span,
                           HostSpan(w.layer, w.shard, *slot_idx,
                                    staging_max_major_per_slot_));
      host = span.ptr;
      host_size = static_cast<int64_t>(span.nbytes);
    }
    const int64_t B = layer_block_bytes(w.layer);
    const int64_t phys = layer_physical_bytes_[w.layer];
    if (!is_partial) {
      if (host == nullptr) {
        return FailedPreconditionError(d2h ? "Destination host pointer is null"
                                           : "Source host pointer is null");
      }
      if (phys > host_size) {
        return d2h ? OutOfRangeError("Copy range exceeds destination host buffer size")
                   : InvalidArgumentError("Source host buffer is too small");
      }
      full_bytes.push_back(phys);
    } else {
      for (size_t j = 0; j < src_c.size(); ++j) {
        const int64_t dev_off = d2h ? src_c[j] : dst_c[j];
        const int64_t host_off = d2h ? dst_c[j] : src_c[j];
        if (d2h) {
          if (!RangeFits(dev_off + sizes_c[j], B, 0, si.dev_bytes)) {
            return InvalidArgumentError("Copy range exceeds source device buffer size");
          }
          if (!RangeFits(host_off + sizes_c[j], B, 0, host_size)) {
            return InvalidArgumentError("Copy range exceeds destination host buffer size");
          }
        } else {
          if (!RangeFits(host_off + sizes_c[j], B, 0, host_size)) {
            return InvalidArgumentError("Copy range exceeds source host buffer size");
          }
          if (!RangeFits(dev_off + sizes_c[j], B, 0, si.dev_bytes)) {
            return InvalidArgumentError(
                "Copy range exceeds destination device buffer size");
          }
        }
      }
    }
    views.push_back(StorageView{si.dev, si.dev_bytes, host, host_size, B,
                                host_kernel_access_});
  }
  if (!is_partial) return engine_->CopyFull(dir, views, full_bytes, dep);
  return engine_->Copy(dir, views, src_c, dst_c, sizes_c, dep);
}

StatusOr<CopyFuture> KVCacheManager::D2h(const std::vector<int64_t>& src,
                                         const std::vector<int64_t>& dst,
                                         const std::vector<int64_t>& sizes,
                                         std::optional<int64_t> slot_idx,
                                         std::optional<size_t> layer_idx,
                                         std::optional<size_t> shard_idx,
                                         hipStream_t dep) {
  if (queued_) {
    return Enqueue(Direction::kD2H, src, dst, sizes, slot_idx, layer_idx, shard_idx, dep);
  }
  return Transfer(Direction::kD2H, src, dst, sizes, slot_idx, layer_idx,
                  shard_idx, dep);
}

StatusOr<CopyFuture> KVCacheManager::H2d(const std::vector<int64_t>& src,
                                         const std::vector<int64_t>& dst,
                                         const std::vector<int64_t>& sizes,
                                         std::optional<int64_t> slot_idx,
                                         std::optional<size_t> layer_idx,
                                         std::optional<size_t> shard_idx,
                                         hipStream_t dep) {
  if (queued_) {
    return Enqueue(Direction::kH2D, src, dst, sizes, slot_idx, layer_idx, shard_idx, dep);
  }
  return Transfer(Direction::kH2D, src, dst, sizes, slot_idx, layer_idx,
                  shard_idx, dep);
}

StatusOr<CopyFuture> KVCacheManager::Enqueue(Direction dir, const std::vector<int64_t>& src,
                                             const std::vector<int64_t>& dst,
                                             const std::vector<int64_t>& sizes,
                                             std::optional<int64_t> slot_idx,
                                             std::optional<size_t> layer_idx,
                                             std::optional<size_t> shard_idx,
                                             hipStream_t dep) {
  QueuedCopy q{dir, src, dst, sizes, slot_idx, layer_idx, shard_idx, nullptr,
               CopyFuture::Pending()};
  if (dep != nullptr && engine_) {
    // The copy is ordered after the work on `dep` at submission time.
    DeviceGuard g(cfg_.device);
    KVX_HIP_RETURN_IF_ERROR(hipEventCreateWithFlags(&q.dep_event, hipEventDisableTiming));
    hipError_t e = hipEventRecord(q.dep_event, dep);
    if (e != hipSuccess) {
      (void)hipEventDestroy(q.dep_event);
      return HipStatus(e, "hipEventRecord(dep)");
    }
  }
  CopyFuture f = q.future;
  {
    std::lock_guard<std::mutex> l(queue_mu_);
    if (shutdown_) {
      if (q.dep_event != nullptr) (void)hipEventDestroy(q.dep_event);
      return CancelledError("KVCacheManagerBase is shutting down");
    }
    queue_.push_back(std::move(q));
  }
  queue_cv_.notify_one();
  return f;
}

void KVCacheManager::WorkerLoop() {
  while (true) {
    QueuedCopy q;
    {
      std::unique_lock<std::mutex> l(queue_mu_);
      queue_cv_.wait(l, [this] { return shutdown_ || !queue_.empty(); });
      if (shutdown_ && queue_.empty()) return;
      q = std::move(queue_.front());
      queue_.pop_front();
    }
    hipStream_t dep = nullptr;
    if (q.dep_event != nullptr) {
      DeviceGuard g(cfg_.device);
      if (hipStreamWaitEvent(dep_proxy_, q.dep_event, 0) == hipSuccess) dep = dep_proxy_;
      (void)hipEventDestroy(q.dep_event);
    }
    StatusOr<CopyFuture> r = Transfer(q.dir, q.src, q.dst, q.sizes, q.slot_idx, q.layer_idx,
                                      q.shard_idx, dep);
    if (r.ok()) {
      q.future.Fulfill(*r);
    } else {
      q.future.Reject(r.status());
    }
  }
}

void KVCacheManager::StopWorker() {
  if (!worker_.joinable()) return;
  {
    std::lock_guard<std::mutex> l(queue_mu_);
    shutdown_ = true;
    // Copies not yet dispatched are cancelled, as the reference's destructor does.
    while (!queue_.empty()) {
      QueuedCopy& q = queue_.front();
      if (q.dep_event != nullptr) (void)hipEventDestroy(q.dep_event);
      q.future.Reject(
          CancelledError("KVCacheManagerBase destroyed before task dispatch completed"));
      queue_.pop_front();
    }
  }
  queue_cv_.notify_all();
  worker_.join();
}

std::string KVCacheManager::DispatchLog() {
  std::lock_guard<std::mutex> l(log_mu_);
  return dispatch_log_;
}

StatusOr<std::pair<std::vector<int>, CopyFuture>>
KVCacheManager::D2hAutoAllocate(const std::vector<int64_t>& src,
                                const std::vector<int64_t>& sizes,
                                hipStream_t dep) {
  // kv_cache_manager_base.cc:1093-1140: allocate sum(sizes) locked host ids,
  // then copy block src[j]+k to the k-th id allocated for chunk j.
  if (src.size() != sizes.size()) {
    return InvalidArgumentError("Lengths of offset and size lists must match");
  }
  int64_t total = 0;
  for (int64_t s : sizes) total += s;
  if (total > std::numeric_limits<int>::max() || total < 0) {
    return InvalidArgumentError("Requested blocks out of range");
  }
  std::vector<int> ids;
  {
    std::lock_guard<std::mutex> l(lbm_mu_);
    KVX_ASSIGN_OR_RETURN(ids, lbm_->Allocate(static_cast<int>(total), /*lock=*/true));
  }
  std::vector<int64_t> fsrc, fdst, fsz;
  fsrc.reserve(total);
  fdst.reserve(total);
  fsz.reserve(total);
  size_t next = 0;
  for (size_t j = 0; j < src.size(); ++j) {
    for (int64_t k = 0; k < sizes[j]; ++k) {
      fsrc.push_back(src[j] + k);
      fdst.push_back(ids[next++]);
      fsz.push_back(1);
    }
  }
  KVX_ASSIGN_OR_RETURN(CopyFuture f, D2h(fsrc, fdst, fsz, std::nullopt,
                                         std::nullopt, std::nullopt, dep));
  return std::make_pair(std::move(ids), std::move(f));
}

StatusOr<CopyFuture> KVCacheManager::DeviceCopy(
    bool gather, const std::vector<int64_t>& ids, uint64_t staging,
    int64_t staging_bytes, bool block_major, std::optional<size_t> layer_idx,
    std::optional<size_t> shard_idx, hipStream_t stream) {
  if (!engine_) {
    return FailedPreconditionError(
        "Gather/Scatter requires a device-backed KVCacheManagerBase");
  }
  KVX_ASSIGN_OR_RETURN(std::vector<Work> works, SelectWorks(layer_idx, shard_idx));
  std::vector<StorageView> views;
  int64_t need = 0;
  for (const Work& w : works) {
    const StorageInfo& si = storage(w.layer, w.shard);
    const int64_t B = layer_block_bytes(w.layer);
    for (int64_t id : ids) {
      if (id < 0) return InvalidArgumentError("block ids must be non-negative");
      if (!RangeFits(id + 1, B, 0, si.dev_bytes)) {
        return OutOfRangeError("block id exceeds device buffer");
      }
    }
    views.push_back(StorageView{si.dev, si.dev_bytes, nullptr, 0, B});
    need += B * static_cast<int64_t>(ids.size());
  }
  if (!gather) {
    // Two staging slots naming one device block would race in the scatter.
    std::vector<int64_t> sorted = ids;
    std::sort(sorted.begin(), sorted.end());
    if (std::adjacent_find(sorted.begin(), sorted.end()) != sorted.end()) {
      return InvalidArgumentError("scatter block ids must be unique");
    }
  }
  if (staging == 0 && need > 0) return InvalidArgumentError("null staging buffer");
  if (staging_bytes < need) {
    return InvalidArgumentError("staging buffer too small: need " +
                                std::to_string(need) + " bytes");
  }
  return engine_->DeviceCopy(gather, views, ids, staging, block_major, stream);
}

StatusOr<CopyFuture> KVCacheManager::Gather(const std::vector<int64_t>& ids,
                                            uint64_t staging,
                                            int64_t staging_bytes,
                                            bool block_major,
                                            std::optional<size_t> layer_idx,
                                            std::optional<size_t> shard_idx,
                                            hipStream_t stream) {
  return DeviceCopy(true, ids, staging, staging_bytes, block_major, layer_idx,
                    shard_idx, stream);
}

StatusOr<CopyFuture> KVCacheManager::Scatter(const std::vector<int64_t>& ids,
                                             uint64_t staging,
                                             int64_t staging_bytes,
                                             bool block_major,
                                             std::optional<size_t> layer_idx,
                                             std::optional<size_t> shard_idx,
                                             hipStream_t stream) {
  return DeviceCopy(false, ids, staging, staging_bytes, block_major, layer_idx,
                    shard_idx, stream);
}

Status KVCacheManager::ConfigureHostStagingSlots(int64_t num_slots,
                                                 int64_t max_major_per_slot) {
  if (num_slots <= 0) return InvalidArgumentError("num_slots must be positive");
  if (max_major_per_slot <= 0) {
    return InvalidArgumentError("max_major_per_slot must be positive");
  }
  staging_num_slots_ = num_slots;
  staging_max_major_per_slot_ = max_major_per_slot;
  return OkStatus();
}

StatusOr<KVCacheHostSpan> KVCacheManager::HostSpan(size_t layer_idx,
                                                   size_t shard_idx,
                                                   int64_t slot_idx,
                                                   int64_t num_major) {
  // kv_cache_manager_base.cc:1434-1466.
  if (staging_num_slots_ <= 0 || staging_max_major_per_slot_ <= 0) {
    return FailedPreconditionError("Host staging slots have not been configured");
  }
  if (slot_idx < 0 || slot_idx >= staging_num_slots_) {
    return OutOfRangeError("slot_idx out of range");
  }
  if (num_major < 0 || num_major > staging_max_major_per_slot_) {
    return OutOfRangeError("num_major out of range");
  }
  if (layer_idx >= static_cast<size_t>(num_layers_) ||
      shard_idx >= static_cast<size_t>(num_shards_)) {
    return OutOfRangeError("HostSpan layer or shard index out of range");
  }
  const int64_t B = layer_block_bytes(layer_idx);
  const int64_t base_major = slot_idx * staging_max_major_per_slot_;
  const size_t byte_offset = static_cast<size_t>(base_major) * B;
  const size_t nbytes = static_cast<size_t>(num_major) * B;
  const StorageInfo& si = storage(layer_idx, shard_idx);
  if (byte_offset + nbytes > static_cast<size_t>(si.host_bytes)) {
    return OutOfRangeError("HostSpan exceeds host staging buffer");
  }
  KVCacheHostSpan span;
  span.ptr = si.host + byte_offset;
  span.nbytes = nbytes;
  span.slot_idx = slot_idx;
  span.base_major = base_major;
  span.num_major = num_major;
  span.layer_idx = layer_idx;
  span.shard_idx = shard_idx;
  return span;
}

uint8_t* KVCacheManager::GetHostPointer(size_t layer_idx, size_t shard_idx) {
  // Shard ids wrap modulo the local shard count
  // (tpu_sync/core/raiden_manager_base.cc:202-230).
  if (layer_idx >= static_cast<size_t>(num_layers_) || num_shards_ == 0) {
    return nullptr;
  }
  return storage(layer_idx, shard_idx % num_shards_).host;
}

size_t KVCacheManager::GetHostSize(size_t layer_idx, size_t shard_idx) {
  if (layer_idx >= static_cast<size_t>(num_layers_) || num_shards_ == 0) return 0;
  return static_cast<size_t>(storage(layer_idx, shard_idx % num_shards_).host_bytes);
}

int64_t KVCacheManager::LayerBlockByteSize(size_t layer_idx) const {
  if (layer_idx >= static_cast<size_t>(num_layers_)) return -1;
  return layer_block_bytes_[layer_idx];
}

size_t KVCacheManager::num_block_arrays() const {
  std::lock_guard<std::mutex> l(pools_mu_);
  return explicit_pools_ ? pools_.size() : static_cast<size_t>(num_layers_);
}

size_t KVCacheManager::block_bytes(size_t block_array_idx) const {
  {
    std::lock_guard<std::mutex> l(pools_mu_);
    if (explicit_pools_) {
      if (block_array_idx >= pools_.size() || pools_[block_array_idx].block_stride_bytes <= 0) {
        return 0;
      }
      return static_cast<size_t>(pools_[block_array_idx].block_stride_bytes);
    }
  }
  const int64_t per_layer = LayerBlockByteSize(block_array_idx);
  if (per_layer > 0) return static_cast<size_t>(per_layer);
  return bytes_per_block();
}

uint8_t* KVCacheManager::GetBlockArrayHostPointer(size_t block_array_idx,
                                                  size_t shard_idx) {
  PoolSpec p;
  {
    std::lock_guard<std::mutex> l(pools_mu_);
    if (!explicit_pools_) return GetHostPointer(block_array_idx, shard_idx);
    if (block_array_idx >= pools_.size()) return nullptr;
    p = pools_[block_array_idx];
  }
  uint8_t* base = GetHostPointer(p.storage_index, shard_idx);
  return base == nullptr ? nullptr : base + p.base_offset_bytes;
}

size_t KVCacheManager::GetBlockArrayHostSize(size_t block_array_idx,
                                             size_t shard_idx) {
  PoolSpec p;
  {
    std::lock_guard<std::mutex> l(pools_mu_);
    if (!explicit_pools_) return GetHostSize(block_array_idx, shard_idx);
    if (block_array_idx >= pools_.size()) return 0;
    p = pools_[block_array_idx];
  }
  const size_t storage = GetHostSize(p.storage_index, shard_idx);
  const int64_t end = p.storage_extent_end_bytes();
  if (end < p.base_offset_bytes || static_cast<uint64_t>(end) > storage ||
      static_cast<size_t>(p.base_offset_bytes) > storage) {
    return 0;
  }
  return static_cast<size_t>(end - p.base_offset_bytes);
}

uint8_t* KVCacheManager::GetBlockHostPointer(size_t block_array_idx, size_t shard_idx,
                                             int64_t block_id) {
  {
    std::lock_guard<std::mutex> l(pools_mu_);
    if (explicit_pools_ && (block_array_idx >= pools_.size() || block_id < 0 ||
                            block_id >= pools_[block_array_idx].num_blocks)) {
      return nullptr;
    }
  }
  uint8_t* base = GetBlockArrayHostPointer(block_array_idx, shard_idx);
  if (base == nullptr || block_id < 0) return nullptr;
  return base + static_cast<size_t>(block_id) * block_bytes(block_array_idx);
}

std::vector<KVCacheManager::BlockChunk> KVCacheManager::GetBlockChunks(
    size_t block_array_idx, size_t shard_idx, const std::vector<int64_t>& block_ids,
    size_t total_bytes) {
  std::vector<BlockChunk> chunks;
  size_t acc = 0;
  PoolSpec p;
  bool pools = false;
  {
    std::lock_guard<std::mutex> l(pools_mu_);
    pools = explicit_pools_;
    if (pools) {
      if (block_array_idx >= pools_.size()) return {};
      p = pools_[block_array_idx];
    }
  }
  if (pools) {
    for (int64_t id : block_ids) {
      if (id < 0 || id >= p.num_blocks) return {};
    }
    uint8_t* storage_base = GetHostPointer(p.storage_index, shard_idx);
    if (storage_base == nullptr) return {};
    for (int64_t id : block_ids) {
      if (acc >= total_bytes) break;
      StatusOr<std::vector<PoolBlockCopyExtent>> ext = ComputePoolBlockCopyExtents(p, {id});
      if (!ext.ok()) return {};
      for (const PoolBlockCopyExtent& e : *ext) {
        if (acc >= total_bytes) break;
        const size_t size = std::min(static_cast<size_t>(e.size_bytes), total_bytes - acc);
        chunks.push_back(BlockChunk{storage_base + e.offset_bytes, size});
        acc += size;
      }
    }
    return chunks;
  }
  const size_t bb = block_bytes(block_array_idx);
  for (int64_t id : block_ids) {
    if (acc >= total_bytes) break;
    const size_t size = std::min(bb, total_bytes - acc);
    chunks.push_back(BlockChunk{GetBlockHostPointer(block_array_idx, shard_idx, id), size});
    acc += size;
  }
  return chunks;
}

StatusOr<uintptr_t> KVCacheManager::GetBlockHostPointerValue(size_t layer_idx,
                                                             size_t shard_idx,
                                                             int block_id) {
  if (block_id < 0) return InvalidArgumentError("block_id must be non-negative");
  const size_t bb = block_bytes(layer_idx);
  const size_t host_size = GetHostSize(layer_idx, shard_idx);
  uint8_t* base = GetHostPointer(layer_idx, shard_idx);
  if (base == nullptr) return OutOfRangeError("layer or shard index out of range");
  const size_t block = static_cast<size_t>(block_id);
  if (bb == 0 || block > host_size / bb || block * bb + bb > host_size) {
    return OutOfRangeError("block range exceeds host buffer");
  }
  return reinterpret_cast<uintptr_t>(base + block * bb);
}

StatusOr<std::string> KVCacheManager::ReadBlockBytes(size_t layer_idx,
                                                     int block_id,
                                                     size_t shard_idx) {
  KVX_ASSIGN_OR_RETURN(uintptr_t p,
                       GetBlockHostPointerValue(layer_idx, shard_idx, block_id));
  return std::string(reinterpret_cast<const char*>(p), block_bytes(layer_idx));
}

Status KVCacheManager::WriteBlockBytes(size_t layer_idx, int block_id,
                                       const void* payload, size_t payload_size,
                                       size_t shard_idx) {
  if (block_id < 0) return InvalidArgumentError("block_id must be non-negative");
  const size_t bb = block_bytes(layer_idx);
  if (payload_size != bb) {
    return InvalidArgumentError("payload size must equal block size: got " +
                                std::to_string(payload_size) + ", expected " +
                                std::to_string(bb));
  }
  KVX_ASSIGN_OR_RETURN(uintptr_t p,
                       GetBlockHostPointerValue(layer_idx, shard_idx, block_id));
  std::memcpy(reinterpret_cast<void*>(p), payload, bb);
  return OkStatus();
}

void KVCacheManager::EnsureImplicitPoolsLocked() {
  if (explicit_pools_ || !pools_.empty()) return;
  for (int64_t l = 0; l < num_layers_; ++l) {
    const int64_t stride = LayerBlockByteSize(static_cast<size_t>(l));
    if (stride <= 0) continue;
    const int64_t nb = static_cast<int64_t>(GetHostSize(static_cast<size_t>(l), 0)) / stride;
    if (nb <= 0) continue;
    PoolSpec p;
    p.tag = "opaque";
    p.storage_index = static_cast<size_t>(l);
    p.block_stride_bytes = stride;
    p.num_blocks = nb;
    RegionSpec r;
    r.name = "block";
    r.stride_bytes = stride;
    r.unit_bytes = stride;
    r.num_units = 1;
    p.regions.push_back(std::move(r));
    pools_.push_back(std::move(p));
  }
}

Status KVCacheManager::EnsureHostMirrorCovers(size_t storage_idx, int64_t needed_bytes) {
  if (storage_idx >= static_cast<size_t>(num_layers_) || needed_bytes <= 0) return OkStatus();
  for (int64_t s = 0; s < num_shards_; ++s) {
    StorageInfo& si = storage(storage_idx, static_cast<size_t>(s));
    if (si.host_bytes >= needed_bytes) continue;
    if (cfg_.host_alloc == HostAllocKind::kShm) {
      // Mirrors are carved out of one fixed shared-memory segment.
      return FailedPreconditionError(
          "shared-memory host mirror cannot grow to cover pool: storage " +
          std::to_string(storage_idx) + " needs " + std::to_string(needed_bytes) +
          " bytes, has " + std::to_string(si.host_bytes));
    }
    const size_t want = static_cast<size_t>(needed_bytes);
    StatusOr<HostBufferAllocation> a =
        cfg_.host_alloc == HostAllocKind::kPinned
            ? AllocatePinnedHost(want, cfg_.device, numa_node_)
            : AllocateMallocHost(want, numa_node_);
    if (!a.ok()) return a.status();
    if (a->ptr == nullptr || a->size < want) {
      return InternalError(
          "host allocator returned undersized buffer for pool mirror: requested=" +
          std::to_string(want));
    }
    // Copies in flight may still read or write the old mirror.
    KVX_RETURN_IF_ERROR(WaitForPendingWork());
    if (si.host != nullptr && si.host_bytes > 0) {
      std::memcpy(a->ptr, si.host, static_cast<size_t>(si.host_bytes));
    }
    allocated_host_bytes_ = allocated_host_bytes_ - static_cast<size_t>(si.host_bytes) + a->size;
    si.host = a->ptr;
    si.host_bytes = static_cast<int64_t>(a->size);
    si.host_owner = a->owner;
  }
  return OkStatus();
}

Status KVCacheManager::RegisterPools(std::vector<PoolSpec> pools) {
  if (pools.empty()) return InvalidArgumentError("pool table must be non-empty");
  const bool dev = engine_ != nullptr;
  for (size_t i = 0; i < pools.size(); ++i) {
    const PoolSpec& p = pools[i];
    if (p.storage_index >= static_cast<size_t>(num_layers_)) {
      return InvalidArgumentError("pool " + std::to_string(i) + " (" + p.tag +
                                  ") storage_index " + std::to_string(p.storage_index) +
                                  " out of range: manager wraps " +
                                  std::to_string(num_layers_) + " storages");
    }
    // The device storage bounds a device-backed pool; the host mirror (the
    // storage itself) bounds a host-only one; -1 checks geometry only.
    int64_t storage_bytes = -1;
    if (dev && layer_physical_bytes_[p.storage_index] > 0) {
      storage_bytes = layer_physical_bytes_[p.storage_index];
    } else if (GetHostSize(p.storage_index, 0) > 0) {
      storage_bytes = static_cast<int64_t>(GetHostSize(p.storage_index, 0));
    }
    Status st = p.Validate(storage_bytes);
    if (!st.ok()) {
      return InvalidArgumentError("invalid pool " + std::to_string(i) + ": " + st.message());
    }
    if (dev) KVX_RETURN_IF_ERROR(EnsureHostMirrorCovers(p.storage_index,
                                                        p.storage_extent_end_bytes()));
  }
  std::lock_guard<std::mutex> l(pools_mu_);
  pools_ = std::move(pools);
  explicit_pools_ = true;
  return OkStatus();
}

StatusOr<PoolBlockRef> KVCacheManager::GetPoolBlockRef(size_t pool_idx, size_t shard_idx,
                                                       int64_t block_id) {
  std::lock_guard<std::mutex> l(pools_mu_);
  EnsureImplicitPoolsLocked();
  if (pool_idx >= pools_.size()) {
    return OutOfRangeError("pool index " + std::to_string(pool_idx) +
                           " out of range: " + std::to_string(pools_.size()) + " pools");
  }
  if (block_id < 0) return InvalidArgumentError("block_id must be non-negative");
  const PoolSpec& p = pools_[pool_idx];
  if (p.storage_index >= static_cast<size_t>(num_layers_) ||
      shard_idx >= static_cast<size_t>(num_shards_)) {
    return OutOfRangeError("storage or shard index out of range");
  }
  const StorageInfo& si = storage(p.storage_index, shard_idx);
  if (si.host == nullptr) return FailedPreconditionError("host pointer is null");
  if (block_id >= p.num_blocks) {
    return OutOfRangeError("block_id " + std::to_string(block_id) + " out of range for pool " +
                           std::to_string(pool_idx) + " (" + p.tag +
                           "): num_blocks=" + std::to_string(p.num_blocks));
  }
  const int64_t off = p.base_offset_bytes + block_id * p.block_stride_bytes;
  int64_t live_end = 0;
  for (const RegionSpec& r : p.regions) live_end = std::max(live_end, r.extent_end_bytes());
  if (off > si.host_bytes || live_end > si.host_bytes - off) {
    return OutOfRangeError("block live regions exceed host buffer");
  }
  PoolBlockRef ref;
  ref.ptr = si.host + off;
  ref.block_stride_bytes = p.block_stride_bytes;
  ref.pool_idx = pool_idx;
  ref.shard_idx = shard_idx;
  ref.block_id = block_id;
  return ref;
}

StatusOr<PoolSpec> KVCacheManager::pool_spec(size_t pool_idx) {
  std::lock_guard<std::mutex> l(pools_mu_);
  EnsureImplicitPoolsLocked();
  if (pool_idx >= pools_.size()) {
    return OutOfRangeError("pool index out of range: " + std::to_string(pool_idx));
  }
  return pools_[pool_idx];
}

size_t KVCacheManager::num_pools() {
  std::lock_guard<std::mutex> l(pools_mu_);
  EnsureImplicitPoolsLocked();
  return pools_.size();
}

bool KVCacheManager::has_explicit_pools() {
  std::lock_guard<std::mutex> l(pools_mu_);
  return explicit_pools_;
}

std::vector<size_t> KVCacheManager::PoolIndicesWithTag(const std::string& tag) {
  std::lock_guard<std::mutex> l(pools_mu_);
  EnsureImplicitPoolsLocked();
  std::vector<size_t> out;
  for (size_t i = 0; i < pools_.size(); ++i) {
    if (pools_[i].tag == tag) out.push_back(i);
  }
  return out;
}

StatusOr<CopyFuture> KVCacheManager::CopyPoolBlocks(size_t pool_idx,
                                                    const std::vector<int64_t>& block_ids,
                                                    std::optional<size_t> shard_idx,
                                                    bool d2h, hipStream_t dep) {
  PoolSpec p;
  {
    std::lock_guard<std::mutex> l(pools_mu_);
    EnsureImplicitPoolsLocked();
    if (pool_idx >= pools_.size()) {
      return OutOfRangeError("pool index " + std::to_string(pool_idx) +
                             " out of range: " + std::to_string(pools_.size()) + " pools");
    }
    p = pools_[pool_idx];
  }
  if (!engine_ || p.storage_index >= static_cast<size_t>(num_layers_)) {
    return FailedPreconditionError("pool storage has no device buffers (host-only manager)");
  }
  if (shard_idx.has_value() && *shard_idx >= static_cast<size_t>(num_shards_)) {
    return OutOfRangeError("shard index out of range");
  }
  KVX_ASSIGN_OR_RETURN(std::vector<PoolBlockCopyExtent> extents,
                       ComputePoolBlockCopyExtents(p, block_ids));
  std::vector<StorageView> views;
  for (int64_t s = 0; s < num_shards_; ++s) {
    if (shard_idx.has_value() && static_cast<size_t>(s) != *shard_idx) continue;
    const StorageInfo& si = storage(p.storage_index, static_cast<size_t>(s));
    if (si.host == nullptr) return FailedPreconditionError("host pointer is null");
    for (const PoolBlockCopyExtent& e : extents) {
      const int64_t end = e.offset_bytes + e.size_bytes;
      if (end > si.host_bytes) {
        return OutOfRangeError("pool block copy exceeds host buffer size");
      }
      if (end > si.dev_bytes) {
        return OutOfRangeError("pool block copy exceeds device buffer size");
      }
    }
    views.push_back(StorageView{si.dev, si.dev_bytes, si.host, si.host_bytes,
                                layer_block_bytes(p.storage_index), host_kernel_access_});
  }
  std::vector<ByteExtent> ext;
  ext.reserve(extents.size());
  for (const PoolBlockCopyExtent& e : extents) ext.push_back({e.offset_bytes, e.size_bytes});
  return engine_->CopyExtents(d2h ? Direction::kD2H : Direction::kH2D, views, ext, dep);
}

StatusOr<CopyFuture> KVCacheManager::D2hPoolBlocks(size_t pool_idx,
                                                   const std::vector<int64_t>& block_ids,
                                                   std::optional<size_t> shard_idx,
                                                   hipStream_t dep) {
  return CopyPoolBlocks(pool_idx, block_ids, shard_idx, true, dep);
}

StatusOr<CopyFuture> KVCacheManager::H2dPoolBlocks(size_t pool_idx,
                                                   const std::vector<int64_t>& block_ids,
                                                   std::optional<size_t> shard_idx,
                                                   hipStream_t dep) {
  return CopyPoolBlocks(pool_idx, block_ids, shard_idx, false, dep);
}

Status KVCacheManager::InitializeSlotPool(int64_t num_slots) {
  if (num_slots <= 0) return InvalidArgumentError("num_slots must be positive");
  if (staging_max_major_per_slot_ <= 0) {
    return FailedPreconditionError("host staging slots are not configured");
  }
  const int64_t max_blocks = staging_max_major_per_slot_;
  std::lock_guard<std::mutex> sl(slots_mu_);
  std::lock_guard<std::mutex> bl(lbm_mu_);
  if (lbm_->num_free_blocks() < num_slots * max_blocks) {
    return FailedPreconditionError(
        "Insufficient free host blocks to initialize slot pool. Required: " +
        std::to_string(num_slots * max_blocks) +
        ", Available: " + std::to_string(lbm_->num_free_blocks()));
  }
  // Slots of an earlier pool go back to the block manager.
  for (const StagingSlot& s : all_slots_) {
    std::vector<int> ids(s.block_ids.begin(), s.block_ids.end());
    KVX_RETURN_IF_ERROR(lbm_->Unlock(ids));
    KVX_RETURN_IF_ERROR(lbm_->Deallocate(ids));
  }
  all_slots_.clear();
  free_slots_.clear();
  for (int64_t i = 0; i < num_slots; ++i) {
    KVX_ASSIGN_OR_RETURN(std::vector<int> ids,
                         lbm_->Allocate(static_cast<int>(max_blocks), /*lock=*/true));
    if (static_cast<int64_t>(ids.size()) != max_blocks) {
      return InternalError("Slot pool allocation returned incorrect number of blocks: " +
                           std::to_string(ids.size()) + ", expected: " +
                           std::to_string(max_blocks));
    }
    all_slots_.push_back(StagingSlot{i, std::vector<int64_t>(ids.begin(), ids.end())});
    free_slots_.push_back(i);
  }
  return OkStatus();
}

StatusOr<StagingSlot> KVCacheManager::AcquireSlot() {
  std::lock_guard<std::mutex> l(slots_mu_);
  if (free_slots_.empty()) return ResourceExhaustedError("Raiden host slot pool exhausted");
  const int64_t i = free_slots_.front();
  free_slots_.pop_front();
  return all_slots_[static_cast<size_t>(i)];
}

void KVCacheManager::ReleaseSlot(int64_t slot_idx) {
  std::lock_guard<std::mutex> l(slots_mu_);
  if (slot_idx < 0 || slot_idx >= static_cast<int64_t>(all_slots_.size())) return;
  free_slots_.push_back(slot_idx);
}

int64_t KVCacheManager::num_free_slots() {
  std::lock_guard<std::mutex> l(slots_mu_);
  return static_cast<int64_t>(free_slots_.size());
}

StatusOr<std::vector<int64_t>> KVCacheManager::SlotBlockIds(int64_t slot_idx) {
  std::lock_guard<std::mutex> l(slots_mu_);
  if (slot_idx < 0 || slot_idx >= static_cast<int64_t>(all_slots_.size())) {
    return OutOfRangeError("slot_idx out of range");
  }
  return all_slots_[static_cast<size_t>(slot_idx)].block_ids;
}

StatusOr<std::vector<KVCacheHostSpan>> KVCacheManager::LayerSpans(int64_t slot_idx,
                                                                  int64_t num_blocks) {
  if (num_layers_ == 0) return FailedPreconditionError("KV cache manager is not registered");
  KVX_ASSIGN_OR_RETURN(std::vector<int64_t> ids, SlotBlockIds(slot_idx));
  if (num_blocks < 0 || num_blocks > static_cast<int64_t>(ids.size())) {
    return OutOfRangeError("num_blocks out of range");
  }
  ids.resize(static_cast<size_t>(num_blocks));
  const CopySpec runs = OffsetsImpl(ids, /*source_is_compact=*/false);
  std::vector<KVCacheHostSpan> spans;
  spans.reserve(static_cast<size_t>(num_layers_ * num_shards_) * runs.sizes.size());
  for (int64_t l = 0; l < num_layers_; ++l) {
    const int64_t per_layer = LayerBlockByteSize(static_cast<size_t>(l));
    const int64_t bytes = per_layer > 0 ? per_layer : slice_byte_size_;
    for (int64_t s = 0; s < num_shards_; ++s) {
      const StorageInfo& si = storage(static_cast<size_t>(l), static_cast<size_t>(s));
      for (size_t r = 0; r < runs.sizes.size(); ++r) {
        KVCacheHostSpan span;
        span.ptr = si.host + runs.src_offsets[r] * bytes;
        span.nbytes = static_cast<size_t>(runs.sizes[r] * bytes);
        span.slot_idx = slot_idx;
        span.base_major = runs.src_offsets[r];
        span.num_major = runs.sizes[r];
        span.layer_idx = static_cast<size_t>(l);
        span.shard_idx = static_cast<size_t>(s);
        spans.push_back(span);
      }
    }
  }
  return spans;
}

StatusOr<StageResult> KVCacheManager::IssueH2D(int64_t slot_idx, int64_t num_blocks,
                                               const std::vector<int64_t>& local_block_ids,
                                               hipStream_t dep) {
  if (num_layers_ == 0) return FailedPreconditionError("KV cache manager is not registered");
  std::vector<int64_t> host_ids;
  {
    std::lock_guard<std::mutex> l(slots_mu_);
    if (slot_idx < 0 || slot_idx >= static_cast<int64_t>(all_slots_.size())) {
      return OutOfRangeError("slot_idx out of range");
    }
    host_ids = all_slots_[static_cast<size_t>(slot_idx)].block_ids;
  }
  if (num_blocks < 0 || num_blocks > static_cast<int64_t>(host_ids.size())) {
    return OutOfRangeError("num_blocks out of range");
  }
  if (num_blocks != static_cast<int64_t>(local_block_ids.size())) {
    return InvalidArgumentError("num_blocks must match len(local_block_ids)");
  }
  host_ids.resize(static_cast<size_t>(num_blocks));
  KVX_ASSIGN_OR_RETURN(CopySpec spec, BuildCoalescedCopySpec(host_ids, local_block_ids));
  StageResult r;
  KVX_ASSIGN_OR_RETURN(r.host_spans, LayerSpans(slot_idx, num_blocks));
  for (const KVCacheHostSpan& s : r.host_spans) r.total_bytes += static_cast<int64_t>(s.nbytes);
  r.copy_segments = static_cast<int64_t>(spec.sizes.size());
  if (spec.sizes.empty()) return r;
  // The reference issues through H2dSyncDispatch here, whatever the dispatch mode.
  KVX_ASSIGN_OR_RETURN(r.future, Transfer(Direction::kH2D, spec.src_offsets, spec.dst_offsets,
                                          spec.sizes, std::nullopt, std::nullopt,
                                          std::nullopt, dep));
  return r;
}

StatusOr<PushStage> KVCacheManager::StageForPush(const std::vector<int64_t>& src_block_ids,
                                                 hipStream_t dep) {
  if (num_layers_ == 0) return FailedPreconditionError("KV cache manager is not registered");
  if (static_cast<int64_t>(src_block_ids.size()) > staging_max_major_per_slot_) {
    return InvalidArgumentError("push of " + std::to_string(src_block_ids.size()) +
                                " blocks exceeds the slot size " +
                                std::to_string(staging_max_major_per_slot_));
  }
  KVX_ASSIGN_OR_RETURN(StagingSlot slot, AcquireSlot());
  PushStage st;
  st.slot_idx = slot.slot_idx;
  st.host_block_ids.assign(slot.block_ids.begin(),
                           slot.block_ids.begin() + static_cast<int64_t>(src_block_ids.size()));
  auto fail = [&](const Status& s) {
    for (const CopyFuture& f : st.layer_futures) (void)f.Await();
    ReleaseSlot(slot.slot_idx);
    return s;
  };
  StatusOr<CopySpec> spec = BuildCoalescedCopySpec(src_block_ids, st.host_block_ids);
  if (!spec.ok()) return fail(spec.status());
  st.copy_segments = static_cast<int64_t>(spec->sizes.size());
  if (spec->sizes.empty()) return st;
  for (int64_t l = 0; l < num_layers_; ++l) {
    StatusOr<CopyFuture> f =
        Transfer(Direction::kD2H, spec->src_offsets, spec->dst_offsets, spec->sizes,
                 std::nullopt, static_cast<size_t>(l), std::nullopt, dep);
    if (!f.ok()) return fail(f.status());
    st.layer_futures.push_back(*f);
  }
  return st;
}

StatusOr<LoadStage> KVCacheManager::PrepareLoad(
    const std::vector<int64_t>& remote_block_ids, const std::vector<int64_t>& local_block_ids,
    const std::vector<int64_t>* local_host_block_ids) {
  LoadStage st;
  if (local_host_block_ids != nullptr) {
    st.host_block_ids = *local_host_block_ids;
  } else if (!local_block_ids.empty()) {
    std::vector<int64_t> distinct = local_block_ids;
    std::sort(distinct.begin(), distinct.end());
    distinct.erase(std::unique(distinct.begin(), distinct.end()), distinct.end());
    if (static_cast<int64_t>(distinct.size()) > staging_max_major_per_slot_) {
      return ResourceExhaustedError("load of " + std::to_string(distinct.size()) +
                                    " distinct blocks exceeds the slot size " +
                                    std::to_string(staging_max_major_per_slot_));
    }
    KVX_ASSIGN_OR_RETURN(StagingSlot slot, AcquireSlot());
    st.slot_idx = slot.slot_idx;
    // First occurrence of each local id takes the next host id of the slot.
    std::vector<std::pair<int64_t, int64_t>> assigned;  // (local, host), by local
    size_t next = 0;
    for (int64_t local : local_block_ids) {
      auto it = std::lower_bound(assigned.begin(), assigned.end(),
                                 std::make_pair(local, INT64_MIN));
      if (it != assigned.end() && it->first == local) {
        st.host_block_ids.push_back(it->second);
        continue;
      }
      const int64_t host = slot.block_ids[next++];
      assigned.insert(it, {local, host});
      st.host_block_ids.push_back(host);
    }
  }
  StatusOr<CopyPlan> plan =
      BuildLoadCopyPlan(remote_block_ids, local_block_ids, st.host_block_ids);
  if (!plan.ok()) {
    if (st.slot_idx >= 0) ReleaseSlot(st.slot_idx);
    return plan.status();
  }
  st.plan = std::move(*plan);
  return st;
}

}  // namespace kvx
