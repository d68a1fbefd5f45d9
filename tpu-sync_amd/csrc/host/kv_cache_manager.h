// Paged KV manager for one MI355X: the counterpart of the reference's
// KVCacheManagerBase (tpu_sync/kv_cache/kv_cache_manager_base.h:111-599).
//
// It wraps per-(layer, shard) device buffers of shape [major_dim][...]
// (borrowed; the caller keeps them alive) and owns a host mirror with the
// same per-(layer, shard) layout, [host_blocks][block bytes]. D2h/H2d move
// whole blocks addressed by major-dimension offsets between the two and
// return a CopyFuture; an empty spec copies the whole layer. Offsets are
// validated and coalesced exactly as the reference does
// (kv_cache_manager_base.cc:72-141) and every range is checked before any
// copy is issued. Device data moves through TransferEngine (gather/scatter
// kernels + pipelined hipMemcpyAsync) instead of one DMA per run.
#ifndef KVX_HOST_KV_CACHE_MANAGER_H_
#define KVX_HOST_KV_CACHE_MANAGER_H_

#include <hip/hip_runtime_api.h>

#include <condition_variable>
#include <cstdint>
#include <deque>
#include <memory>
#include <mutex>
#include <optional>
#include <string>
#include <thread>
#include <utility>
#include <vector>

#include "copy_future.h"
#include "copy_plan.h"
#include "host_allocator.h"
#include "logical_block_manager.h"
#include "pool_layout.h"
#include "status.h"
#include "transfer_engine.h"

namespace kvx {

struct ManagerConfig {
  int device = 0;
  int64_t num_layers = 0;
  int64_t num_shards = 1;
  // Device base address of each (layer, shard) buffer, index
  // layer * num_shards + shard. Empty: a CPU-only manager (host mirror only),
  // like the reference's CPU-only constructor (kv_cache_manager_base.cc:374-450).
  std::vector<uint64_t> device_ptrs;
  std::vector<int64_t> device_bytes;  // bytes of each device buffer
  int64_t major_dim = 0;              // blocks along the major dimension
  // Bytes per block; required for a CPU-only manager, otherwise derived from
  // layer 0 (device bytes / major_dim) when 0.
  int64_t slice_byte_size = 0;
  int64_t host_blocks = 64;
  HostAllocKind host_alloc = HostAllocKind::kPinned;
  // Used when host_alloc == kShm.
  std::string shm_key;
  std::string shm_server_name;
  std::string model_uid;
  // Host mirror placement: kAuto prefers the GPU's NUMA node (device-backed
  // managers), kOff leaves placement to the OS, kNode prefers numa_node.
  enum class Numa : int { kAuto = 0, kOff = 1, kNode = 2 };
  Numa numa = Numa::kAuto;
  int numa_node = -1;
  // D2h/H2d dispatch (kv_cache_manager_base.cc:452-512): kEnv follows
  // RAIDEN_ENABLE_ASYNC_DISPATCH=1; kQueued plans and issues every copy on
  // one background thread in submission order and returns at once (errors,
  // validation included, then arrive through the future).
  enum class Dispatch : int { kEnv = 0, kQueued = 1, kInline = 2 };
  Dispatch dispatch = Dispatch::kEnv;
  EngineOptions engine;
};

// A contiguous host range of one (layer, shard) staging slot
// (kv_cache_manager_base.h KVCacheHostSpan).
struct KVCacheHostSpan {
  uint8_t* ptr = nullptr;
  size_t nbytes = 0;
  int64_t slot_idx = -1;
  int64_t base_major = 0;
  int64_t num_major = 0;
  size_t layer_idx = 0;
  size_t shard_idx = 0;
};

// One staging slot: max_blocks host block ids reserved (locked) in the host
// block manager (kv_cache_manager_with_transfer.h Slot).
struct StagingSlot {
  int64_t slot_idx = -1;
  std::vector<int64_t> block_ids;
};

// kv_cache_manager_with_transfer.h:120-128 StageResult.
struct StageResult {
  CopyFuture future;
  std::vector<KVCacheHostSpan> host_spans;
  int64_t total_bytes = 0;
  int64_t copy_segments = 0;
};

// The D2H half of a push: the device blocks staged into a slot's host ids,
// one future per layer so each layer can be sent as soon as it lands.
struct PushStage {
  int64_t slot_idx = -1;
  std::vector<int64_t> host_block_ids;
  std::vector<CopyFuture> layer_futures;
  int64_t copy_segments = 0;
};

// The receive half: host ids assigned to the local ids and the load plan.
struct LoadStage {
  int64_t slot_idx = -1;  // -1 when the caller supplied the host ids
  std::vector<int64_t> host_block_ids;
  CopyPlan plan;
};

// A host-side pool block (kv_cache_manager_base.h PoolBlockRef): the block's
// first byte in the host mirror of one shard.
struct PoolBlockRef {
  uint8_t* ptr = nullptr;
  int64_t block_stride_bytes = 0;
  size_t pool_idx = 0;
  size_t shard_idx = 0;
  int64_t block_id = 0;
};

class KVCacheManager {
 public:
  static StatusOr<std::unique_ptr<KVCacheManager>> Create(ManagerConfig cfg);
  ~KVCacheManager();

  StatusOr<CopyFuture> D2h(const std::vector<int64_t>& src_offsets_major_dim,
                           const std::vector<int64_t>& dst_offsets_major_dim,
                           const std::vector<int64_t>& copy_sizes_major_dim,
                           std::optional<int64_t> slot_idx = std::nullopt,
                           std::optional<size_t> layer_idx = std::nullopt,
                           std::optional<size_t> shard_idx = std::nullopt,
                           hipStream_t dep = nullptr);
  StatusOr<CopyFuture> H2d(const std::vector<int64_t>& src_offsets_major_dim,
                           const std::vector<int64_t>& dst_offsets_major_dim,
                           const std::vector<int64_t>& copy_sizes_major_dim,
                           std::optional<int64_t> slot_idx = std::nullopt,
                           std::optional<size_t> layer_idx = std::nullopt,
                           std::optional<size_t> shard_idx = std::nullopt,
                           hipStream_t dep = nullptr);
  StatusOr<std::pair<std::vector<int>, CopyFuture>> D2hAutoAllocate(
      const std::vector<int64_t>& src_offsets_major_dim,
      const std::vector<int64_t>& copy_sizes_major_dim,
      hipStream_t dep = nullptr);

  // Device-side extract/insert: gathers blocks `ids` of the selected
  // storages into a device staging buffer (or scatters them back). Staging
  // is layer-major [storage][n][block] or block-major [n][storage][block];
  // storages are (layer, shard) in layer-major order, optionally restricted
  // to one layer and/or one shard.
  StatusOr<CopyFuture> Gather(const std::vector<int64_t>& ids, uint64_t staging,
                              int64_t staging_bytes, bool block_major,
                              std::optional<size_t> layer_idx,
                              std::optional<size_t> shard_idx,
                              hipStream_t stream);
  StatusOr<CopyFuture> Scatter(const std::vector<int64_t>& ids,
                               uint64_t staging, int64_t staging_bytes,
                               bool block_major,
                               std::optional<size_t> layer_idx,
                               std::optional<size_t> shard_idx,
                               hipStream_t stream);

  Status ConfigureHostStagingSlots(int64_t num_slots,
                                   int64_t max_major_per_slot);
  StatusOr<KVCacheHostSpan> HostSpan(size_t layer_idx, size_t shard_idx,
                                     int64_t slot_idx, int64_t num_major);

  // Staging-slot pool (kv_cache_manager_with_transfer.cc:1751-1916):
  // num_slots slots of max_major_per_slot host ids each, allocated locked
  // from the host block manager once ConfigureHostStagingSlots has set the
  // slot size. Slots are handed out first-in first-out.
  Status InitializeSlotPool(int64_t num_slots);
  StatusOr<StagingSlot> AcquireSlot();
  void ReleaseSlot(int64_t slot_idx);
  int64_t num_free_slots();
  StatusOr<std::vector<int64_t>> SlotBlockIds(int64_t slot_idx);
  // Per-(layer, shard) contiguous host runs of the slot's first num_blocks
  // host ids, layer-major.
  StatusOr<std::vector<KVCacheHostSpan>> LayerSpans(int64_t slot_idx, int64_t num_blocks);
  // Host ids slot.block_ids[0..n) -> device ids local_block_ids, coalesced.
  StatusOr<StageResult> IssueH2D(int64_t slot_idx, int64_t num_blocks,
                                 const std::vector<int64_t>& local_block_ids,
                                 hipStream_t dep = nullptr);
  // Acquires a slot and copies device blocks src_block_ids into its host ids
  // layer by layer (StartPushInternal, :2253-2335). The caller releases the
  // slot once the staged bytes have been consumed.
  StatusOr<PushStage> StageForPush(const std::vector<int64_t>& src_block_ids,
                                   hipStream_t dep = nullptr);
  // Host ids for a receive (StartRead, :1520-1565): the caller's, or a slot
  // acquired here with one host id per distinct local id; then the load plan.
  StatusOr<LoadStage> PrepareLoad(const std::vector<int64_t>& remote_block_ids,
                                  const std::vector<int64_t>& local_block_ids,
                                  const std::vector<int64_t>* local_host_block_ids);

  // Host block accessors (kv_cache_manager_base.cc:1468-1552,
  // tpu_sync/frameworks/torch/kv_cache_manager.cc:224-267).
  StatusOr<uintptr_t> GetBlockHostPointerValue(size_t layer_idx,
                                               size_t shard_idx, int block_id);
  StatusOr<std::string> ReadBlockBytes(size_t layer_idx, int block_id,
                                       size_t shard_idx);
  Status WriteBlockBytes(size_t layer_idx, int block_id, const void* payload,
                         size_t payload_size, size_t shard_idx);
  uint8_t* GetHostPointer(size_t layer_idx, size_t shard_idx);
  size_t GetHostSize(size_t layer_idx, size_t shard_idx);

  // Pool table over the wrapped storages (storage index = layer)
  // (kv_cache_manager_base.cc:1554-1872). Until RegisterPools succeeds each
  // storage is one implicit pool tagged "opaque" whose single region
  // "block" covers a whole block, with as many blocks as the host mirror
  // holds. RegisterPools validates every pool against its device storage
  // (or host mirror for a host-only manager) and grows a device-backed
  // storage's host mirror to cover the pool's last live byte, since pool
  // offsets address the device buffer and the mirror alike.
  Status RegisterPools(std::vector<PoolSpec> pools);
  StatusOr<PoolBlockRef> GetPoolBlockRef(size_t pool_idx, size_t shard_idx,
                                         int64_t block_id);
  StatusOr<PoolSpec> pool_spec(size_t pool_idx);
  size_t num_pools();
  bool has_explicit_pools();
  std::vector<size_t> PoolIndicesWithTag(const std::string& tag);
  // Copies the live bytes of pool blocks `block_ids` (padding skipped,
  // extents coalesced) between the device storage and the host mirror, at
  // the same byte offsets on both sides, for every shard or one.
  StatusOr<CopyFuture> D2hPoolBlocks(size_t pool_idx,
                                     const std::vector<int64_t>& block_ids,
                                     std::optional<size_t> shard_idx,
                                     hipStream_t dep = nullptr);
  StatusOr<CopyFuture> H2dPoolBlocks(size_t pool_idx,
                                     const std::vector<int64_t>& block_ids,
                                     std::optional<size_t> shard_idx,
                                     hipStream_t dep = nullptr);

  LogicalBlockManager* host_block_manager() const { return lbm_.get(); }
  std::mutex& host_block_mutex() { return lbm_mu_; }
  size_t bytes_per_block() const { return static_cast<size_t>(slice_byte_size_); }
  // Block-array addressing of the transport delegate
  // (kv_cache_manager_base.cc:1470-1523, 2321-2395, 2530-2548): the layers,
  // or -- once RegisterPools has succeeded -- the pools (a pool's blocks start
  // at its base offset and stride at its block stride). GetBlockChunks lists
  // the host ranges that carry `total_bytes` of the given blocks: whole
  // blocks, or each pool block's live extents (the reference's path without
  // a registered transfer plan; plans belong to its network transport).
  size_t num_block_arrays() const;
  size_t block_bytes(size_t block_array_idx) const;
  uint8_t* GetBlockArrayHostPointer(size_t block_array_idx, size_t shard_idx);
  size_t GetBlockArrayHostSize(size_t block_array_idx, size_t shard_idx);
  uint8_t* GetBlockHostPointer(size_t block_array_idx, size_t shard_idx, int64_t block_id);
  struct BlockChunk {
    uint8_t* ptr = nullptr;
    size_t size = 0;
  };
  std::vector<BlockChunk> GetBlockChunks(size_t block_array_idx, size_t shard_idx,
                                         const std::vector<int64_t>& block_ids,
                                         size_t total_bytes);
  int64_t LayerBlockByteSize(size_t layer_idx) const;
  size_t GetAllocatedHostDramBytes() const { return allocated_host_bytes_; }

  size_t num_layers() const { return static_cast<size_t>(num_layers_); }
  size_t num_shards() const { return static_cast<size_t>(num_shards_); }
  int64_t major_dim() const { return major_dim_; }
  int64_t host_blocks() const { return host_blocks_; }
  bool device_backed() const { return engine_ != nullptr; }
  // Device base address and bytes of one (layer, shard) storage, with no
  // allocation (false for a bad index or a CPU-only manager).
  bool DeviceStorage(size_t layer, size_t shard, uint64_t* dev, int64_t* dev_bytes) const {
    if (!device_backed() || layer >= static_cast<size_t>(num_layers_) ||
        shard >= static_cast<size_t>(num_shards_)) {
      return false;
    }
    const StorageInfo& si = storages_[layer * num_shards_ + shard];
    *dev = si.dev;
    *dev_bytes = si.dev_bytes;
    return true;
  }
  // True when the shared-memory host tier attached to a surviving segment.
  bool shm_warm() const { return shm_warm_; }
  HostAllocKind host_alloc() const { return cfg_.host_alloc; }
  int device() const { return cfg_.device; }
  // The NUMA node host mirrors were placed on (the reference's
  // assigned_numa_node), or -1.
  int assigned_numa_node() const { return numa_node_; }
  TransferEngine* engine() { return engine_.get(); }
  const TransferEngine* engine() const { return engine_.get(); }
  bool queued_dispatch() const { return queued_; }
  // The kinds ('D' = D2h, 'H' = H2d) of the last dispatched copies, oldest
  // first (at most 256).
  std::string DispatchLog();
  Status WaitForPendingWork();

 private:
  struct StorageInfo {
    uint64_t dev = 0;
    int64_t dev_bytes = 0;
    uint8_t* host = nullptr;
    int64_t host_bytes = 0;
    std::shared_ptr<void> host_owner;
  };
  explicit KVCacheManager(ManagerConfig cfg) : cfg_(std::move(cfg)) {}
  Status Init();
  int64_t layer_block_bytes(size_t layer) const { return layer_block_bytes_[layer]; }
  StorageInfo& storage(size_t layer, size_t shard) {
    return storages_[layer * num_shards_ + shard];
  }
  struct Work {
    size_t layer;
    size_t shard;
  };
  StatusOr<std::vector<Work>> SelectWorks(std::optional<size_t> layer_idx,
                                          std::optional<size_t> shard_idx) const;
  StatusOr<CopyFuture> Transfer(Direction dir,
                                const std::vector<int64_t>& src,
                                const std::vector<int64_t>& dst,
                                const std::vector<int64_t>& sizes,
                                std::optional<int64_t> slot_idx,
                                std::optional<size_t> layer_idx,
                                std::optional<size_t> shard_idx,
                                hipStream_t dep);
  // Callers hold pools_mu_.
  void EnsureImplicitPoolsLocked();
  Status EnsureHostMirrorCovers(size_t storage_idx, int64_t needed_bytes);
  StatusOr<CopyFuture> CopyPoolBlocks(size_t pool_idx,
                                      const std::vector<int64_t>& block_ids,
                                      std::optional<size_t> shard_idx, bool d2h,
                                      hipStream_t dep);
  StatusOr<CopyFuture> Enqueue(Direction dir, const std::vector<int64_t>& src,
                               const std::vector<int64_t>& dst,
                               const std::vector<int64_t>& sizes,
                               std::optional<int64_t> slot_idx,
                               std::optional<size_t> layer_idx,
                               std::optional<size_t> shard_idx, hipStream_t dep);
  void WorkerLoop();
  void StopWorker();
  StatusOr<CopyFuture> DeviceCopy(bool gather, const std::vector<int64_t>& ids,
                                  uint64_t staging, int64_t staging_bytes,
                                  bool block_major,
                                  std::optional<size_t> layer_idx,
                                  std::optional<size_t> shard_idx,
                                  hipStream_t stream);

  ManagerConfig cfg_;
  int64_t num_layers_ = 0;
  int64_t num_shards_ = 0;
  int64_t major_dim_ = 0;
  int64_t slice_byte_size_ = 0;
  int64_t host_blocks_ = 0;
  std::vector<int64_t> layer_block_bytes_;
  std::vector<int64_t> layer_physical_bytes_;
  std::vector<StorageInfo> storages_;
  size_t allocated_host_bytes_ = 0;
  bool host_kernel_access_ = false;
  bool shm_warm_ = false;
  int numa_node_ = -1;
  int64_t staging_num_slots_ = 0;
  int64_t staging_max_major_per_slot_ = 0;
  std::unique_ptr<LogicalBlockManager> lbm_;
  std::mutex lbm_mu_;
  std::unique_ptr<TransferEngine> engine_;
  struct QueuedCopy {
    Direction dir;
    std::vector<int64_t> src, dst, sizes;
    std::optional<int64_t> slot_idx;
    std::optional<size_t> layer_idx, shard_idx;
    hipEvent_t dep_event = nullptr;  // recorded on the caller's stream at submission
    CopyFuture future;
  };
  bool queued_ = false;
  std::thread worker_;
  std::mutex queue_mu_;
  std::condition_variable queue_cv_;
  std::deque<QueuedCopy> queue_;
  bool shutdown_ = false;
  hipStream_t dep_proxy_ = nullptr;  // carries submission-time dependencies
  std::mutex log_mu_;
  std::string dispatch_log_;
  std::mutex slots_mu_;
  std::vector<StagingSlot> all_slots_;
  std::deque<int64_t> free_slots_;
  mutable std::mutex pools_mu_;
  std::vector<PoolSpec> pools_;
  bool explicit_pools_ = false;
};

// The reference's offset validation (kv_cache_manager_base.cc:72-102) and
// run coalescing (kv_cache_manager_base.cc:121-141), exposed for tests.
Status ValidateOffsetsAndSizes(const std::vector<int64_t>& src_offsets,
                               const std::vector<int64_t>& dst_offsets,
                               const std::vector<int64_t>& sizes);
void CoalesceMajorDimCopies(const std::vector<int64_t>& src_offsets,
                            const std::vector<int64_t>& dst_offsets,
                            const std::vector<int64_t>& sizes,
                            std::vector<int64_t>& out_src,
                            std::vector<int64_t>& out_dst,
                            std::vector<int64_t>& out_sizes);

}  // namespace kvx

#endif  // KVX_HOST_KV_CACHE_MANAGER_H_
