// Tier-2 host store on one GPU: the local flows of the reference's
// KVCacheStore (tpu_sync/kv_cache/kv_cache_store.h:100-560) over its
// HostOffloadBackend (tpu_sync/kv_cache/host_offload_backend.cc), with the
// same pin contract and state machine:
//
//   read what is cached:   Lookup (pins hits) -> Load (consumes the pin)
//   cache something new:   Insert (pins)      -> Save (consumes the pin)
//
// A save moves HBM blocks into freshly allocated host blocks (evicting LRU
// candidates when the host pool is short), a load moves host blocks into
// caller device blocks; both are asynchronous and finish in PollSaveStatus /
// PollLoadStatus, which advance entries to HOST_AND_HBM. Failed operations
// keep their pins. An optional crash-persistent KVCacheMetadata table in
// shared memory mirrors every host-resident entry so a restarted process can
// rebuild the index (RecoverFromLocalManifest).
//
// Where the reference reaches its transfer worker through a RaidenController
// over loopback gRPC, this store calls the KV manager directly: the
// controller is an in-process object owning the host block allocator, and
// a KVCacheManager joins it by controller address (RegisterWorker), as the
// reference's worker does with raiden_controller_address. Remote peers,
// the global registry and the store server are out of scope: a REMOTE slice
// is refused.
#ifndef KVX_HOST_KV_CACHE_STORE_H_
#define KVX_HOST_KV_CACHE_STORE_H_

#include <cstdint>
#include <deque>
#include <functional>
#include <memory>
#include <mutex>
#include <optional>
#include <string>
#include <unordered_set>
#include <utility>
#include <vector>

#include "copy_future.h"
#include "kv_cache_metadata.h"
#include "logical_block_manager.h"
#include "lru_cache.h"
#include "status.h"

namespace kvx {

class KVCacheManager;

// tpu_sync/kv_cache/kv_cache_store_backend.h:39-77 (same numbering).
enum class BlockStatus : int {
  kInit = 0,
  kRemote = 1,
  kHbm = 2,
  kHost = 3,
  kHostAndHbm = 4,
};

struct RaidenId {
  std::string job_name;
  std::string job_replica_id;
  std::string data_name;
  int data_replica_idx = 0;
  bool operator==(const RaidenId& o) const {
    return job_name == o.job_name && job_replica_id == o.job_replica_id &&
           data_name == o.data_name && data_replica_idx == o.data_replica_idx;
  }
};

struct RaidenBlockId {
  RaidenId raiden_id;
  int host_block_id = -1;
  int device_block_id = -1;
  BlockStatus status = BlockStatus::kInit;
};

using BlockSliceList = std::vector<std::pair<std::string, RaidenBlockId>>;

struct StoreOptions {
  size_t capacity = 0;  // LRU capacity (entries)
  // Host blocks of the controller's allocator; 0 = capacity (the reference
  // sizes its controller by the store capacity, kv_cache_store.cc:150-166).
  size_t host_blocks = 0;
  RaidenId raiden_id;
  int num_shards = 1;
  int64_t shard_size_bytes = 0;
  std::string store_server_ip;
  int raiden_controller_port = 0;  // 0: pick an unused in-process address
  // Crash-persistent metadata table (empty key: none).
  std::string metadata_shm_key;
  std::string model_uid = "default_model";
  // Rebuild the index from a surviving table inside Create (falling back to
  // an empty table if that fails), as the reference's store wrapper does.
  bool recover_at_create = true;
};

// A caller-supplied transfer: moves whole blocks src[i] -> dst[i] (device to
// host when d2h, else host to device) and returns the outcome.
using StoreTransferFn = std::function<Status(bool d2h, const std::vector<int64_t>& src,
                                             const std::vector<int64_t>& dst)>;

class KVCacheStore {
 public:
  struct PollSaveStatusResult {
    std::vector<std::string> done, failed, pending, existing, unregistered;
  };
  struct PollLoadStatusResult {
    std::vector<std::string> done, failed, pending;
  };

  // Validates the options, binds the controller address and, when a
  // metadata table survived (warm), rebuilds the index from it.
  static StatusOr<std::unique_ptr<KVCacheStore>> Create(const StoreOptions& o);
  ~KVCacheStore();
  KVCacheStore(const KVCacheStore&) = delete;
  KVCacheStore& operator=(const KVCacheStore&) = delete;

  const std::string& raiden_controller_address() const { return address_; }
  const RaidenId& raiden_id() const { return opts_.raiden_id; }
  size_t capacity() const { return opts_.capacity; }
  size_t size() const;
  bool metadata_warm() const { return region_ != nullptr && region_->warm(); }
  // Blocks recovered at construction (0 on a cold start).
  size_t recovered_blocks() const { return recovered_; }

  // The transfer worker (one per store on one GPU). A save or load issued
  // with no worker fails in the poll, as the reference's controller fails
  // TransferBuffers with no registered workers.
  void SetWorker(KVCacheManager* worker);
  KVCacheManager* worker() const;
  // Routes saves and loads through `fn` instead of the worker (empty fn:
  // back to the worker). The counterpart of the transfer manager a
  // reference worker is built with; tests use a recording or failing one.
  void SetTransferFn(StoreTransferFn fn);

  // Drops unpinned host-resident entries and frees their host blocks;
  // returns how many were dropped (kv_cache_store.cc:1553-1570).
  size_t Evict(const std::vector<std::string>& hashes);

  StatusOr<BlockSliceList> Lookup(const std::vector<std::string>& hashes,
                                  bool pin_found);
  Status Insert(const std::vector<std::string>& hashes,
                const std::vector<RaidenBlockId>& slices, bool on_host);
  void Release(const std::vector<std::string>& hashes);
  Status Save(const std::vector<std::string>& hashes);
  Status Load(const std::vector<std::string>& hashes,
              const std::vector<int>& device_block_ids);
  Status Load(const std::vector<std::string>& hashes,
              const std::vector<RaidenBlockId>& slices,
              const std::vector<int>& device_block_ids);
  PollSaveStatusResult PollSaveStatus();
  PollLoadStatusResult PollLoadStatus();
  StatusOr<size_t> RecoverFromLocalManifest();
  int GetPinCount(const std::string& hash) const;

  // Controller-side host block bookkeeping (RaidenController::Allocate/
  // DeallocateBlockIds): ids are locked on allocation.
  LogicalBlockManager& block_manager() { return lbm_; }
  std::mutex& block_manager_mutex() { return lbm_mu_; }
  // Evictable keys and eviction candidates of the index (for tests).
  std::vector<std::string> GetEvictableKeys(size_t count) const;
  std::vector<std::string> GetEvictCandidateKeys() const;

 private:
  struct SaveState {
    CopyFuture future;
    std::vector<std::string> hashes;
    std::vector<int> host_block_ids;
  };
  struct LoadState {
    CopyFuture future;
    std::vector<std::string> hashes;
    std::vector<int> device_block_ids;
  };

  explicit KVCacheStore(const StoreOptions& o);

  // Backend (HostOffloadBackend) operations; callers hold mu_.
  BlockSliceList BackendLookupLocked(const std::vector<std::string>& hashes,
                                     bool pin_found);
  void BackendUpdateLocked(const std::vector<std::string>& hashes,
                           const std::vector<RaidenBlockId>& slices);
  bool BackendInsertAndLockLocked(const std::vector<std::string>& hashes,
                                  const std::vector<RaidenBlockId>& slices);
  void BackendReleaseAndDeleteLocked(const std::vector<std::string>& hashes);
  void BackendReleaseLocked(const std::vector<std::string>& hashes);
  std::vector<int> BackendEvictLocked(const std::vector<std::string>& hashes);
  void SetMetadataLocked(const std::string& hash, const RaidenBlockId& b);
  void ClearMetadataLocked(const RaidenBlockId& b);

  StatusOr<std::vector<int>> AllocateBlockIds(int needed);
  void DeallocateBlockIds(const std::vector<int>& ids);
  // One whole-block copy per pair through the worker (TransferBuffers).
  CopyFuture Transfer(bool d2h, const std::vector<int64_t>& src,
                      const std::vector<int64_t>& dst);
  void PollFutures();

  StoreOptions opts_;
  std::string address_;
  mutable std::mutex mu_;
  LRUCache<std::string, RaidenBlockId> lru_;
  std::unique_ptr<KVCacheMetadataShmRegion> region_;
  uint64_t next_seq_ = 0;
  size_t recovered_ = 0;
  std::unordered_set<std::string> saving_, loading_;
  std::deque<SaveState> active_saves_;
  std::deque<LoadState> active_loads_;
  std::vector<std::string> done_saves_, failed_saves_, done_loads_, failed_loads_;

  std::mutex lbm_mu_;
  LogicalBlockManager lbm_;
  mutable std::mutex worker_mu_;
  KVCacheManager* worker_ = nullptr;
  StoreTransferFn transfer_fn_;
};

// In-process controller directory: a store registers its controller
// address; a manager created with that address becomes its worker.
Status RegisterWorkerAtController(const std::string& address,
                                  KVCacheManager* worker);
// Detaches `worker` from whichever store uses it (manager teardown).
void UnregisterWorker(KVCacheManager* worker);

}  // namespace kvx

#endif  // KVX_HOST_KV_CACHE_STORE_H_
