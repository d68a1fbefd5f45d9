#include "kv_cache_store.h"

#include <algorithm>
#include <cstdio>
#include <map>
#include <unordered_map>

#include "kv_cache_manager.h"

namespace kvx {
namespace {

bool OnHost(const RaidenBlockId& b) {
  return b.status == BlockStatus::kHost || b.status == BlockStatus::kHostAndHbm;
}

std::string Hex(const std::string& s) {
  static const char* d = "0123456789abcdef";
  std::string out;
  out.reserve(2 * s.size());
  for (unsigned char c : s) {
    out.push_back(d[c >> 4]);
    out.push_back(d[c & 15]);
  }
  return out;
}

// Process-wide directory of in-process controllers, by address.
struct Directory {
  std::mutex mu;
  std::map<std::string, KVCacheStore*> stores;
};
Directory& Dir() {
  static Directory* d = new Directory();
  return *d;
}

}  // namespace

Status RegisterWorkerAtController(const std::string& address,
                                  KVCacheManager* worker) {
  Directory& d = Dir();
  std::lock_guard<std::mutex> l(d.mu);
  auto it = d.stores.find(address);
  if (it == d.stores.end()) {
    return UnavailableError("no RaidenController at " + address +
                            " in this process");
  }
  it->second->SetWorker(worker);
  return OkStatus();
}

void UnregisterWorker(KVCacheManager* worker) {
  Directory& d = Dir();
  std::lock_guard<std::mutex> l(d.mu);
  for (auto& kv : d.stores) {
    if (kv.second->worker() == worker) kv.second->SetWorker(nullptr);
  }
}

KVCacheStore::KVCacheStore(const StoreOptions& o)
    : opts_(o),
      lru_(o.capacity),
      lbm_(static_cast<int>(o.host_blocks > 0 ? o.host_blocks : o.capacity)) {}

StatusOr<std::unique_ptr<KVCacheStore>> KVCacheStore::Create(const StoreOptions& o) {
  const std::string& ip = o.store_server_ip;
  if (ip.empty()) {
    return InvalidArgumentError(
        "store_server_ip is required: it is the host peers use to reach this "
        "store's services. Same-host use: \"127.0.0.1\".");
  }
  if (ip == "[::]" || ip == "::" || ip == "0.0.0.0" || ip == "0:0:0:0:0:0:0:0") {
    return InvalidArgumentError("store_server_ip may not be a wildcard (got \"" +
                                ip + "\")");
  }
  if (o.num_shards < 1) {
    return InvalidArgumentError(
        "num_shards must be >= 1: every KVCacheStore has a RaidenController");
  }
  if (o.capacity == 0) {
    return InvalidArgumentError("HostOffloadBackend requires capacity > 0");
  }
  if (o.capacity > static_cast<size_t>(INT32_MAX) ||
      o.host_blocks > static_cast<size_t>(INT32_MAX)) {
    return InvalidArgumentError("capacity too large");
  }
  std::unique_ptr<KVCacheStore> s(new KVCacheStore(o));
  {
    Directory& d = Dir();
    std::lock_guard<std::mutex> l(d.mu);
    if (o.raiden_controller_port > 0) {
      s->address_ = ip + ":" + std::to_string(o.raiden_controller_port);
      if (d.stores.count(s->address_)) {
        return AlreadyExistsError("a RaidenController already serves " + s->address_);
      }
    } else {
      // Port 0: the next free in-process "port", as a bound socket would get.
      for (int port = 20000; port < 65536; ++port) {
        std::string a = ip + ":" + std::to_string(port);
        if (!d.stores.count(a)) {
          s->address_ = a;
          break;
        }
      }
    }
    d.stores[s->address_] = s.get();
  }
  if (!o.metadata_shm_key.empty()) {
    // One slot per host block: the table is indexed by host block id.
    auto region = KVCacheMetadataShmRegion::AttachOrFormat(
        o.metadata_shm_key, static_cast<int>(o.host_blocks > 0 ? o.host_blocks : o.capacity),
        o.model_uid);
    // Without a table the store serves, but cannot recover after a crash.
    if (region.ok()) s->region_ = std::move(region.value());
  }
  if (o.recover_at_create && s->region_ != nullptr && s->region_->warm()) {
    auto n = s->RecoverFromLocalManifest();
    if (n.ok()) {
      s->recovered_ = n.value();
    } else {
      (void)s->region_->Reformat();
    }
  }
  return s;
}

KVCacheStore::~KVCacheStore() {
  {
    Directory& d = Dir();
    std::lock_guard<std::mutex> l(d.mu);
    auto it = d.stores.find(address_);
    if (it != d.stores.end() && it->second == this) d.stores.erase(it);
  }
  // Outstanding copies still write into the worker's buffers; let them land.
  std::lock_guard<std::mutex> l(mu_);
  for (SaveState& s : active_saves_) (void)s.future.Await();
  for (LoadState& s : active_loads_) (void)s.future.Await();
}

size_t KVCacheStore::size() const {
  std::lock_guard<std::mutex> l(mu_);
  return lru_.size();
}

void KVCacheStore::SetWorker(KVCacheManager* worker) {
  std::lock_guard<std::mutex> l(worker_mu_);
  worker_ = worker;
}

KVCacheManager* KVCacheStore::worker() const {
  std::lock_guard<std::mutex> l(worker_mu_);
  return worker_;
}

void KVCacheStore::SetTransferFn(StoreTransferFn fn) {
  std::lock_guard<std::mutex> l(worker_mu_);
  transfer_fn_ = std::move(fn);
}

size_t KVCacheStore::Evict(const std::vector<std::string>& hashes) {
  if (hashes.empty()) return 0;
  std::vector<int> ids;
  {
    std::lock_guard<std::mutex> l(mu_);
    ids = BackendEvictLocked(hashes);
  }
  if (!ids.empty()) DeallocateBlockIds(ids);
  return ids.size();
}

int KVCacheStore::GetPinCount(const std::string& hash) const {
  std::lock_guard<std::mutex> l(mu_);
  return lru_.GetPinCount(hash);
}

std::vector<std::string> KVCacheStore::GetEvictableKeys(size_t count) const {
  std::lock_guard<std::mutex> l(mu_);
  return lru_.GetEvictableKeys(count);
}

std::vector<std::string> KVCacheStore::GetEvictCandidateKeys() const {
  std::lock_guard<std::mutex> l(mu_);
  return lru_.GetEvictCandidateKeys();
}

// ---- backend (HostOffloadBackend local subset) -----------------------------

void KVCacheStore::SetMetadataLocked(const std::string& hash, const RaidenBlockId& b) {
  if (region_ == nullptr || !OnHost(b)) return;
  Status st = region_->metadata().Set(b.host_block_id, hash, next_seq_++);
  if (!st.ok()) {
    std::fprintf(stderr, "kvx: metadata set for block %d failed: %s\n",
                 b.host_block_id, st.message().c_str());
  }
}

void KVCacheStore::ClearMetadataLocked(const RaidenBlockId& b) {
  if (region_ == nullptr || !OnHost(b)) return;
  (void)region_->metadata().Clear(b.host_block_id);
}

// host_offload_backend.cc:154-288 without the registry: every local hit is
// pinned (when asked) in a first sweep, the answer runs to the first miss,
// and pins of hits past the end are handed back -- which moves those entries
// to the active front, exactly as the reference's pin/unpin round trip does.
BlockSliceList KVCacheStore::BackendLookupLocked(const std::vector<std::string>& hashes,
                                                 bool pin_found) {
  BlockSliceList out;
  if (hashes.empty()) return out;
  std::vector<char> hit(hashes.size(), 0);
  for (size_t i = 0; i < hashes.size(); ++i) {
    if (lru_.Peek(hashes[i]) != nullptr) {
      if (pin_found) lru_.Pin(hashes[i]);
      hit[i] = 1;
    }
  }
  for (size_t i = 0; i < hashes.size(); ++i) {
    if (!hit[i]) break;
    const RaidenBlockId* b = lru_.Peek(hashes[i]);
    if (b == nullptr) break;
    out.emplace_back(hashes[i], *b);
  }
  if (pin_found) {
    for (size_t i = out.size(); i < hashes.size(); ++i) {
      if (hit[i]) lru_.Unpin(hashes[i]);
    }
  }
  return out;
}

// host_offload_backend.cc:290-368 (Insert): updates present entries in
// place, inserts the rest.
void KVCacheStore::BackendUpdateLocked(const std::vector<std::string>& hashes,
                                       const std::vector<RaidenBlockId>& slices) {
  for (size_t i = 0; i < hashes.size(); ++i) {
    const std::string& h = hashes[i];
    if (lru_.Contains(h)) {
      if (i < slices.size()) {
        if (RaidenBlockId* cur = lru_.PeekMutable(h)) {
          *cur = slices[i];
          SetMetadataLocked(h, slices[i]);
        }
      }
      continue;
    }
    if (const RaidenBlockId* stale = lru_.PeekIncludingCandidates(h)) {
      ClearMetadataLocked(*stale);
    }
    if (i < slices.size()) {
      (void)lru_.Put(h, slices[i]);
      SetMetadataLocked(h, slices[i]);
    } else {
      (void)lru_.Put(h, RaidenBlockId());
    }
  }
}

// host_offload_backend.cc:370-460 (InsertAndLock): all-or-nothing pin of
// present hashes, insert of new ones in reverse order (tail blocks evict
// first), then pin of the new ones.
bool KVCacheStore::BackendInsertAndLockLocked(const std::vector<std::string>& hashes,
                                              const std::vector<RaidenBlockId>& slices) {
  std::vector<size_t> have, fresh;
  for (size_t i = 0; i < hashes.size(); ++i) {
    (lru_.Contains(hashes[i]) ? have : fresh).push_back(i);
  }
  for (size_t k = 0; k < have.size(); ++k) {
    const size_t i = have[k];
    if (!lru_.Pin(hashes[i])) {
      for (size_t j = 0; j < k; ++j) lru_.Unpin(hashes[have[j]]);
      return false;
    }
    // An HBM-only entry describes nothing but a device block; the caller's
    // binding replaces it. Host-resident entries are kept.
    if (i < slices.size()) {
      RaidenBlockId* cur = lru_.PeekMutable(hashes[i]);
      if (cur != nullptr && cur->status == BlockStatus::kHbm) {
        ClearMetadataLocked(*cur);
        *cur = slices[i];
        SetMetadataLocked(hashes[i], slices[i]);
      }
    }
  }
  if (lru_.available_space() < fresh.size()) {
    for (size_t i : have) lru_.Unpin(hashes[i]);
    return false;
  }
  for (auto it = fresh.rbegin(); it != fresh.rend(); ++it) {
    const size_t i = *it;
    if (const RaidenBlockId* stale = lru_.PeekIncludingCandidates(hashes[i])) {
      ClearMetadataLocked(*stale);
    }
    if (i < slices.size()) {
      (void)lru_.Put(hashes[i], slices[i]);
      SetMetadataLocked(hashes[i], slices[i]);
    } else {
      (void)lru_.Put(hashes[i], RaidenBlockId());
    }
  }
  for (size_t k = 0; k < fresh.size(); ++k) {
    if (!lru_.Pin(hashes[fresh[k]])) {
      for (size_t j = 0; j < k; ++j) lru_.Unpin(hashes[fresh[j]]);
      for (size_t i : have) lru_.Unpin(hashes[i]);
      for (size_t i : fresh) {
        if (const RaidenBlockId* v = lru_.PeekIncludingCandidates(hashes[i])) {
          ClearMetadataLocked(*v);
        }
        lru_.Erase(hashes[i]);
      }
      return false;
    }
  }
  return true;
}

void KVCacheStore::BackendReleaseLocked(const std::vector<std::string>& hashes) {
  // Reverse order leaves hashes[0] (the head of a prefix chain) nearest the
  // MRU end.
  for (auto it = hashes.rbegin(); it != hashes.rend(); ++it) lru_.Unpin(*it);
}

std::vector<int> KVCacheStore::BackendEvictLocked(const std::vector<std::string>& hashes) {
  std::vector<int> ids;
  for (const std::string& h : hashes) {
    const RaidenBlockId* b = lru_.PeekIncludingCandidates(h);
    if (b != nullptr && lru_.GetPinCount(h) == 0 && OnHost(*b)) {
      ids.push_back(b->host_block_id);
      ClearMetadataLocked(*b);
      lru_.Erase(h);
    }
  }
  return ids;
}

// ---- store flows ------------------------------------------------------------

StatusOr<BlockSliceList> KVCacheStore::Lookup(const std::vector<std::string>& hashes,
                                              bool pin_found) {
  std::lock_guard<std::mutex> l(mu_);
  BlockSliceList out = BackendLookupLocked(hashes, pin_found);
  const size_t cap = opts_.capacity;
  if (cap > 0 && out.size() > cap) {
    if (pin_found) {
      std::vector<std::string> excess;
      for (size_t i = cap; i < out.size(); ++i) excess.push_back(out[i].first);
      BackendReleaseLocked(excess);
    }
    out.resize(cap);
  }
  return out;
}

Status KVCacheStore::Insert(const std::vector<std::string>& hashes,
                            const std::vector<RaidenBlockId>& slices, bool /*on_host*/) {
  for (size_t i = 0; i < slices.size(); ++i) {
    if (slices[i].status == BlockStatus::kRemote) {
      return InvalidArgumentError(
          "Insert only takes LOCAL entries; slice " + std::to_string(i) + " (hash " +
          (i < hashes.size() ? Hex(hashes[i]) : std::string("<none>")) +
          ") has status REMOTE");
    }
  }
  std::lock_guard<std::mutex> l(mu_);
  if (!BackendInsertAndLockLocked(hashes, slices)) {
    return ResourceExhaustedError(
        "Insert refused: not enough unpinned space, or a hash could not be pinned");
  }
  return OkStatus();
}

void KVCacheStore::Release(const std::vector<std::string>& hashes) {
  std::lock_guard<std::mutex> l(mu_);
  BackendReleaseLocked(hashes);
}

StatusOr<std::vector<int>> KVCacheStore::AllocateBlockIds(int needed) {
  std::vector<std::string> victims;
  {
    std::lock_guard<std::mutex> l(mu_);
    int free_count;
    {
      std::lock_guard<std::mutex> lb(lbm_mu_);
      free_count = lbm_.num_free_blocks();
    }
    const int to_free = needed - free_count;
    if (to_free > 0) {
      victims = lru_.GetEvictableKeys(static_cast<size_t>(to_free));
      if (victims.size() < static_cast<size_t>(to_free)) {
        return ResourceExhaustedError(
            "Insufficient free blocks and not enough evictable blocks. Needed: " +
            std::to_string(needed) + ", Free: " + std::to_string(free_count) +
            ", Evictable: " + std::to_string(victims.size()));
      }
    }
  }
  (void)Evict(victims);
  std::lock_guard<std::mutex> lb(lbm_mu_);
  return lbm_.Allocate(needed, /*lock=*/true);
}

void KVCacheStore::DeallocateBlockIds(const std::vector<int>& ids) {
  std::lock_guard<std::mutex> lb(lbm_mu_);
  Status st = lbm_.Deallocate(ids);
  if (!st.ok()) {
    std::fprintf(stderr, "kvx: failed to deallocate host block ids: %s\n",
                 st.message().c_str());
  }
}

CopyFuture KVCacheStore::Transfer(bool d2h, const std::vector<int64_t>& src,
                                  const std::vector<int64_t>& dst) {
  StoreTransferFn fn;
  KVCacheManager* w;
  {
    std::lock_guard<std::mutex> l(worker_mu_);
    fn = transfer_fn_;
    w = worker_;
  }
  if (fn) return CopyFuture(fn(d2h, src, dst));
  if (w == nullptr) {
    return CopyFuture(
        FailedPreconditionError("No registered workers available for TransferBuffers"));
  }
  std::vector<int64_t> sizes(src.size(), 1);
  StatusOr<CopyFuture> f = d2h ? w->D2h(src, dst, sizes) : w->H2d(src, dst, sizes);
  if (!f.ok()) return CopyFuture(f.status());
  return f.value();
}

Status KVCacheStore::Save(const std::vector<std::string>& hashes) {
  std::vector<int64_t> src;
  {
    std::lock_guard<std::mutex> l(mu_);
    BlockSliceList found = BackendLookupLocked(hashes, false);
    if (found.size() < hashes.size()) {
      return NotFoundError("Block hash not found: " + hashes[found.size()]);
    }
    for (size_t i = 0; i < found.size(); ++i) {
      const std::string& h = hashes[i];
      const RaidenBlockId& b = found[i].second;
      if (b.status != BlockStatus::kHbm) {
        return FailedPreconditionError("Block is not in HBM status: " + h);
      }
      if (b.device_block_id == -1) {
        return FailedPreconditionError("Block device_block_id is -1: " + h);
      }
      if (lru_.GetPinCount(h) <= 0) {
        return FailedPreconditionError("Block is not pinned: " + h);
      }
      if (saving_.count(h)) {
        return FailedPreconditionError("Block is already saving: " + h);
      }
      src.push_back(b.device_block_id);
    }
    for (const std::string& h : hashes) saving_.insert(h);
  }
  StatusOr<std::vector<int>> host = AllocateBlockIds(static_cast<int>(hashes.size()));
  if (!host.ok()) {
    std::lock_guard<std::mutex> l(mu_);
    for (const std::string& h : hashes) saving_.erase(h);
    return host.status();
  }
  std::vector<int64_t> dst(host->begin(), host->end());
  CopyFuture f = Transfer(/*d2h=*/true, src, dst);
  std::lock_guard<std::mutex> l(mu_);
  active_saves_.push_back(SaveState{f, hashes, host.value()});
  return OkStatus();
}

Status KVCacheStore::Load(const std::vector<std::string>& hashes,
                          const std::vector<int>& device_block_ids) {
  if (hashes.size() != device_block_ids.size()) {
    return InvalidArgumentError("block_hashes and device_block_ids size mismatch");
  }
  if (hashes.empty()) return OkStatus();
  std::vector<int64_t> src;
  {
    std::lock_guard<std::mutex> l(mu_);
    BlockSliceList found = BackendLookupLocked(hashes, false);
    if (found.size() < hashes.size()) {
      return NotFoundError("Block hash not found: " + hashes[found.size()]);
    }
    for (size_t i = 0; i < found.size(); ++i) {
      const std::string& h = hashes[i];
      const RaidenBlockId& b = found[i].second;
      if (b.status == BlockStatus::kRemote) {
        return InvalidArgumentError(
            "Load without slices is local-only, but block is REMOTE: " + h);
      }
      if (lru_.GetPinCount(h) <= 0) {
        return FailedPreconditionError("Block is not pinned: " + h);
      }
      if (loading_.count(h)) {
        return FailedPreconditionError("Block is already loading: " + h);
      }
      if (!OnHost(b)) return FailedPreconditionError("Block is not on host: " + h);
      if (b.host_block_id == -1) {
        return FailedPreconditionError("Block host_block_id is -1: " + h);
      }
    }
    for (const std::string& h : hashes) loading_.insert(h);
    // Source host ids, read as the backend's local load does
    // (host_offload_backend.cc:1084-1139).
    for (const std::string& h : hashes) src.push_back(lru_.Peek(h)->host_block_id);
  }
  std::vector<int64_t> dst(device_block_ids.begin(), device_block_ids.end());
  CopyFuture f = Transfer(/*d2h=*/false, src, dst);
  std::lock_guard<std::mutex> l(mu_);
  active_loads_.push_back(LoadState{f, hashes, device_block_ids});
  return OkStatus();
}

Status KVCacheStore::Load(const std::vector<std::string>& hashes,
                          const std::vector<RaidenBlockId>& slices,
                          const std::vector<int>& device_block_ids) {
  if (hashes.size() != slices.size() || slices.size() != device_block_ids.size()) {
    return InvalidArgumentError("block_hashes, slices, and device_block_ids size mismatch");
  }
  if (hashes.empty()) return OkStatus();
  const bool remote = slices[0].status == BlockStatus::kRemote;
  {
    std::lock_guard<std::mutex> l(mu_);
    for (size_t i = 0; i < slices.size(); ++i) {
      const std::string& h = hashes[i];
      const RaidenBlockId& b = slices[i];
      if (loading_.count(h)) {
        return FailedPreconditionError("Block is already loading: " + h);
      }
      if (remote) {
        if (b.status != BlockStatus::kRemote) {
          return InvalidArgumentError("Mixed block statuses in a single Load call");
        }
        if (!(b.raiden_id == slices[0].raiden_id)) {
          return InvalidArgumentError("Mixed remote node IDs in a single Load call");
        }
      } else {
        if (lru_.GetPinCount(h) <= 0) {
          return FailedPreconditionError("Block is not pinned: " + h);
        }
        if (!OnHost(b)) return FailedPreconditionError("Block is not on host: " + h);
        if (b.host_block_id == -1) {
          return FailedPreconditionError("Block host_block_id is -1: " + h);
        }
      }
    }
    for (const std::string& h : hashes) loading_.insert(h);
  }
  CopyFuture f;
  if (remote) {
    // A peer is resolved through the global registry, which a single-node
    // store does not have: the load fails in the poll.
    f = CopyFuture(FailedPreconditionError(
        "No global registry client; cannot resolve peer store address"));
  } else {
    std::vector<int64_t> src, dst(device_block_ids.begin(), device_block_ids.end());
    for (const RaidenBlockId& b : slices) src.push_back(b.host_block_id);
    f = Transfer(/*d2h=*/false, src, dst);
  }
  std::lock_guard<std::mutex> l(mu_);
  active_loads_.push_back(LoadState{f, hashes, device_block_ids});
  return OkStatus();
}

void KVCacheStore::PollFutures() {
  std::vector<SaveState> saves;
  std::vector<LoadState> loads;
  {
    std::lock_guard<std::mutex> l(mu_);
    for (auto it = active_saves_.begin(); it != active_saves_.end();) {
      if (it->future.IsReady()) {
        saves.push_back(std::move(*it));
        it = active_saves_.erase(it);
      } else {
        ++it;
      }
    }
    for (auto it = active_loads_.begin(); it != active_loads_.end();) {
      if (it->future.IsReady()) {
        loads.push_back(std::move(*it));
        it = active_loads_.erase(it);
      } else {
        ++it;
      }
    }
  }
  // kv_cache_store.cc:2113-2191: a landed save rebinds each entry to its new
  // host block as HOST_AND_HBM and spends the Insert pin; a failed one frees
  // the host blocks and keeps the pins.
  for (SaveState& s : saves) {
    Status st = s.future.Await();
    std::lock_guard<std::mutex> l(mu_);
    if (st.ok()) {
      BlockSliceList found = BackendLookupLocked(s.hashes, false);
      std::vector<std::string> upd_h;
      std::vector<RaidenBlockId> upd_s;
      for (size_t i = 0; i < s.hashes.size(); ++i) {
        if (i < found.size()) {
          RaidenBlockId b = found[i].second;
          b.host_block_id = s.host_block_ids[i];
          b.status = BlockStatus::kHostAndHbm;
          upd_h.push_back(s.hashes[i]);
          upd_s.push_back(b);
        }
        done_saves_.push_back(s.hashes[i]);
      }
      if (!upd_h.empty()) {
        BackendUpdateLocked(upd_h, upd_s);
        BackendReleaseLocked(upd_h);
      }
    } else {
      DeallocateBlockIds(s.host_block_ids);
      for (const std::string& h : s.hashes) failed_saves_.push_back(h);
    }
    for (const std::string& h : s.hashes) saving_.erase(h);
  }
  // kv_cache_store.cc:2193-2253: a landed local load records the device
  // block (HOST_AND_HBM) and spends the Lookup pin.
  for (LoadState& s : loads) {
    Status st = s.future.Await();
    std::lock_guard<std::mutex> l(mu_);
    if (st.ok()) {
      BlockSliceList found = BackendLookupLocked(s.hashes, false);
      std::vector<std::string> upd_h;
      std::vector<RaidenBlockId> upd_s;
      for (size_t i = 0; i < s.hashes.size(); ++i) {
        if (i < found.size()) {
          RaidenBlockId b = found[i].second;
          b.device_block_id = s.device_block_ids[i];
          b.status = BlockStatus::kHostAndHbm;
          upd_h.push_back(s.hashes[i]);
          upd_s.push_back(b);
        }
        done_loads_.push_back(s.hashes[i]);
      }
      if (!upd_h.empty()) {
        BackendUpdateLocked(upd_h, upd_s);
        BackendReleaseLocked(upd_h);
      }
    } else {
      for (const std::string& h : s.hashes) failed_loads_.push_back(h);
    }
    for (const std::string& h : s.hashes) loading_.erase(h);
  }
}

KVCacheStore::PollSaveStatusResult KVCacheStore::PollSaveStatus() {
  PollFutures();
  std::lock_guard<std::mutex> l(mu_);
  PollSaveStatusResult r;
  for (const SaveState& s : active_saves_) {
    r.pending.insert(r.pending.end(), s.hashes.begin(), s.hashes.end());
  }
  r.done.swap(done_saves_);
  r.failed.swap(failed_saves_);
  return r;
}

KVCacheStore::PollLoadStatusResult KVCacheStore::PollLoadStatus() {
  PollFutures();
  std::lock_guard<std::mutex> l(mu_);
  PollLoadStatusResult r;
  for (const LoadState& s : active_loads_) {
    r.pending.insert(r.pending.end(), s.hashes.begin(), s.hashes.end());
  }
  r.done.swap(done_loads_);
  r.failed.swap(failed_loads_);
  return r;
}

// kv_cache_store.cc:1541-1551 and host_offload_backend.cc:559-620.
StatusOr<size_t> KVCacheStore::RecoverFromLocalManifest() {
  std::lock_guard<std::mutex> l(mu_);
  if (lru_.size() > 0) {
    return FailedPreconditionError(
        "RecoverFromLocalManifest can only be called on an empty cache store");
  }
  if (region_ == nullptr) {
    return FailedPreconditionError("KVCacheMetadata is required for crash recovery");
  }
  KVCacheMetadata& md = region_->metadata();
  std::vector<KVCacheMetadata::Entry> entries = md.ValidEntries();
  if (entries.empty()) return size_t{0};
  // The newest binding (largest seq) of each hash wins; on a tie the lower
  // block id, which ValidEntries lists first.
  std::unordered_map<std::string, size_t> newest;
  for (size_t k = 0; k < entries.size(); ++k) {
    auto it = newest.emplace(entries[k].hash, k);
    if (!it.second && entries[k].seq > entries[it.first->second].seq) {
      it.first->second = k;
    }
  }
  std::vector<size_t> keep;
  for (const auto& kv : newest) keep.push_back(kv.second);
  std::sort(keep.begin(), keep.end(), [&](size_t a, size_t b) {
    return entries[a].seq != entries[b].seq ? entries[a].seq < entries[b].seq
                                            : entries[a].block_id < entries[b].block_id;
  });
  std::vector<int> ids;
  for (size_t k : keep) ids.push_back(entries[k].block_id);
  {
    std::lock_guard<std::mutex> lb(lbm_mu_);
    KVX_RETURN_IF_ERROR(lbm_.AllocateTarget(ids));
  }
  uint64_t max_seq = 0;
  for (size_t k : keep) {
    RaidenBlockId b;
    b.raiden_id = opts_.raiden_id;
    b.host_block_id = entries[k].block_id;
    b.status = BlockStatus::kHost;
    (void)lru_.Put(entries[k].hash, b);
    max_seq = std::max(max_seq, entries[k].seq);
  }
  next_seq_ = max_seq + 1;
  for (size_t k = 0; k < entries.size(); ++k) {
    if (entries[newest.at(entries[k].hash)].block_id != entries[k].block_id) {
      (void)md.Clear(entries[k].block_id);
    }
  }
  return keep.size();
}

}  // namespace kvx
