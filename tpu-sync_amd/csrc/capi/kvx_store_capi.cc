// extern "C" layer over the host tier: the KV store (local flows), its LRU
// index and the crash-persistent metadata table.
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "../host/kv_cache_metadata.h"
#include "../host/kv_cache_store.h"
#include "../host/lru_cache.h"
#include "../host/raiden_env.h"
#include "capi_internal.h"

struct kvx_store {
  std::unique_ptr<kvx::KVCacheStore> impl;
  kvx_block_manager lbm_view;
};

struct kvx_slices {
  kvx::BlockSliceList items;
  // kvx_slices_flat: the hashes back to back, their offsets and one
  // kvx_block_slice per item (built on first use).
  std::string hashes;
  std::vector<int64_t> offsets;
  std::vector<kvx_block_slice> blocks;
};

struct kvx_lru {
  kvx::LRUCache<std::string, int64_t> impl;
  explicit kvx_lru(size_t cap) : impl(cap) {}
};

struct kvx_metadata_region {
  std::unique_ptr<kvx::KVCacheMetadataShmRegion> impl;
};

namespace {

using kvx_capi::BadArray;
using kvx_capi::Done;
using kvx_capi::Fail;

const char* Str(const char* s) { return s == nullptr ? "" : s; }

// Packed byte strings: item i is bytes[offsets[i], offsets[i+1]).
bool Unpack(const uint8_t* bytes, const int64_t* offsets, int64_t n,
            std::vector<std::string>* out) {
  out->clear();
  if (n < 0 || (n > 0 && offsets == nullptr)) return false;
  for (int64_t i = 0; i < n; ++i) {
    const int64_t a = offsets[i], b = offsets[i + 1];
    if (a < 0 || b < a || (b > a && bytes == nullptr)) return false;
    out->emplace_back(reinterpret_cast<const char*>(bytes) + a,
                      static_cast<size_t>(b - a));
  }
  return true;
}

bool ToSlices(const kvx_block_slice* s, int64_t n, std::vector<kvx::RaidenBlockId>* out) {
  out->clear();
  if (BadArray(s, n)) return false;
  for (int64_t i = 0; i < n; ++i) {
    if (s[i].status < KVX_BLOCK_INIT || s[i].status > KVX_BLOCK_HOST_AND_HBM) return false;
    kvx::RaidenBlockId b;
    b.raiden_id.job_name = Str(s[i].job_name);
    b.raiden_id.job_replica_id = Str(s[i].job_replica_id);
    b.raiden_id.data_name = Str(s[i].data_name);
    b.raiden_id.data_replica_idx = s[i].data_replica_idx;
    b.host_block_id = s[i].host_block_id;
    b.device_block_id = s[i].device_block_id;
    b.status = static_cast<kvx::BlockStatus>(s[i].status);
    out->push_back(std::move(b));
  }
  return true;
}

kvx_strings* NewStrings(std::vector<std::string> v) {
  auto* s = new kvx_strings;
  s->items = std::move(v);
  return s;
}

#define KVX_UNPACK_HASHES(var)                                               \
  std::vector<std::string> var;                                              \
  if (!Unpack(bytes, offsets, n, &var)) {                                    \
    return Fail(KVX_INVALID_ARGUMENT, "malformed packed hash list");          \
  }

}  // namespace

extern "C" {

// ---- string lists and slice lists ------------------------------------------

int64_t kvx_strings_count(const kvx_strings* s) {
  return s == nullptr ? 0 : static_cast<int64_t>(s->items.size());
}

int kvx_strings_get(const kvx_strings* s, int64_t i, const uint8_t** data,
                    int64_t* len) {
  if (s == nullptr || data == nullptr || len == nullptr || i < 0 ||
      i >= static_cast<int64_t>(s->items.size())) {
    return Fail(KVX_OUT_OF_RANGE, "string index out of range");
  }
  *data = reinterpret_cast<const uint8_t*>(s->items[i].data());
  *len = static_cast<int64_t>(s->items[i].size());
  return KVX_OK;
}

int kvx_strings_flat(kvx_strings* s, const uint8_t** data, const int64_t** offsets) {
  if (s == nullptr || data == nullptr || offsets == nullptr) {
    return Fail(KVX_INVALID_ARGUMENT, "null list or output");
  }
  if (s->offsets.empty()) {
    s->offsets.reserve(s->items.size() + 1);
    s->offsets.push_back(0);
    for (const std::string& it : s->items) {
      s->flat += it;
      s->offsets.push_back(static_cast<int64_t>(s->flat.size()));
    }
  }
  *data = reinterpret_cast<const uint8_t*>(s->flat.data());
  *offsets = s->offsets.data();
  return KVX_OK;
}

void kvx_strings_release(kvx_strings* s) { delete s; }

int64_t kvx_slices_count(const kvx_slices* s) {
  return s == nullptr ? 0 : static_cast<int64_t>(s->items.size());
}

int kvx_slices_get(const kvx_slices* s, int64_t i, const uint8_t** hash,
                   int64_t* hash_len, kvx_block_slice* out) {
  if (s == nullptr || hash == nullptr || hash_len == nullptr || out == nullptr ||
      i < 0 || i >= static_cast<int64_t>(s->items.size())) {
    return Fail(KVX_OUT_OF_RANGE, "slice index out of range");
  }
  const auto& p = s->items[i];
  *hash = reinterpret_cast<const uint8_t*>(p.first.data());
  *hash_len = static_cast<int64_t>(p.first.size());
  out->host_block_id = p.second.host_block_id;
  out->device_block_id = p.second.device_block_id;
  out->status = static_cast<int32_t>(p.second.status);
  out->data_replica_idx = p.second.raiden_id.data_replica_idx;
  out->job_name = p.second.raiden_id.job_name.c_str();
  out->job_replica_id = p.second.raiden_id.job_replica_id.c_str();
  out->data_name = p.second.raiden_id.data_name.c_str();
  return KVX_OK;
}

int kvx_slices_flat(kvx_slices* s, const uint8_t** hashes, const int64_t** offsets,
                    const kvx_block_slice** blocks) {
  if (s == nullptr || hashes == nullptr || offsets == nullptr || blocks == nullptr) {
    return Fail(KVX_INVALID_ARGUMENT, "null list or output");
  }
  if (s->offsets.empty()) {
    s->offsets.reserve(s->items.size() + 1);
    s->offsets.push_back(0);
    s->blocks.reserve(s->items.size());
    // Slices with equal owner names share the first one's name pointers, so
    // a binding can recognise the owner by pointer (a store's slices nearly
    // always have one owner). At most kMaxOwners are interned, which bounds
    // the search per slice.
    constexpr size_t kMaxOwners = 16;
    std::vector<const kvx::RaidenId*> owners;
    for (const auto& p : s->items) {
      s->hashes += p.first;
      s->offsets.push_back(static_cast<int64_t>(s->hashes.size()));
      const kvx::RaidenId& id = p.second.raiden_id;
      const kvx::RaidenId* owner = &id;
      for (const kvx::RaidenId* o : owners) {
        if (o->job_name == id.job_name && o->job_replica_id == id.job_replica_id &&
            o->data_name == id.data_name) {
          owner = o;
          break;
        }
      }
      if (owner == &id && owners.size() < kMaxOwners) owners.push_back(owner);
      kvx_block_slice b{};
      b.host_block_id = p.second.host_block_id;
      b.device_block_id = p.second.device_block_id;
      b.status = static_cast<int32_t>(p.second.status);
      b.data_replica_idx = id.data_replica_idx;
      b.job_name = owner->job_name.c_str();
      b.job_replica_id = owner->job_replica_id.c_str();
      b.data_name = owner->data_name.c_str();
      s->blocks.push_back(b);
    }
  }
  *hashes = reinterpret_cast<const uint8_t*>(s->hashes.data());
  *offsets = s->offsets.data();
  *blocks = s->blocks.data();
  return KVX_OK;
}

void kvx_slices_release(kvx_slices* s) { delete s; }

// ---- store --------------------------------------------------------------------

int kvx_store_create(const kvx_store_config* cfg, kvx_store** out) {
  if (cfg == nullptr || out == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null config or output");
  *out = nullptr;
  if (cfg->capacity < 0) return Fail(KVX_INVALID_ARGUMENT, "capacity must be non-negative");
  kvx::StoreOptions o;
  o.capacity = static_cast<size_t>(cfg->capacity);
  o.raiden_id.job_name = Str(cfg->job_name);
  o.raiden_id.job_replica_id = Str(cfg->job_replica_id);
  o.raiden_id.data_name = Str(cfg->data_name);
  o.raiden_id.data_replica_idx = cfg->data_replica_idx;
  o.num_shards = cfg->num_shards;
  o.shard_size_bytes = cfg->shard_size_bytes;
  o.store_server_ip = Str(cfg->store_server_ip);
  o.raiden_controller_port = cfg->raiden_controller_port;
  // NULL fields take the reference's RAIDEN_SHM_* defaults
  // (tpu_sync/kv_cache/kv_cache_store_wrapper.cc:46-58, 116-123); an empty
  // metadata key disables the table.
  o.metadata_shm_key = cfg->metadata_shm_key != nullptr ? std::string(cfg->metadata_shm_key)
                                                        : kvx::MetadataShmKeyFromEnv();
  o.model_uid = cfg->model_uid != nullptr ? std::string(cfg->model_uid)
                                          : kvx::ShmModelUidFromEnv();
  o.recover_at_create = cfg->no_auto_recover == 0;
  if (cfg->host_blocks < 0) return Fail(KVX_INVALID_ARGUMENT, "host_blocks must be non-negative");
  o.host_blocks = static_cast<size_t>(cfg->host_blocks);
  auto r = kvx::KVCacheStore::Create(o);
  if (!r.ok()) return Fail(r.status());
  auto* s = new kvx_store;
  s->impl = std::move(r).value();
  s->lbm_view.lbm = &s->impl->block_manager();
  s->lbm_view.mu = &s->impl->block_manager_mutex();
  *out = s;
  return KVX_OK;
}

void kvx_store_destroy(kvx_store* s) { delete s; }

const char* kvx_store_controller_address(const kvx_store* s) {
  return s == nullptr ? "" : s->impl->raiden_controller_address().c_str();
}
int64_t kvx_store_capacity(const kvx_store* s) {
  return s == nullptr ? 0 : static_cast<int64_t>(s->impl->capacity());
}
int64_t kvx_store_size(const kvx_store* s) {
  return s == nullptr ? 0 : static_cast<int64_t>(s->impl->size());
}
int64_t kvx_store_recovered_blocks(const kvx_store* s) {
  return s == nullptr ? 0 : static_cast<int64_t>(s->impl->recovered_blocks());
}
int32_t kvx_store_metadata_warm(const kvx_store* s) {
  return s != nullptr && s->impl->metadata_warm() ? 1 : 0;
}
kvx_block_manager* kvx_store_host_block_manager(kvx_store* s) {
  return s == nullptr ? nullptr : &s->lbm_view;
}

int kvx_store_lookup(kvx_store* s, const uint8_t* bytes, const int64_t* offsets,
                     int64_t n, int32_t pin_found, kvx_slices** out) {
  if (s == nullptr || out == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null store or output");
  KVX_UNPACK_HASHES(hashes);
  auto r = s->impl->Lookup(hashes, pin_found != 0);
  if (!r.ok()) return Fail(r.status());
  auto* sl = new kvx_slices;
  sl->items = std::move(r).value();
  *out = sl;
  return KVX_OK;
}

int kvx_store_insert(kvx_store* s, const uint8_t* bytes, const int64_t* offsets,
                     int64_t n, const kvx_block_slice* slices, int64_t n_slices,
                     int32_t on_host) {
  if (s == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null store");
  KVX_UNPACK_HASHES(hashes);
  std::vector<kvx::RaidenBlockId> sl;
  if (!ToSlices(slices, n_slices, &sl)) return Fail(KVX_INVALID_ARGUMENT, "malformed slices");
  return Done(s->impl->Insert(hashes, sl, on_host != 0));
}

int kvx_store_release(kvx_store* s, const uint8_t* bytes, const int64_t* offsets,
                      int64_t n) {
  if (s == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null store");
  KVX_UNPACK_HASHES(hashes);
  s->impl->Release(hashes);
  return KVX_OK;
}

int kvx_store_save(kvx_store* s, const uint8_t* bytes, const int64_t* offsets,
                   int64_t n) {
  if (s == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null store");
  KVX_UNPACK_HASHES(hashes);
  return Done(s->impl->Save(hashes));
}

int kvx_store_load(kvx_store* s, const uint8_t* bytes, const int64_t* offsets,
                   int64_t n, const int32_t* device_block_ids, int64_t n_dev) {
  if (s == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null store");
  if (BadArray(device_block_ids, n_dev)) return Fail(KVX_INVALID_ARGUMENT, "null device ids");
  KVX_UNPACK_HASHES(hashes);
  std::vector<int> dev(device_block_ids, device_block_ids + n_dev);
  return Done(s->impl->Load(hashes, dev));
}

int kvx_store_load_slices(kvx_store* s, const uint8_t* bytes, const int64_t* offsets,
                          int64_t n, const kvx_block_slice* slices, int64_t n_slices,
                          const int32_t* device_block_ids, int64_t n_dev) {
  if (s == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null store");
  if (BadArray(device_block_ids, n_dev)) return Fail(KVX_INVALID_ARGUMENT, "null device ids");
  KVX_UNPACK_HASHES(hashes);
  std::vector<kvx::RaidenBlockId> sl;
  if (!ToSlices(slices, n_slices, &sl)) return Fail(KVX_INVALID_ARGUMENT, "malformed slices");
  std::vector<int> dev(device_block_ids, device_block_ids + n_dev);
  return Done(s->impl->Load(hashes, sl, dev));
}

int kvx_store_poll_save_status(kvx_store* s, kvx_strings** out5) {
  if (s == nullptr || out5 == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null store or output");
  auto r = s->impl->PollSaveStatus();
  out5[0] = NewStrings(std::move(r.done));
  out5[1] = NewStrings(std::move(r.failed));
  out5[2] = NewStrings(std::move(r.pending));
  out5[3] = NewStrings(std::move(r.existing));
  out5[4] = NewStrings(std::move(r.unregistered));
  return KVX_OK;
}

int kvx_store_poll_load_status(kvx_store* s, kvx_strings** out3) {
  if (s == nullptr || out3 == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null store or output");
  auto r = s->impl->PollLoadStatus();
  out3[0] = NewStrings(std::move(r.done));
  out3[1] = NewStrings(std::move(r.failed));
  out3[2] = NewStrings(std::move(r.pending));
  return KVX_OK;
}

int32_t kvx_store_pin_count(kvx_store* s, const uint8_t* hash, int64_t len) {
  if (s == nullptr || BadArray(hash, len)) return 0;
  return s->impl->GetPinCount(std::string(reinterpret_cast<const char*>(hash),
                                          static_cast<size_t>(len)));
}

int kvx_store_recover_from_local_manifest(kvx_store* s, int64_t* out_n) {
  if (s == nullptr || out_n == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null store or output");
  auto r = s->impl->RecoverFromLocalManifest();
  if (!r.ok()) return Fail(r.status());
  *out_n = static_cast<int64_t>(r.value());
  return KVX_OK;
}

int kvx_store_candidate_keys(kvx_store* s, kvx_strings** out) {
  if (s == nullptr || out == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null store or output");
  *out = NewStrings(s->impl->GetEvictCandidateKeys());
  return KVX_OK;
}

int kvx_store_evict(kvx_store* s, const uint8_t* bytes, const int64_t* offsets,
                    int64_t n, int64_t* out_evicted) {
  if (s == nullptr || out_evicted == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null store or output");
  KVX_UNPACK_HASHES(hashes);
  *out_evicted = static_cast<int64_t>(s->impl->Evict(hashes));
  return KVX_OK;
}

int kvx_store_set_transfer_fn(kvx_store* s, kvx_transfer_fn fn, void* user) {
  if (s == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null store");
  if (fn == nullptr) {
    s->impl->SetTransferFn(nullptr);
    return KVX_OK;
  }
  s->impl->SetTransferFn([fn, user](bool d2h, const std::vector<int64_t>& src,
                                    const std::vector<int64_t>& dst) -> kvx::Status {
    const int32_t code = fn(user, d2h ? 1 : 0, src.data(), dst.data(),
                            static_cast<int64_t>(src.size()));
    if (code == KVX_OK) return kvx::OkStatus();
    return kvx::Status(static_cast<kvx::Code>(code), "transfer function failed");
  });
  return KVX_OK;
}

int kvx_store_evictable_keys(kvx_store* s, int64_t count, kvx_strings** out) {
  if (s == nullptr || out == nullptr || count < 0) {
    return Fail(KVX_INVALID_ARGUMENT, "null store, output or negative count");
  }
  *out = NewStrings(s->impl->GetEvictableKeys(static_cast<size_t>(count)));
  return KVX_OK;
}

// ---- LRU index ----------------------------------------------------------------

int kvx_lru_create(int64_t capacity, kvx_lru** out) {
  if (out == nullptr || capacity < 0) return Fail(KVX_INVALID_ARGUMENT, "bad capacity or output");
  *out = new kvx_lru(static_cast<size_t>(capacity));
  return KVX_OK;
}
void kvx_lru_destroy(kvx_lru* c) { delete c; }

static std::string Key(const uint8_t* k, int64_t len) {
  return std::string(reinterpret_cast<const char*>(k), static_cast<size_t>(len < 0 ? 0 : len));
}

int kvx_lru_put(kvx_lru* c, const uint8_t* key, int64_t len, int64_t value,
                int32_t* out_evicted, kvx_strings** out_key, int64_t* out_value) {
  if (c == nullptr || BadArray(key, len) || out_evicted == nullptr) {
    return Fail(KVX_INVALID_ARGUMENT, "bad arguments");
  }
  auto ev = c->impl.Put(Key(key, len), value);
  *out_evicted = ev.has_value() ? 1 : 0;
  if (ev.has_value()) {
    if (out_key) *out_key = NewStrings({ev->first});
    if (out_value) *out_value = ev->second;
  }
  return KVX_OK;
}
int kvx_lru_put_back(kvx_lru* c, const uint8_t* key, int64_t len, int64_t value) {
  if (c == nullptr || BadArray(key, len)) return Fail(KVX_INVALID_ARGUMENT, "bad arguments");
  c->impl.PutBack(Key(key, len), value);
  return KVX_OK;
}
// Returns 1 and the value when found (get: promotes; peek: does not, and
// skips candidates; peek_any: includes candidates; get_and_pin: pins).
int32_t kvx_lru_find(kvx_lru* c, int32_t how, const uint8_t* key, int64_t len,
                     int64_t* out_value) {
  if (c == nullptr || BadArray(key, len)) return 0;
  const std::string k = Key(key, len);
  const int64_t* v = nullptr;
  switch (how) {
    case KVX_LRU_GET: v = c->impl.Get(k); break;
    case KVX_LRU_PEEK: v = c->impl.Peek(k); break;
    case KVX_LRU_PEEK_ANY: v = c->impl.PeekIncludingCandidates(k); break;
    case KVX_LRU_GET_AND_PIN: v = c->impl.GetAndPin(k); break;
    default: return 0;
  }
  if (v == nullptr) return 0;
  if (out_value) *out_value = *v;
  return 1;
}
int32_t kvx_lru_contains(kvx_lru* c, const uint8_t* key, int64_t len) {
  return c != nullptr && !BadArray(key, len) && c->impl.Contains(Key(key, len)) ? 1 : 0;
}
int32_t kvx_lru_pin(kvx_lru* c, const uint8_t* key, int64_t len) {
  return c != nullptr && !BadArray(key, len) && c->impl.Pin(Key(key, len)) ? 1 : 0;
}
int32_t kvx_lru_unpin(kvx_lru* c, const uint8_t* key, int64_t len) {
  return c != nullptr && !BadArray(key, len) && c->impl.Unpin(Key(key, len)) ? 1 : 0;
}
int32_t kvx_lru_erase(kvx_lru* c, const uint8_t* key, int64_t len) {
  return c != nullptr && !BadArray(key, len) && c->impl.Erase(Key(key, len)) ? 1 : 0;
}
int32_t kvx_lru_pin_count(kvx_lru* c, const uint8_t* key, int64_t len) {
  return c == nullptr || BadArray(key, len) ? 0 : c->impl.GetPinCount(Key(key, len));
}
int32_t kvx_lru_evict(kvx_lru* c, kvx_strings** out_key, int64_t* out_value) {
  if (c == nullptr) return 0;
  auto ev = c->impl.Evict();
  if (!ev.has_value()) return 0;
  if (out_key) *out_key = NewStrings({ev->first});
  if (out_value) *out_value = ev->second;
  return 1;
}
int kvx_lru_evictable_keys(kvx_lru* c, int64_t count, kvx_strings** out) {
  if (c == nullptr || out == nullptr || count < 0) return Fail(KVX_INVALID_ARGUMENT, "bad arguments");
  *out = NewStrings(c->impl.GetEvictableKeys(static_cast<size_t>(count)));
  return KVX_OK;
}
int kvx_lru_candidate_keys(kvx_lru* c, kvx_strings** out) {
  if (c == nullptr || out == nullptr) return Fail(KVX_INVALID_ARGUMENT, "bad arguments");
  *out = NewStrings(c->impl.GetEvictCandidateKeys());
  return KVX_OK;
}
void kvx_lru_clear(kvx_lru* c) {
  if (c != nullptr) c->impl.Clear();
}
int kvx_lru_sizes(const kvx_lru* c, int64_t* out4) {
  if (c == nullptr || out4 == nullptr) return Fail(KVX_INVALID_ARGUMENT, "bad arguments");
  out4[0] = static_cast<int64_t>(c->impl.capacity());
  out4[1] = static_cast<int64_t>(c->impl.size());
  out4[2] = static_cast<int64_t>(c->impl.active_size());
  out4[3] = static_cast<int64_t>(c->impl.available_space());
  return KVX_OK;
}

// ---- metadata table -----------------------------------------------------------

int64_t kvx_metadata_required_size(int32_t num_blocks) {
  return num_blocks <= 0 ? 0
                         : static_cast<int64_t>(kvx::KVCacheMetadata::RequiredSizeBytes(num_blocks));
}

int kvx_metadata_format(uint8_t* region, int64_t size, int32_t num_blocks,
                        const char* model_uid) {
  if (size < 0) return Fail(KVX_INVALID_ARGUMENT, "negative size");
  auto r = kvx::KVCacheMetadata::Format(region, static_cast<size_t>(size), num_blocks,
                                        Str(model_uid));
  return Done(r.status());
}

int kvx_metadata_attach(uint8_t* region, int64_t size, int32_t num_blocks,
                        const char* model_uid) {
  if (size < 0) return Fail(KVX_INVALID_ARGUMENT, "negative size");
  auto r = kvx::KVCacheMetadata::Attach(region, static_cast<size_t>(size), num_blocks,
                                        Str(model_uid));
  return Done(r.status());
}

// Set / Clear on a region in caller memory (attached under num_blocks and
// model_uid first).
int kvx_metadata_set(uint8_t* region, int64_t size, int32_t num_blocks,
                     const char* model_uid, int32_t block_id, const uint8_t* hash,
                     int64_t hash_len, uint64_t seq) {
  if (size < 0 || BadArray(hash, hash_len)) return Fail(KVX_INVALID_ARGUMENT, "bad arguments");
  auto r = kvx::KVCacheMetadata::Attach(region, static_cast<size_t>(size), num_blocks,
                                        Str(model_uid));
  if (!r.ok()) return Fail(r.status());
  return Done(r->Set(block_id, Key(hash, hash_len), seq));
}

int kvx_metadata_clear(uint8_t* region, int64_t size, int32_t num_blocks,
                       const char* model_uid, int32_t block_id) {
  if (size < 0) return Fail(KVX_INVALID_ARGUMENT, "negative size");
  auto r = kvx::KVCacheMetadata::Attach(region, static_cast<size_t>(size), num_blocks,
                                        Str(model_uid));
  if (!r.ok()) return Fail(r.status());
  return Done(r->Clear(block_id));
}

// Valid entries as three parallel outputs: block ids and seqs (capacity
// num_blocks) and the hashes.
int kvx_metadata_valid_entries(uint8_t* region, int64_t size, int32_t num_blocks,
                               const char* model_uid, int32_t* out_ids,
                               uint64_t* out_seqs, int64_t* out_count,
                               kvx_strings** out_hashes) {
  if (size < 0 || out_count == nullptr || out_hashes == nullptr ||
      (num_blocks > 0 && (out_ids == nullptr || out_seqs == nullptr))) {
    return Fail(KVX_INVALID_ARGUMENT, "bad arguments");
  }
  auto r = kvx::KVCacheMetadata::Attach(region, static_cast<size_t>(size), num_blocks,
                                        Str(model_uid));
  if (!r.ok()) return Fail(r.status());
  std::vector<std::string> hashes;
  int64_t k = 0;
  for (const auto& e : r->ValidEntries()) {
    out_ids[k] = e.block_id;
    out_seqs[k] = e.seq;
    hashes.push_back(e.hash);
    ++k;
  }
  *out_count = k;
  *out_hashes = NewStrings(std::move(hashes));
  return KVX_OK;
}

int kvx_metadata_shm_attach_or_format(const char* shm_key, int32_t num_blocks,
                                      const char* model_uid,
                                      kvx_metadata_region** out, int32_t* out_warm) {
  if (shm_key == nullptr || out == nullptr) return Fail(KVX_INVALID_ARGUMENT, "bad arguments");
  auto r = kvx::KVCacheMetadataShmRegion::AttachOrFormat(shm_key, num_blocks, Str(model_uid));
  if (!r.ok()) return Fail(r.status());
  auto* m = new kvx_metadata_region;
  m->impl = std::move(r).value();
  if (out_warm) *out_warm = m->impl->warm() ? 1 : 0;
  *out = m;
  return KVX_OK;
}

int kvx_metadata_shm_region(kvx_metadata_region* m, uint64_t* out_ptr,
                            int64_t* out_size) {
  if (m == nullptr || out_ptr == nullptr || out_size == nullptr) {
    return Fail(KVX_INVALID_ARGUMENT, "bad arguments");
  }
  *out_ptr = reinterpret_cast<uint64_t>(m->impl->data());
  *out_size = static_cast<int64_t>(m->impl->size());
  return KVX_OK;
}

int kvx_metadata_shm_reformat(kvx_metadata_region* m) {
  if (m == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null region");
  return Done(m->impl->Reformat());
}

void kvx_metadata_shm_release(kvx_metadata_region* m) { delete m; }

}  // extern "C"
