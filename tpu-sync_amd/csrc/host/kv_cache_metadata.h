// Crash-persistent mirror of the host tier's LRU index: one fixed-size slot
// per host block, recording which prefix hash the block holds and a recency
// stamp, kept in POSIX shared memory next to the host KV pool so a restarted
// engine can rebuild its index without re-reading any block.
//
// The byte layout is a persistent format and is identical to the
// reference's (tpu_sync/kv_cache/kv_cache_metadata.h:34-70): a 128-byte
// header {magic "RAIDENKM", version 1, num_blocks, entry_size 128,
// model_uid[64]} followed by 128-byte entries {seq u64, hash_len u16,
// valid u8 (committed last with release ordering), reserved[5],
// hash[112]} indexed by host block id. A table written by either side can
// therefore be attached by the other.
//
// KVCacheMetadata is a non-owning view; KVCacheMetadataShmRegion owns the
// shared-memory mapping (reference: tpu_sync/kv_cache/kv_cache_metadata_shm.h:
// 33-86). Not thread-safe: the store serialises access.
#ifndef KVX_HOST_KV_CACHE_METADATA_H_
#define KVX_HOST_KV_CACHE_METADATA_H_

#include <atomic>
#include <cstddef>
#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "status.h"

namespace kvx {

struct alignas(64) KVCacheMetadataHeader {
  uint64_t magic = 0x52414944454E4B4Dull;  // "RAIDENKM"
  uint32_t version = 1;
  uint32_t num_blocks = 0;
  uint32_t entry_size = 0;
  char model_uid[64] = {0};
};
static_assert(sizeof(KVCacheMetadataHeader) == 128, "on-memory format");
static_assert(offsetof(KVCacheMetadataHeader, model_uid) == 20, "on-memory format");

struct alignas(64) KVCacheMetadataEntry {
  uint64_t seq = 0;
  uint16_t hash_len = 0;
  std::atomic<uint8_t> valid{0};
  uint8_t reserved[5] = {0};
  char hash[112] = {0};
};
static_assert(sizeof(KVCacheMetadataEntry) == 128, "on-memory format");
static_assert(offsetof(KVCacheMetadataEntry, valid) == 10, "on-memory format");
static_assert(offsetof(KVCacheMetadataEntry, hash) == 16, "on-memory format");
static_assert(std::atomic<uint8_t>::is_always_lock_free, "valid byte");

class KVCacheMetadata {
 public:
  static constexpr size_t kMaxHashLength = sizeof(KVCacheMetadataEntry::hash);

  struct Entry {
    int block_id;
    std::string hash;
    uint64_t seq;
  };

  static size_t RequiredSizeBytes(int num_blocks);
  // Cold start: writes an empty table for num_blocks blocks of model_uid.
  static StatusOr<KVCacheMetadata> Format(uint8_t* region, size_t region_size,
                                          int num_blocks,
                                          const std::string& model_uid);
  // Warm start: validates magic, version, entry size, num_blocks and
  // model_uid of a previously formatted region.
  static StatusOr<KVCacheMetadata> Attach(uint8_t* region, size_t region_size,
                                          int num_blocks,
                                          const std::string& model_uid);

  // Binds block_id to hash with recency stamp seq (invalidate, write, then
  // commit the valid byte last).
  Status Set(int block_id, const std::string& hash, uint64_t seq);
  Status Clear(int block_id);
  std::vector<Entry> ValidEntries() const;
  int num_blocks() const { return num_blocks_; }

 private:
  KVCacheMetadata(KVCacheMetadataEntry* e, int n) : entries_(e), num_blocks_(n) {}
  KVCacheMetadataEntry* entries_;
  int num_blocks_;
};

// Owns the shared-memory segment that backs a metadata table. AttachOrFormat
// attaches to a surviving table under `shm_key` (a leading '/' is added) or,
// if the segment is missing, too small or fails validation, re-creates it
// and formats an empty table. The segment is never unlinked here: it must
// outlive the process to be recoverable.
class KVCacheMetadataShmRegion {
 public:
  static StatusOr<std::unique_ptr<KVCacheMetadataShmRegion>> AttachOrFormat(
      const std::string& shm_key, int num_blocks, const std::string& model_uid);
  ~KVCacheMetadataShmRegion();
  KVCacheMetadataShmRegion(const KVCacheMetadataShmRegion&) = delete;
  KVCacheMetadataShmRegion& operator=(const KVCacheMetadataShmRegion&) = delete;

  KVCacheMetadata& metadata() { return metadata_; }
  // True when the table survived from an earlier process.
  bool warm() const { return warm_; }
  // Empties the table in place (fallback to a cold start).
  Status Reformat();
  // The mapped segment (header first).
  uint8_t* data() const { return map_; }
  size_t size() const { return size_; }

 private:
  KVCacheMetadataShmRegion(int fd, uint8_t* map, size_t size,
                           KVCacheMetadata md, bool warm, int num_blocks,
                           std::string model_uid)
      : fd_(fd), map_(map), size_(size), metadata_(md), warm_(warm),
        num_blocks_(num_blocks), model_uid_(std::move(model_uid)) {}
  int fd_;
  uint8_t* map_;
  size_t size_;
  KVCacheMetadata metadata_;
  bool warm_;
  int num_blocks_;
  std::string model_uid_;
};

// "/name" form of a POSIX shared-memory key.
std::string NormalizeShmKey(const std::string& key);

}  // namespace kvx

#endif  // KVX_HOST_KV_CACHE_METADATA_H_
