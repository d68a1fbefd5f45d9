#include "kv_cache_metadata.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>

namespace kvx {
namespace {

Status CheckRegion(const uint8_t* region, size_t size, int num_blocks,
                   const std::string& model_uid) {
  if (num_blocks <= 0) {
    return InvalidArgumentError("num_blocks must be positive, got " +
                                std::to_string(num_blocks));
  }
  if (model_uid.size() >= sizeof(KVCacheMetadataHeader::model_uid)) {
    return InvalidArgumentError(
        "model_uid length " + std::to_string(model_uid.size()) +
        " exceeds the maximum of " +
        std::to_string(sizeof(KVCacheMetadataHeader::model_uid) - 1));
  }
  if (region == nullptr) return InvalidArgumentError("Metadata region is null");
  if (reinterpret_cast<uintptr_t>(region) % alignof(KVCacheMetadataHeader) != 0) {
    return InvalidArgumentError("Metadata region must be " +
                                std::to_string(alignof(KVCacheMetadataHeader)) +
                                "-byte aligned");
  }
  const size_t need = KVCacheMetadata::RequiredSizeBytes(num_blocks);
  if (size < need) {
    return InvalidArgumentError("Metadata region too small: " +
                                std::to_string(size) + " bytes, need " +
                                std::to_string(need));
  }
  return OkStatus();
}

size_t PageAligned(size_t n) { return (n + 4095) & ~size_t{4095}; }

}  // namespace

std::string NormalizeShmKey(const std::string& key) {
  return (!key.empty() && key[0] == '/') ? key : "/" + key;
}

size_t KVCacheMetadata::RequiredSizeBytes(int num_blocks) {
  return sizeof(KVCacheMetadataHeader) +
         static_cast<size_t>(num_blocks) * sizeof(KVCacheMetadataEntry);
}

StatusOr<KVCacheMetadata> KVCacheMetadata::Format(uint8_t* region,
                                                  size_t region_size,
                                                  int num_blocks,
                                                  const std::string& model_uid) {
  KVX_RETURN_IF_ERROR(CheckRegion(region, region_size, num_blocks, model_uid));
  std::memset(region, 0, RequiredSizeBytes(num_blocks));
  // Field by field into the zeroed region, so the header's padding (bytes
  // 84-127) is written as zeros rather than copied from a stack object.
  auto* h = reinterpret_cast<KVCacheMetadataHeader*>(region);
  const KVCacheMetadataHeader defaults;
  h->magic = defaults.magic;
  h->version = defaults.version;
  h->num_blocks = static_cast<uint32_t>(num_blocks);
  h->entry_size = sizeof(KVCacheMetadataEntry);
  std::memcpy(h->model_uid, model_uid.data(), model_uid.size());
  return KVCacheMetadata(
      reinterpret_cast<KVCacheMetadataEntry*>(region + sizeof(KVCacheMetadataHeader)),
      num_blocks);
}

StatusOr<KVCacheMetadata> KVCacheMetadata::Attach(uint8_t* region,
                                                  size_t region_size,
                                                  int num_blocks,
                                                  const std::string& model_uid) {
  KVX_RETURN_IF_ERROR(CheckRegion(region, region_size, num_blocks, model_uid));
  const auto* h = reinterpret_cast<const KVCacheMetadataHeader*>(region);
  const KVCacheMetadataHeader want;
  if (h->magic != want.magic) {
    return FailedPreconditionError("Metadata region magic mismatch");
  }
  if (h->version != want.version) {
    return FailedPreconditionError("Metadata region version mismatch: " +
                                   std::to_string(h->version) + " vs " +
                                   std::to_string(want.version));
  }
  if (h->entry_size != sizeof(KVCacheMetadataEntry)) {
    return FailedPreconditionError("Metadata entry size mismatch: " +
                                   std::to_string(h->entry_size) + " vs " +
                                   std::to_string(sizeof(KVCacheMetadataEntry)));
  }
  if (h->num_blocks != static_cast<uint32_t>(num_blocks)) {
    return FailedPreconditionError("Metadata num_blocks mismatch: " +
                                   std::to_string(h->num_blocks) + " vs " +
                                   std::to_string(num_blocks));
  }
  const std::string recorded(h->model_uid, strnlen(h->model_uid, sizeof(h->model_uid)));
  if (recorded != model_uid) {
    return FailedPreconditionError("Metadata model_uid mismatch: \"" + recorded +
                                   "\" vs \"" + model_uid + "\"");
  }
  return KVCacheMetadata(
      reinterpret_cast<KVCacheMetadataEntry*>(region + sizeof(KVCacheMetadataHeader)),
      num_blocks);
}

Status KVCacheMetadata::Set(int block_id, const std::string& hash, uint64_t seq) {
  if (block_id < 0 || block_id >= num_blocks_) {
    return InvalidArgumentError("Block ID out of range: " + std::to_string(block_id));
  }
  if (hash.empty()) return InvalidArgumentError("Hash must not be empty");
  if (hash.size() > kMaxHashLength) {
    return InvalidArgumentError("Hash length " + std::to_string(hash.size()) +
                                " exceeds the maximum of " +
                                std::to_string(kMaxHashLength));
  }
  KVCacheMetadataEntry& e = entries_[block_id];
  // A crash between these stores leaves the slot invalid, never half-written.
  e.valid.store(0, std::memory_order_release);
  e.seq = seq;
  e.hash_len = static_cast<uint16_t>(hash.size());
  std::memcpy(e.hash, hash.data(), hash.size());
  e.valid.store(1, std::memory_order_release);
  return OkStatus();
}

Status KVCacheMetadata::Clear(int block_id) {
  if (block_id < 0 || block_id >= num_blocks_) {
    return InvalidArgumentError("Block ID out of range: " + std::to_string(block_id));
  }
  entries_[block_id].valid.store(0, std::memory_order_release);
  return OkStatus();
}

std::vector<KVCacheMetadata::Entry> KVCacheMetadata::ValidEntries() const {
  std::vector<Entry> out;
  for (int i = 0; i < num_blocks_; ++i) {
    const KVCacheMetadataEntry& e = entries_[i];
    if (e.valid.load(std::memory_order_acquire) == 0) continue;
    if (e.hash_len == 0 || e.hash_len > kMaxHashLength) continue;
    out.push_back(Entry{i, std::string(e.hash, e.hash_len), e.seq});
  }
  return out;
}

StatusOr<std::unique_ptr<KVCacheMetadataShmRegion>>
KVCacheMetadataShmRegion::AttachOrFormat(const std::string& shm_key,
                                         int num_blocks,
                                         const std::string& model_uid) {
  const std::string key = NormalizeShmKey(shm_key);
  if (num_blocks <= 0) {
    return InvalidArgumentError("num_blocks must be positive, got " +
                                std::to_string(num_blocks));
  }
  const size_t size = PageAligned(KVCacheMetadata::RequiredSizeBytes(num_blocks));

  // Warm path: a segment left by an earlier process, if it validates.
  int fd = shm_open(key.c_str(), O_RDWR, 0666);
  if (fd >= 0) {
    struct stat st;
    void* map = MAP_FAILED;
    if (fstat(fd, &st) == 0 && static_cast<size_t>(st.st_size) >= size) {
      map = mmap(nullptr, size, PROT_READ | PROT_WRITE, MAP_SHARED, fd, 0);
    }
    if (map != MAP_FAILED) {
      auto md = KVCacheMetadata::Attach(static_cast<uint8_t*>(map), size,
                                        num_blocks, model_uid);
      if (md.ok()) {
        return std::unique_ptr<KVCacheMetadataShmRegion>(new KVCacheMetadataShmRegion(
            fd, static_cast<uint8_t*>(map), size, md.value(), true, num_blocks,
            model_uid));
      }
      munmap(map, size);
    }
    close(fd);
    shm_unlink(key.c_str());
  }

  // Cold path: a fresh segment with an empty table.
  fd = shm_open(key.c_str(), O_CREAT | O_RDWR, 0666);
  if (fd < 0) {
    return InternalError("shm_open failed to create KV metadata segment " + key +
                         ": " + std::strerror(errno));
  }
  if (ftruncate(fd, static_cast<off_t>(size)) != 0) {
    Status st = InternalError("ftruncate failed on KV metadata segment " + key +
                              ": " + std::strerror(errno));
    close(fd);
    shm_unlink(key.c_str());
    return st;
  }
  void* map = mmap(nullptr, size, PROT_READ | PROT_WRITE, MAP_SHARED, fd, 0);
  if (map == MAP_FAILED) {
    Status st = ResourceExhaustedError("mmap failed on KV metadata segment " +
                                       key + ": " + std::strerror(errno));
    close(fd);
    shm_unlink(key.c_str());
    return st;
  }
  auto md = KVCacheMetadata::Format(static_cast<uint8_t*>(map), size, num_blocks,
                                    model_uid);
  if (!md.ok()) {
    munmap(map, size);
    close(fd);
    shm_unlink(key.c_str());
    return md.status();
  }
  return std::unique_ptr<KVCacheMetadataShmRegion>(new KVCacheMetadataShmRegion(
      fd, static_cast<uint8_t*>(map), size, md.value(), false, num_blocks, model_uid));
}

KVCacheMetadataShmRegion::~KVCacheMetadataShmRegion() {
  munmap(map_, size_);
  close(fd_);
}

Status KVCacheMetadataShmRegion::Reformat() {
  auto md = KVCacheMetadata::Format(map_, size_, num_blocks_, model_uid_);
  if (!md.ok()) return md.status();
  metadata_ = md.value();
  warm_ = false;
  return OkStatus();
}

}  // namespace kvx
