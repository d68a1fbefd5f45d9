#include "host_allocator.h"

#include <fcntl.h>
#include <hip/hip_runtime_api.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstdlib>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "hip_util.h"
#include "numa.h"

namespace kvx {
namespace {

// Writes one byte per 4 KiB page so the pages exist (on the preferred node)
// before the first copy lands; up to 8 threads of at least 256 MiB each.
void FirstTouch(uint8_t* p, size_t bytes) {
  constexpr size_t kPage = 4096;
  constexpr size_t kMinShare = 256u << 20;
  const size_t hw = std::max(1u, std::thread::hardware_concurrency());
  const size_t n = std::max<size_t>(1, std::min<size_t>({8, hw, bytes / kMinShare}));
  const size_t share = (bytes / n + kPage - 1) / kPage * kPage;
  auto touch = [p, bytes](size_t lo, size_t hi) {
    volatile uint8_t* v = p;
    for (size_t i = lo; i < hi && i < bytes; i += kPage) v[i] = 0;
  };
  std::vector<std::thread> ts;
  for (size_t t = 1; t < n; ++t) ts.emplace_back(touch, t * share, (t + 1) * share);
  touch(0, share);
  for (std::thread& t : ts) t.join();
}

}  // namespace

StatusOr<HostBufferAllocation> AllocateMallocHost(size_t bytes, int numa_node) {
  HostBufferAllocation a;
  if (bytes == 0) return a;
  ScopedNumaPreference prefer(numa_node);
  void* p = nullptr;
  if (posix_memalign(&p, 64, bytes) != 0) {
    return ResourceExhaustedError("Failed to allocate host buffer of size: " +
                                  std::to_string(bytes));
  }
  std::memset(p, 0, bytes);
  a.ptr = static_cast<uint8_t*>(p);
  a.size = bytes;
  a.owner = std::shared_ptr<void>(p, [](void* q) { free(q); });
  return a;
}

StatusOr<HostBufferAllocation> AllocatePinnedHost(size_t bytes, int device, int numa_node) {
  HostBufferAllocation a;
  if (bytes == 0) return a;
  DeviceGuard g(device);
  ScopedNumaPreference prefer(numa_node);
  void* p = nullptr;
  hipError_t e = hipHostMalloc(&p, bytes, prefer.active() ? hipHostMallocNumaUser
                                                          : hipHostMallocDefault);
  if (e != hipSuccess) {
    return ResourceExhaustedError("hipHostMalloc of " + std::to_string(bytes) +
                                  " bytes failed: " + hipGetErrorString(e));
  }
  std::memset(p, 0, bytes);
  a.ptr = static_cast<uint8_t*>(p);
  a.size = bytes;
  a.owner = std::shared_ptr<void>(p, [](void* q) { (void)hipHostFree(q); });
  return a;
}

std::string ShmSegmentName(const std::string& key, const std::string& server_name,
                           int device) {
  std::string name = key;
  if (!server_name.empty()) name += "_" + server_name;
  if (device >= 0) name += "_dev_" + std::to_string(device);
  if (name.empty() || name[0] != '/') name.insert(0, "/");
  return name;
}

namespace {

bool SchemaMatches(const SharedMemoryHeader& h, const SharedMemoryHeader& want,
                   size_t bytes) {
  return h.magic == want.magic && h.version == want.version &&
         strncmp(h.model_uid, want.model_uid, sizeof(h.model_uid)) == 0 &&
         h.num_blocks == want.num_blocks && h.block_size == want.block_size &&
         h.num_heads == want.num_heads && h.head_dim == want.head_dim &&
         h.itemsize == want.itemsize && h.total_payload_bytes == bytes;
}

struct ShmMapping {
  int fd = -1;
  void* map = nullptr;
  size_t size = 0;
  ~ShmMapping() {
    if (map != nullptr) {
      auto* h = static_cast<SharedMemoryHeader*>(map);
      if (h->reference_count > 0) --h->reference_count;
      munmap(map, size);
    }
    if (fd >= 0) close(fd);
  }
};

}  // namespace

StatusOr<HostBufferAllocation> AllocateShmHost(const std::string& name,
                                               const SharedMemoryHeader& expected,
                                               size_t bytes, bool* warm, int numa_node) {
  const size_t total =
      (sizeof(SharedMemoryHeader) + ((bytes + 4095) & ~size_t{4095}) + 4095) &
      ~size_t{4095};
  *warm = false;
  int fd = shm_open(name.c_str(), O_RDWR, 0666);
  if (fd >= 0) {
    struct stat st;
    bool ok = fstat(fd, &st) == 0 && static_cast<size_t>(st.st_size) >= total;
    if (ok) {
      void* hp = mmap(nullptr, sizeof(SharedMemoryHeader), PROT_READ, MAP_SHARED, fd, 0);
      ok = hp != MAP_FAILED &&
           SchemaMatches(*static_cast<SharedMemoryHeader*>(hp), expected, bytes);
      if (hp != MAP_FAILED) munmap(hp, sizeof(SharedMemoryHeader));
    }
    if (ok) {
      *warm = true;
    } else {
      close(fd);
      fd = -1;
      shm_unlink(name.c_str());
    }
  }
  if (fd < 0) {
    fd = shm_open(name.c_str(), O_CREAT | O_RDWR, 0666);
    if (fd < 0) {
      return InternalError("shm_open failed to create segment " + name + ": " +
                           std::strerror(errno));
    }
    if (ftruncate(fd, static_cast<off_t>(total)) != 0) {
      Status st = InternalError("ftruncate failed on shm segment " + name + ": " +
                                std::strerror(errno));
      close(fd);
      shm_unlink(name.c_str());
      return st;
    }
  }
  auto m = std::make_shared<ShmMapping>();
  m->fd = fd;
  void* map = mmap(nullptr, total, PROT_READ | PROT_WRITE, MAP_SHARED, fd, 0);
  if (map == MAP_FAILED) {
    return ResourceExhaustedError("mmap failed on shm segment " + name + ": " +
                                  std::strerror(errno));
  }
  m->map = map;
  m->size = total;
  KVX_RETURN_IF_ERROR(PreferNodeForRange(map, total, numa_node));
  auto* h = static_cast<SharedMemoryHeader*>(map);
  if (*warm) {
    ++h->reference_count;
  } else {
    // A fresh segment reads as zeros; write the schema field by field (the
    // padding stays zero) and take the first reference.
    h->magic = expected.magic;
    h->version = expected.version;
    std::memcpy(h->model_uid, expected.model_uid, sizeof(h->model_uid));
    std::memcpy(h->global_mesh_shape, expected.global_mesh_shape,
                sizeof(h->global_mesh_shape));
    std::memcpy(h->shard_layout, expected.shard_layout, sizeof(h->shard_layout));
    h->num_blocks = expected.num_blocks;
    h->block_size = expected.block_size;
    h->num_heads = expected.num_heads;
    h->head_dim = expected.head_dim;
    h->itemsize = expected.itemsize;
    h->total_payload_bytes = bytes;
    h->reference_count = 1;
    // host_memory_allocator.cc:388-392: a fresh segment is faulted in at
    // creation, so copies never pay the page faults.
    FirstTouch(static_cast<uint8_t*>(map) + sizeof(SharedMemoryHeader), bytes);
  }
  HostBufferAllocation a;
  a.ptr = static_cast<uint8_t*>(map) + sizeof(SharedMemoryHeader);
  a.size = bytes;
  a.owner = m;
  return a;
}

}  // namespace kvx
