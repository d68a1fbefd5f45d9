// extern "C" layer over the C++ manager, futures and block allocator.
// Each entry point validates its arguments, calls the C++ object and turns
// a Status into its code plus a thread-local message.
#include <algorithm>
#include <cstring>
#include <memory>
#include <optional>
#include <string>
#include <vector>

#include "../host/device_memory.h"
#include "../host/hip_util.h"
#include "../host/kv_cache_store.h"
#include "../host/link_peaks.h"
#include "../host/numa.h"
#include "../host/queue_check.h"
#include "../host/raiden_env.h"
#include "../kernels/block_copy.h"
#include "capi_internal.h"

namespace {
thread_local std::string g_last_error;
}  // namespace

namespace kvx_capi {

int Fail(const kvx::Status& s) {
  g_last_error = s.message();
  return static_cast<int>(s.code());
}

int Fail(int code, const char* msg) {
  g_last_error = msg;
  return code;
}

int Done(const kvx::Status& s) {
  if (!s.ok()) return Fail(s);
  return KVX_OK;
}

}  // namespace kvx_capi

namespace {

using kvx_capi::BadArray;
using kvx_capi::Done;
using kvx_capi::Fail;

std::vector<int64_t> Vec(const int64_t* p, int64_t n) {
  if (p == nullptr || n <= 0) return {};
  return std::vector<int64_t>(p, p + n);
}

std::optional<int64_t> Opt(int64_t v) {
  return v < 0 ? std::nullopt : std::optional<int64_t>(v);
}

std::optional<size_t> OptIdx(int64_t v) {
  return v < 0 ? std::nullopt : std::optional<size_t>(static_cast<size_t>(v));
}


int EmitFuture(kvx::StatusOr<kvx::CopyFuture> r, kvx_future** out) {
  if (!r.ok()) return Fail(r.status());
  *out = new kvx_future{std::move(r).value()};
  return KVX_OK;
}

struct LbmLock {
  explicit LbmLock(kvx_block_manager* b) : mu(b->mu) {
    if (mu) mu->lock();
  }
  ~LbmLock() {
    if (mu) mu->unlock();
  }
  std::mutex* mu;
};

}  // namespace

extern "C" {

const char* kvx_last_error(void) { return g_last_error.c_str(); }

const char* kvx_version(void) { return "kvx 0.1.0 gfx950"; }

int kvx_manager_create(const kvx_manager_config* cfg, kvx_manager** out) {
  if (cfg == nullptr || out == nullptr) {
    return Fail(KVX_INVALID_ARGUMENT, "null config or output");
  }
  *out = nullptr;
  kvx::ManagerConfig c;
  c.device = cfg->device;
  c.num_layers = cfg->num_layers;
  c.num_shards = cfg->num_shards;
  const int64_t nstor = cfg->num_layers * cfg->num_shards;
  if (cfg->num_layers < 0 || cfg->num_shards < 0) {
    return Fail(KVX_INVALID_ARGUMENT, "num_layers and num_shards must be non-negative");
  }
  if (cfg->device_ptrs != nullptr) {
    if (cfg->device_bytes == nullptr) {
      return Fail(KVX_INVALID_ARGUMENT, "device_bytes is required with device_ptrs");
    }
    c.device_ptrs.assign(cfg->device_ptrs, cfg->device_ptrs + nstor);
    c.device_bytes.assign(cfg->device_bytes, cfg->device_bytes + nstor);
  }
  c.major_dim = cfg->major_dim;
  c.slice_byte_size = cfg->slice_byte_size;
  c.host_blocks = cfg->host_blocks;
  if (cfg->host_alloc < KVX_HOST_MALLOC || cfg->host_alloc > KVX_HOST_AUTO) {
    return Fail(KVX_INVALID_ARGUMENT, "unknown host_alloc kind");
  }
  // The reference picks the shared-memory allocator, its key and schema uid
  // from RAIDEN_SHM_* (tpu_sync/core/utils.h:48-91); fields left NULL here
  // take those defaults.
  const std::string key = cfg->shm_key != nullptr ? cfg->shm_key : "";
  int32_t kind = cfg->host_alloc;
  if (kind == KVX_HOST_AUTO) {
    kind = !key.empty() || !kvx::ShmKeyFromEnv().empty() ? KVX_HOST_SHM : KVX_HOST_PINNED;
  }
  c.host_alloc = static_cast<kvx::HostAllocKind>(kind);
  if (kind == KVX_HOST_SHM) {
    c.shm_key = !key.empty() ? key : kvx::ShmKeyFromEnv();
    c.shm_server_name = cfg->shm_server_name != nullptr ? std::string(cfg->shm_server_name)
                                                        : kvx::ShmServerNameFromEnv();
    c.model_uid = cfg->model_uid != nullptr ? std::string(cfg->model_uid)
                                            : kvx::ShmModelUidFromEnv();
  }
  if (cfg->staging_chunk_bytes > 0) c.engine.staging_chunk_bytes = cfg->staging_chunk_bytes;
  if (cfg->staging_chunks > 0) c.engine.staging_chunks = static_cast<int>(cfg->staging_chunks);
  if (cfg->direct_min_bytes > 0) c.engine.direct_min_bytes = cfg->direct_min_bytes;
  c.engine.profile_kernels = cfg->profile_kernels != 0;
  if (cfg->transfer_mode < KVX_MODE_AUTO || cfg->transfer_mode > KVX_MODE_LANES) {
    return Fail(KVX_INVALID_ARGUMENT, "unknown transfer_mode");
  }
  if (cfg->transfer_mode == KVX_MODE_LANES && cfg->host_copy_threads < 0) {
    return Fail(KVX_INVALID_ARGUMENT, "transfer_mode lanes needs host copy threads");
  }
  if (cfg->transfer_mode == KVX_MODE_ZERO_COPY && kind != KVX_HOST_PINNED) {
    return Fail(KVX_INVALID_ARGUMENT, "zero-copy transfers need KVX_HOST_PINNED host memory");
  }
  c.engine.mode = static_cast<kvx::TransferMode>(cfg->transfer_mode);
  switch (cfg->dispatch) {
    case KVX_DISPATCH_ENV:
      c.dispatch = kvx::ManagerConfig::Dispatch::kEnv;
      break;
    case KVX_DISPATCH_QUEUED:
      c.dispatch = kvx::ManagerConfig::Dispatch::kQueued;
      break;
    case KVX_DISPATCH_INLINE:
      c.dispatch = kvx::ManagerConfig::Dispatch::kInline;
      break;
    default:
      return Fail(KVX_INVALID_ARGUMENT, "unknown dispatch mode");
  }
  switch (cfg->numa_policy) {
    case KVX_NUMA_AUTO:
      c.numa = kvx::ManagerConfig::Numa::kAuto;
      break;
    case KVX_NUMA_OFF:
      c.numa = kvx::ManagerConfig::Numa::kOff;
      break;
    case KVX_NUMA_NODE:
      c.numa = kvx::ManagerConfig::Numa::kNode;
      c.numa_node = cfg->numa_node;
      break;
    default:
      return Fail(KVX_INVALID_ARGUMENT, "unknown numa_policy");
  }
  if (cfg->host_copy_threads > 64) {
    return Fail(KVX_INVALID_ARGUMENT, "host_copy_threads must be at most 64");
  }
  if (cfg->host_copy_threads != 0) {
    c.engine.host_copy_threads = cfg->host_copy_threads < 0 ? 0 : cfg->host_copy_threads;
  }
  if (cfg->gather_workgroups_per_cu < -1 || cfg->gather_workgroups_per_cu > 32) {
    return Fail(KVX_INVALID_ARGUMENT, "gather_workgroups_per_cu must be -1, 0 or 1..32");
  }
  if (cfg->gather_workgroups_per_cu != 0) {
    c.engine.gather_workgroups_per_cu =
        cfg->gather_workgroups_per_cu < 0 ? 0 : cfg->gather_workgroups_per_cu;
  }
  if (cfg->zero_copy_workgroups > 0) {
    c.engine.zero_copy_d2h_workgroups = cfg->zero_copy_workgroups;
    c.engine.zero_copy_h2d_workgroups = cfg->zero_copy_workgroups;
  }
  const bool device_backed = cfg->device_ptrs != nullptr;
  const int device = c.device;
  // Every storage must be device memory of cfg->device covering its bytes
  // (checked before anything is allocated or issued).
  kvx::DeviceRangeChecker ranges(device);
  for (size_t k = 0; k < c.device_ptrs.size(); ++k) {
    if (c.device_bytes[k] < 0) return Fail(KVX_INVALID_ARGUMENT, "negative device_bytes");
    kvx::Status st = ranges.Check(c.device_ptrs[k], static_cast<uint64_t>(c.device_bytes[k]),
                                  ("device_ptrs[" + std::to_string(k) + "]").c_str());
    if (!st.ok()) return Fail(st);
  }
  auto r = kvx::KVCacheManager::Create(std::move(c));
  if (!r.ok()) return Fail(r.status());
  if (device_backed) {
    // Set-up of kvx_manager_gather_no_alloc on this device.
    kvx::DeviceGuard dg(device);
    kvx::Status st = dg.ok() ? kvx::InitNoAllocScratch(device)
                             : kvx::InternalError("hipSetDevice failed");
    if (!st.ok()) return Fail(st);
  }
  auto* m = new kvx_manager;
  m->impl = std::move(r).value();
  m->lbm_view.lbm = m->impl->host_block_manager();
  m->lbm_view.mu = &m->impl->host_block_mutex();
  *out = m;
  return KVX_OK;
}

void kvx_manager_destroy(kvx_manager* m) {
  if (m == nullptr) return;
  kvx::UnregisterWorker(m->impl.get());
  delete m;
}

int kvx_manager_register_with_controller(kvx_manager* m, const char* address) {
  if (m == nullptr || address == nullptr) {
    return Fail(KVX_INVALID_ARGUMENT, "null manager or address");
  }
  return Done(kvx::RegisterWorkerAtController(address, m->impl.get()));
}

int32_t kvx_manager_shm_warm(const kvx_manager* m) {
  return m != nullptr && m->impl->shm_warm() ? 1 : 0;
}

int32_t kvx_manager_host_alloc(const kvx_manager* m) {
  return m == nullptr ? -1 : static_cast<int32_t>(m->impl->host_alloc());
}

int32_t kvx_manager_numa_node(const kvx_manager* m) {
  return m == nullptr ? -1 : m->impl->assigned_numa_node();
}

int32_t kvx_manager_queued_dispatch(const kvx_manager* m) {
  return m != nullptr && m->impl->queued_dispatch() ? 1 : 0;
}

int kvx_manager_dispatch_log(kvx_manager* m, char* out, int64_t cap, int64_t* n_out) {
  if (m == nullptr || n_out == nullptr || BadArray(out, cap)) {
    return Fail(KVX_INVALID_ARGUMENT, "null argument");
  }
  const std::string log = m->impl->DispatchLog();
  *n_out = static_cast<int64_t>(log.size());
  std::memcpy(out, log.data(), std::min<size_t>(log.size(), static_cast<size_t>(cap)));
  return KVX_OK;
}

int32_t kvx_gpu_numa_node(int32_t device) { return kvx::GpuNumaNode(device); }

int32_t kvx_host_page_numa_node(uint64_t addr) {
  return addr == 0 ? -1 : kvx::PageNumaNode(reinterpret_cast<const void*>(addr));
}

int kvx_numa_pin_current_thread(int32_t node) {
  return Done(kvx::PinCurrentThreadToNumaNode(node));
}

static int Transfer(bool d2h, kvx_manager* m, const int64_t* src, int64_t n_src,
                    const int64_t* dst, int64_t n_dst, const int64_t* sizes,
                    int64_t n_sizes, int64_t slot_idx, int64_t layer_idx,
                    int64_t shard_idx, void* stream, kvx_future** out) {
  if (m == nullptr || out == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null manager or output");
  if (BadArray(src, n_src) || BadArray(dst, n_dst) || BadArray(sizes, n_sizes)) {
    return Fail(KVX_INVALID_ARGUMENT, "null array with a positive length");
  }
  auto s = Vec(src, n_src);
  auto d = Vec(dst, n_dst);
  auto z = Vec(sizes, n_sizes);
  hipStream_t st = static_cast<hipStream_t>(stream);
  auto r = d2h ? m->impl->D2h(s, d, z, Opt(slot_idx), OptIdx(layer_idx),
                              OptIdx(shard_idx), st)
               : m->impl->H2d(s, d, z, Opt(slot_idx), OptIdx(layer_idx),
                              OptIdx(shard_idx), st);
  return EmitFuture(std::move(r), out);
}

int kvx_manager_d2h(kvx_manager* m, const int64_t* src, int64_t n_src,
                    const int64_t* dst, int64_t n_dst, const int64_t* sizes,
                    int64_t n_sizes, int64_t slot_idx, int64_t layer_idx,
                    int64_t shard_idx, void* stream, kvx_future** out) {
  return Transfer(true, m, src, n_src, dst, n_dst, sizes, n_sizes, slot_idx,
                  layer_idx, shard_idx, stream, out);
}

int kvx_manager_h2d(kvx_manager* m, const int64_t* src, int64_t n_src,
                    const int64_t* dst, int64_t n_dst, const int64_t* sizes,
                    int64_t n_sizes, int64_t slot_idx, int64_t layer_idx,
                    int64_t shard_idx, void* stream, kvx_future** out) {
  return Transfer(false, m, src, n_src, dst, n_dst, sizes, n_sizes, slot_idx,
                  layer_idx, shard_idx, stream, out);
}

int kvx_manager_d2h_auto_allocate(kvx_manager* m, const int64_t* src,
                                  int64_t n_src, const int64_t* sizes,
                                  int64_t n_sizes, int32_t* out_ids,
                                  int64_t out_capacity, int64_t* out_num_ids,
                                  void* stream, kvx_future** out) {
  if (m == nullptr || out == nullptr || out_num_ids == nullptr) {
    return Fail(KVX_INVALID_ARGUMENT, "null manager or output");
  }
  if (BadArray(src, n_src) || BadArray(sizes, n_sizes)) {
    return Fail(KVX_INVALID_ARGUMENT, "null array with a positive length");
  }
  int64_t total = 0;
  for (int64_t i = 0; i < n_sizes; ++i) total += sizes[i] > 0 ? sizes[i] : 0;
  if (out_capacity < total || (total > 0 && out_ids == nullptr)) {
    return Fail(KVX_INVALID_ARGUMENT, "out_ids capacity smaller than sum(sizes)");
  }
  auto r = m->impl->D2hAutoAllocate(Vec(src, n_src), Vec(sizes, n_sizes),
                                    static_cast<hipStream_t>(stream));
  if (!r.ok()) return Fail(r.status());
  auto& ids = r->first;
  for (size_t i = 0; i < ids.size(); ++i) out_ids[i] = ids[i];
  *out_num_ids = static_cast<int64_t>(ids.size());
  *out = new kvx_future{std::move(r->second)};
  return KVX_OK;
}

static int DeviceCopy(bool gather, kvx_manager* m, const int64_t* ids,
                      int64_t n, uint64_t staging, int64_t staging_bytes,
                      int32_t order, int64_t layer_idx, int64_t shard_idx,
                      void* stream, kvx_future** out) {
  if (m == nullptr || out == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null manager or output");
  if (BadArray(ids, n)) return Fail(KVX_INVALID_ARGUMENT, "null ids with a positive length");
  if (order != KVX_LAYER_MAJOR && order != KVX_BLOCK_MAJOR) {
    return Fail(KVX_INVALID_ARGUMENT, "unknown staging order");
  }
  if (staging_bytes < 0) return Fail(KVX_INVALID_ARGUMENT, "negative staging_bytes");
  kvx::Status chk = kvx::CheckDeviceRange(m->impl->device(), staging,
                                          static_cast<uint64_t>(staging_bytes), "staging");
  if (!chk.ok()) return Fail(chk);
  hipStream_t st = static_cast<hipStream_t>(stream);
  auto v = Vec(ids, n);
  auto r = gather ? m->impl->Gather(v, staging, staging_bytes, order == KVX_BLOCK_MAJOR,
                                    OptIdx(layer_idx), OptIdx(shard_idx), st)
                  : m->impl->Scatter(v, staging, staging_bytes, order == KVX_BLOCK_MAJOR,
                                     OptIdx(layer_idx), OptIdx(shard_idx), st);
  return EmitFuture(std::move(r), out);
}

int kvx_manager_gather(kvx_manager* m, const int64_t* ids, int64_t n,
                       uint64_t staging, int64_t staging_bytes, int32_t order,
                       int64_t layer_idx, int64_t shard_idx, void* stream,
                       kvx_future** out) {
  return DeviceCopy(true, m, ids, n, staging, staging_bytes, order, layer_idx,
                    shard_idx, stream, out);
}

int kvx_manager_scatter(kvx_manager* m, const int64_t* ids, int64_t n,
                        uint64_t staging, int64_t staging_bytes, int32_t order,
                        int64_t layer_idx, int64_t shard_idx, void* stream,
                        kvx_future** out) {
  return DeviceCopy(false, m, ids, n, staging, staging_bytes, order, layer_idx,
                    shard_idx, stream, out);
}

int kvx_manager_configure_host_staging_slots(kvx_manager* m, int64_t num_slots,
                                             int64_t max_major_per_slot) {
  if (m == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null manager");
  return Done(m->impl->ConfigureHostStagingSlots(num_slots, max_major_per_slot));
}

int kvx_manager_host_span(kvx_manager* m, int64_t layer_idx, int64_t shard_idx,
                          int64_t slot_idx, int64_t num_major,
                          uint64_t* out_ptr, int64_t* out_nbytes,
                          int64_t* out_base_major) {
  if (m == nullptr || out_ptr == nullptr || out_nbytes == nullptr) {
    return Fail(KVX_INVALID_ARGUMENT, "null manager or output");
  }
  if (layer_idx < 0 || shard_idx < 0) {
    return Fail(KVX_OUT_OF_RANGE, "HostSpan layer or shard index out of range");
  }
  auto r = m->impl->HostSpan(static_cast<size_t>(layer_idx),
                             static_cast<size_t>(shard_idx), slot_idx, num_major);
  if (!r.ok()) return Fail(r.status());
  *out_ptr = reinterpret_cast<uint64_t>(r->ptr);
  *out_nbytes = static_cast<int64_t>(r->nbytes);
  if (out_base_major) *out_base_major = r->base_major;
  return KVX_OK;
}

int kvx_manager_block_host_ptr(kvx_manager* m, int64_t layer_idx,
                               int64_t shard_idx, int32_t block_id,
                               uint64_t* out_ptr) {
  if (m == nullptr || out_ptr == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null manager or output");
  if (layer_idx < 0 || shard_idx < 0) {
    return Fail(KVX_OUT_OF_RANGE, "layer or shard index out of range");
  }
  auto r = m->impl->GetBlockHostPointerValue(static_cast<size_t>(layer_idx),
                                             static_cast<size_t>(shard_idx), block_id);
  if (!r.ok()) return Fail(r.status());
  *out_ptr = static_cast<uint64_t>(r.value());
  return KVX_OK;
}

int kvx_manager_read_block(kvx_manager* m, int64_t layer_idx, int32_t block_id,
                           int64_t shard_idx, void* buf, int64_t len) {
  if (m == nullptr || buf == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null manager or buffer");
  if (layer_idx < 0 || shard_idx < 0) {
    return Fail(KVX_OUT_OF_RANGE, "layer or shard index out of range");
  }
  auto r = m->impl->ReadBlockBytes(static_cast<size_t>(layer_idx), block_id,
                                   static_cast<size_t>(shard_idx));
  if (!r.ok()) return Fail(r.status());
  if (static_cast<int64_t>(r->size()) != len) {
    return Fail(KVX_INVALID_ARGUMENT, "buffer length must equal the block size");
  }
  std::memcpy(buf, r->data(), r->size());
  return KVX_OK;
}

int kvx_manager_write_block(kvx_manager* m, int64_t layer_idx,
                            int32_t block_id, int64_t shard_idx,
                            const void* buf, int64_t len) {
  if (m == nullptr || (buf == nullptr && len > 0)) {
    return Fail(KVX_INVALID_ARGUMENT, "null manager or buffer");
  }
  if (layer_idx < 0 || shard_idx < 0 || len < 0) {
    return Fail(KVX_OUT_OF_RANGE, "layer or shard index out of range");
  }
  return Done(m->impl->WriteBlockBytes(static_cast<size_t>(layer_idx), block_id,
                                       buf, static_cast<size_t>(len),
                                       static_cast<size_t>(shard_idx)));
}

int64_t kvx_manager_num_layers(const kvx_manager* m) {
  return m ? static_cast<int64_t>(m->impl->num_layers()) : -1;
}
int64_t kvx_manager_num_shards(const kvx_manager* m) {
  return m ? static_cast<int64_t>(m->impl->num_shards()) : -1;
}
int64_t kvx_manager_major_dim(const kvx_manager* m) {
  return m ? m->impl->major_dim() : -1;
}
int64_t kvx_manager_host_blocks(const kvx_manager* m) {
  return m ? m->impl->host_blocks() : -1;
}
int64_t kvx_manager_bytes_per_block(const kvx_manager* m) {
  return m ? static_cast<int64_t>(m->impl->bytes_per_block()) : -1;
}
int64_t kvx_manager_layer_block_byte_size(const kvx_manager* m, int64_t layer_idx) {
  if (m == nullptr || layer_idx < 0) return -1;
  return m->impl->LayerBlockByteSize(static_cast<size_t>(layer_idx));
}
uint64_t kvx_manager_host_ptr(kvx_manager* m, int64_t layer_idx, int64_t shard_idx) {
  if (m == nullptr || layer_idx < 0 || shard_idx < 0) return 0;
  return reinterpret_cast<uint64_t>(
      m->impl->GetHostPointer(static_cast<size_t>(layer_idx), static_cast<size_t>(shard_idx)));
}
int64_t kvx_manager_host_size(kvx_manager* m, int64_t layer_idx, int64_t shard_idx) {
  if (m == nullptr || layer_idx < 0 || shard_idx < 0) return 0;
  return static_cast<int64_t>(
      m->impl->GetHostSize(static_cast<size_t>(layer_idx), static_cast<size_t>(shard_idx)));
}
uint64_t kvx_manager_block_array_block_ptr(kvx_manager* m, int64_t block_array_idx,
                                           int64_t shard_idx, int64_t block_id) {
  if (m == nullptr || block_array_idx < 0 || shard_idx < 0) return 0;
  return reinterpret_cast<uint64_t>(m->impl->GetBlockHostPointer(
      static_cast<size_t>(block_array_idx), static_cast<size_t>(shard_idx), block_id));
}
int kvx_manager_block_chunks(kvx_manager* m, int64_t block_array_idx, int64_t shard_idx,
                             const int64_t* block_ids, int64_t n, int64_t total_bytes,
                             uint64_t* out_ptrs, int64_t* out_sizes, int64_t cap,
                             int64_t* n_out) {
  if (m == nullptr || n_out == nullptr || BadArray(block_ids, n) || BadArray(out_ptrs, cap) ||
      BadArray(out_sizes, cap) || block_array_idx < 0 || shard_idx < 0 || total_bytes < 0) {
    return Fail(KVX_INVALID_ARGUMENT, "invalid argument");
  }
  const auto chunks = m->impl->GetBlockChunks(
      static_cast<size_t>(block_array_idx), static_cast<size_t>(shard_idx),
      std::vector<int64_t>(block_ids, block_ids + n), static_cast<size_t>(total_bytes));
  *n_out = static_cast<int64_t>(chunks.size());
  for (int64_t i = 0; i < *n_out && i < cap; ++i) {
    out_ptrs[i] = reinterpret_cast<uint64_t>(chunks[static_cast<size_t>(i)].ptr);
    out_sizes[i] = static_cast<int64_t>(chunks[static_cast<size_t>(i)].size);
  }
  return KVX_OK;
}
int64_t kvx_manager_num_block_arrays(const kvx_manager* m) {
  return m ? static_cast<int64_t>(m->impl->num_block_arrays()) : -1;
}
int64_t kvx_manager_block_bytes(const kvx_manager* m, int64_t block_array_idx) {
  if (m == nullptr || block_array_idx < 0) return -1;
  return static_cast<int64_t>(m->impl->block_bytes(static_cast<size_t>(block_array_idx)));
}
uint64_t kvx_manager_block_array_host_ptr(kvx_manager* m, int64_t block_array_idx,
                                          int64_t shard_idx) {
  if (m == nullptr || block_array_idx < 0 || shard_idx < 0) return 0;
  return reinterpret_cast<uint64_t>(m->impl->GetBlockArrayHostPointer(
      static_cast<size_t>(block_array_idx), static_cast<size_t>(shard_idx)));
}
int64_t kvx_manager_block_array_host_size(kvx_manager* m, int64_t block_array_idx,
                                          int64_t shard_idx) {
  if (m == nullptr || block_array_idx < 0 || shard_idx < 0) return 0;
  return static_cast<int64_t>(m->impl->GetBlockArrayHostSize(
      static_cast<size_t>(block_array_idx), static_cast<size_t>(shard_idx)));
}
int64_t kvx_manager_allocated_host_bytes(const kvx_manager* m) {
  return m ? static_cast<int64_t>(m->impl->GetAllocatedHostDramBytes()) : -1;
}
int kvx_manager_wait_for_pending_work(kvx_manager* m) {
  if (m == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null manager");
  return Done(m->impl->WaitForPendingWork());
}
int kvx_manager_engine_stats(kvx_manager* m, int64_t* out8) {
  if (m == nullptr || out8 == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null manager or output");
  if (m->impl->engine() == nullptr) {
    return Fail(KVX_FAILED_PRECONDITION, "CPU-only manager has no transfer engine");
  }
  kvx::EngineStats s = m->impl->engine()->stats();
  out8[0] = s.direct_copies;
  out8[1] = s.staged_copies;
  out8[2] = s.memcpy_calls;
  out8[3] = s.kernel_launches;
  out8[4] = s.chunks;
  out8[5] = s.zero_copy_copies;
  out8[6] = s.extent_kernel_copies;
  out8[7] = s.bounce_copies;
  return KVX_OK;
}
int32_t kvx_manager_lane_dma_engines(kvx_manager* m) {
  if (m == nullptr || m->impl->engine() == nullptr) return -1;
  return static_cast<int32_t>(m->impl->engine()->LaneDmaEngines());
}
int kvx_manager_stream_placement(kvx_manager* m, int32_t* out2) {
  if (m == nullptr || out2 == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null manager or output");
  if (m->impl->engine() == nullptr) {
    return Fail(KVX_FAILED_PRECONDITION, "CPU-only manager has no transfer engine");
  }
  const kvx::StreamPlacement p = m->impl->engine()->placement();
  out2[0] = p.serialized_pairs;
  out2[1] = p.attempts;
  return KVX_OK;
}
int kvx_probe_stream_queues(const uint64_t* streams, int32_t n, int32_t* pairs_out) {
  if (pairs_out == nullptr || (streams == nullptr && n > 0)) {
    return Fail(KVX_INVALID_ARGUMENT, "null streams or output");
  }
  if (n < 0 || n > 64) return Fail(KVX_INVALID_ARGUMENT, "stream probe takes 0..64 streams");
  std::vector<hipStream_t> ss(static_cast<size_t>(n));
  for (int32_t i = 0; i < n; ++i) ss[i] = reinterpret_cast<hipStream_t>(streams[i]);
  auto pairs = kvx::SerializedStreamPairs(ss);
  if (!pairs.ok()) return Fail(pairs.status());
  *pairs_out = static_cast<int32_t>(pairs->size());
  return KVX_OK;
}

int kvx_measure_link_peaks(uint64_t bytes, int32_t reps, double* out3,
                           uint32_t* engines_out) {
  if (out3 == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null output");
  auto r = kvx::MeasureLinkPeaks(static_cast<size_t>(bytes), reps);
  if (!r.ok()) return Fail(r.status());
  out3[0] = r->d2h_gbps;
  out3[1] = r->h2d_gbps;
  out3[2] = r->bidir_gbps;
  if (engines_out != nullptr) *engines_out = r->engines;
  return KVX_OK;
}

int kvx_manager_kernel_times(kvx_manager* m, int32_t gather, int32_t reset,
                             int64_t* out_launches, double* out_total_ms,
                             int64_t* out_bytes) {
  if (m == nullptr || out_launches == nullptr || out_total_ms == nullptr ||
      out_bytes == nullptr) {
    return Fail(KVX_INVALID_ARGUMENT, "null manager or output");
  }
  if (m->impl->engine() == nullptr) {
    return Fail(KVX_FAILED_PRECONDITION, "CPU-only manager has no transfer engine");
  }
  auto r = m->impl->engine()->ProfiledKernelTimes(gather != 0, reset != 0);
  if (!r.ok()) return Fail(r.status());
  *out_launches = r->launches;
  *out_total_ms = r->total_ms;
  *out_bytes = r->bytes;
  return KVX_OK;
}

int kvx_future_is_ready(kvx_future* f) { return f && f->f.IsReady() ? 1 : 0; }
int kvx_future_poll_error(kvx_future* f) {
  if (f == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null future");
  return Done(f->f.PollError());
}
int kvx_future_await(kvx_future* f) {
  if (f == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null future");
  return Done(f->f.Await());
}
int kvx_future_wait_on_stream(kvx_future* f, void* stream) {
  if (f == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null future");
  return Done(f->f.WaitOnStream(static_cast<hipStream_t>(stream)));
}
int kvx_future_on_ready(kvx_future* f, kvx_ready_fn cb, void* user) {
  if (f == nullptr || cb == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null future or callback");
  f->f.OnReady([cb, user](kvx::Status st) { cb(user, static_cast<int32_t>(st.code())); });
  return KVX_OK;
}
void kvx_future_release(kvx_future* f) { delete f; }

int kvx_block_manager_create(int32_t num_blocks, kvx_block_manager** out) {
  if (out == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null output");
  if (num_blocks < 0) return Fail(KVX_INVALID_ARGUMENT, "num_blocks must be non-negative");
  auto* b = new kvx_block_manager;
  b->owned = std::make_unique<kvx::LogicalBlockManager>(num_blocks);
  b->lbm = b->owned.get();
  *out = b;
  return KVX_OK;
}

void kvx_block_manager_destroy(kvx_block_manager* b) {
  if (b != nullptr && b->owned) delete b;
}

kvx_block_manager* kvx_manager_host_block_manager(kvx_manager* m) {
  return m == nullptr ? nullptr : &m->lbm_view;
}

static std::vector<int> Ids(const int32_t* ids, int64_t n) {
  if (ids == nullptr || n <= 0) return {};
  return std::vector<int>(ids, ids + n);
}

int kvx_block_manager_allocate(kvx_block_manager* b, int32_t n, int32_t lock,
                               int32_t* out_ids) {
  if (b == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null block manager");
  LbmLock l(b);
  auto r = b->lbm->Allocate(n, lock != 0);
  if (!r.ok()) return Fail(r.status());
  if (out_ids == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null output");
  for (size_t i = 0; i < r->size(); ++i) out_ids[i] = (*r)[i];
  return KVX_OK;
}
int kvx_block_manager_allocate_target(kvx_block_manager* b, const int32_t* ids,
                                      int64_t n) {
  if (b == nullptr || BadArray(ids, n)) return Fail(KVX_INVALID_ARGUMENT, "null argument");
  LbmLock l(b);
  return Done(b->lbm->AllocateTarget(Ids(ids, n)));
}
int kvx_block_manager_unlock(kvx_block_manager* b, const int32_t* ids, int64_t n) {
  if (b == nullptr || BadArray(ids, n)) return Fail(KVX_INVALID_ARGUMENT, "null argument");
  LbmLock l(b);
  return Done(b->lbm->Unlock(Ids(ids, n)));
}
int kvx_block_manager_deallocate(kvx_block_manager* b, const int32_t* ids,
                                 int64_t n) {
  if (b == nullptr || BadArray(ids, n)) return Fail(KVX_INVALID_ARGUMENT, "null argument");
  LbmLock l(b);
  return Done(b->lbm->Deallocate(Ids(ids, n)));
}
int kvx_block_manager_access(kvx_block_manager* b, int32_t id) {
  if (b == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null block manager");
  LbmLock l(b);
  return Done(b->lbm->AccessBlock(id));
}
int32_t kvx_block_manager_is_allocated(kvx_block_manager* b, int32_t id) {
  if (b == nullptr) return 0;
  LbmLock l(b);
  return b->lbm->IsAllocated(id) ? 1 : 0;
}
int32_t kvx_block_manager_is_locked(kvx_block_manager* b, int32_t id) {
  if (b == nullptr) return 0;
  LbmLock l(b);
  return b->lbm->IsLocked(id) ? 1 : 0;
}
int32_t kvx_block_manager_total_blocks(kvx_block_manager* b) {
  if (b == nullptr) return -1;
  LbmLock l(b);
  return b->lbm->total_blocks();
}
int32_t kvx_block_manager_num_free(kvx_block_manager* b) {
  if (b == nullptr) return -1;
  LbmLock l(b);
  return b->lbm->num_free_blocks();
}
int32_t kvx_block_manager_num_allocated(kvx_block_manager* b) {
  if (b == nullptr) return -1;
  LbmLock l(b);
  return b->lbm->num_allocated_blocks();
}
int32_t kvx_block_manager_num_locked(kvx_block_manager* b) {
  if (b == nullptr) return -1;
  LbmLock l(b);
  return b->lbm->num_locked_blocks();
}

static int RawCopy(bool gather, uint64_t storage_table, int64_t num_storages,
                   int64_t block_bytes, int64_t pool_blocks, uint64_t ids,
                   int64_t n, uint64_t staging, int32_t order, uint64_t error,
                   void* stream) {
  if (storage_table == 0 || ids == 0 || staging == 0) {
    return Fail(KVX_INVALID_ARGUMENT, "null device pointer");
  }
  if (num_storages <= 0 || n <= 0 || block_bytes <= 0 || pool_blocks <= 0) {
    return Fail(KVX_INVALID_ARGUMENT, "sizes must be positive");
  }
  if (order != KVX_LAYER_MAJOR && order != KVX_BLOCK_MAJOR) {
    return Fail(KVX_INVALID_ARGUMENT, "unknown staging order");
  }
  // Bounds first, then the product as a division: no signed overflow.
  if (n > INT32_MAX || num_storages > static_cast<int64_t>(UINT32_MAX) ||
      static_cast<uint64_t>(num_storages) > UINT32_MAX / static_cast<uint64_t>(n)) {
    return Fail(KVX_INVALID_ARGUMENT, "too many blocks for one launch");
  }
  // Every table and buffer on one device (the storage bases inside the
  // table are device data the host does not read).
  kvx::DeviceRangeChecker ranges(-1);
  const uint64_t W = static_cast<uint64_t>(num_storages), N = static_cast<uint64_t>(n);
  uint64_t staging_bytes = 0;
  if (__builtin_mul_overflow(W * N, static_cast<uint64_t>(block_bytes), &staging_bytes)) {
    return Fail(KVX_INVALID_ARGUMENT, "staging size overflows");
  }
  kvx::Status chk = ranges.Check(storage_table, W * 8, "storage_table");
  if (chk.ok()) chk = ranges.Check(ids, N * 8, "ids");
  if (chk.ok()) chk = ranges.Check(staging, staging_bytes, "staging");
  if (chk.ok()) chk = ranges.Check(error, error != 0 ? 4 : 0, "error");
  if (!chk.ok()) return Fail(chk);
  kvx::CopyLaunch l;
  l.npieces = 1;
  l.ids = reinterpret_cast<const int64_t*>(ids);
  l.n = n;
  l.error = reinterpret_cast<int32_t*>(error);
  kvx::CopyPiece& p = l.pieces[0];
  p.storages = storage_table;
  p.staging = staging;
  p.stride_w = order == KVX_BLOCK_MAJOR ? block_bytes : n * block_bytes;
  p.stride_i = order == KVX_BLOCK_MAJOR ? num_storages * block_bytes : block_bytes;
  p.f0 = 0;
  p.nblocks = num_storages * n;
  p.block_bytes = block_bytes;
  p.pool_blocks = pool_blocks;
  // The storage bases are device data the host cannot inspect; the vector
  // width follows block_bytes and staging. gfx950 global memory accepts
  // unaligned vector accesses, so a base that is not 16-byte aligned is slower
  // but still copied exactly.
  const int vec = kvx::LaunchVectorBytes(l, 0);
  hipError_t e = kvx::LaunchBlockCopy(
      l, gather ? kvx::CopyDir::kGather : kvx::CopyDir::kScatter, vec,
      static_cast<hipStream_t>(stream));
  if (e != hipSuccess) {
    g_last_error = std::string("kernel launch failed: ") + hipGetErrorString(e);
    return e == hipErrorInvalidValue ? KVX_INVALID_ARGUMENT : KVX_INTERNAL;
  }
  return KVX_OK;
}

int kvx_gather_blocks(uint64_t storage_table, int64_t num_storages,
                      int64_t block_bytes, int64_t pool_blocks, uint64_t ids,
                      int64_t n, uint64_t staging, int32_t order, uint64_t error,
                      void* stream) {
  return RawCopy(true, storage_table, num_storages, block_bytes, pool_blocks,
                 ids, n, staging, order, error, stream);
}

int kvx_scatter_blocks(uint64_t storage_table, int64_t num_storages,
                       int64_t block_bytes, int64_t pool_blocks, uint64_t ids,
                       int64_t n, uint64_t staging, int32_t order,
                       uint64_t error, void* stream) {
  return RawCopy(false, storage_table, num_storages, block_bytes, pool_blocks,
                 ids, n, staging, order, error, stream);
}

}  // extern "C"
