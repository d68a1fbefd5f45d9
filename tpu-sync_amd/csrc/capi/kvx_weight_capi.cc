// extern "C" layer over the weight synchronizer and the strided-entry copy.
#include <algorithm>
#include <memory>
#include <string>
#include <vector>

#include "../host/device_memory.h"
#include "../host/weight_synchronizer.h"
#include "capi_internal.h"

struct kvx_weight_sync {
  std::unique_ptr<kvx::WeightSynchronizer> impl;
};

struct kvx_strided_plan {
  std::unique_ptr<kvx::StridedCopyPlan> impl;
};

namespace {

using kvx_capi::BadArray;
using kvx_capi::Done;
using kvx_capi::Fail;

int Emit(kvx::StatusOr<kvx::CopyFuture> r, kvx_future** out) {
  if (!r.ok()) return Fail(r.status());
  *out = new kvx_future{std::move(r).value()};
  return KVX_OK;
}

// Validates the C entries and converts them (offsets folded into addresses):
// every row an entry reads or writes must lie in device memory of `device`.
int ToCopies(int32_t device, const kvx_strided_entry* entries, int64_t n,
             std::vector<kvx::StridedCopy>* out) {
  if (BadArray(entries, n)) return Fail(KVX_INVALID_ARGUMENT, "bad arguments");
  kvx::DeviceRangeChecker ranges(device);
  out->assign(static_cast<size_t>(n), kvx::StridedCopy{});
  for (int64_t i = 0; i < n; ++i) {
    const kvx_strided_entry& e = entries[i];
    if (e.size_bytes <= 0 || e.src_stride_bytes < 0 || e.dst_stride_bytes < 0) {
      return Fail(KVX_INVALID_ARGUMENT, "entry sizes and strides must be non-negative, size > 0");
    }
    const int64_t count = e.count > 0 ? e.count : 1;
    // Rows of one entry must not overlap in the destination.
    if (count > 1 && e.dst_stride_bytes < e.size_bytes) {
      return Fail(KVX_INVALID_ARGUMENT, "destination rows overlap (dst_stride < size)");
    }
    kvx::StridedCopy& c = (*out)[static_cast<size_t>(i)];
    c.src = e.src + static_cast<uint64_t>(e.src_offset_bytes);
    c.dst = e.dst + static_cast<uint64_t>(e.dst_offset_bytes);
    c.size = e.size_bytes;
    c.count = count;
    c.src_stride = e.src_stride_bytes;
    c.dst_stride = e.dst_stride_bytes;
    uint64_t src_bytes = 0, dst_bytes = 0;
    if (!kvx::StridedExtent(c.size, count, c.src_stride, &src_bytes) ||
        !kvx::StridedExtent(c.size, count, c.dst_stride, &dst_bytes)) {
      return Fail(KVX_INVALID_ARGUMENT, "entry extent overflows");
    }
    kvx::Status st = ranges.Check(c.src, src_bytes, "strided entry source");
    if (st.ok()) st = ranges.Check(c.dst, dst_bytes, "strided entry destination");
    if (!st.ok()) {
      return Fail(kvx::InvalidArgumentError("entry " + std::to_string(i) + ": " + st.message()));
    }
  }
  return KVX_OK;
}

// Validates a C layout and converts it.
int ToLayout(const kvx_tiled_layout* l, kvx::TiledLayout* out) {
  if (l == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null layout");
  if (l->rank < 0 || l->rank > KVX_TILED_MAX_RANK || l->num_tiles < 0 ||
      l->num_tiles > KVX_TILED_MAX_TILES) {
    return Fail(KVX_INVALID_ARGUMENT, "tiled layout: rank or tile count out of range");
  }
  out->itemsize = l->itemsize;
  out->dims.assign(l->dims, l->dims + l->rank);
  out->minor_to_major.assign(l->minor_to_major, l->minor_to_major + l->rank);
  out->tiles.clear();
  for (int t = 0; t < l->num_tiles; ++t) {
    const int32_t k = l->tile_rank[t];
    if (k < 1 || k > KVX_TILED_MAX_RANK) {
      return Fail(KVX_INVALID_ARGUMENT, "tiled layout: a tile has 1 to 8 dimensions");
    }
    out->tiles.emplace_back(l->tile_dims[t], l->tile_dims[t] + k);
  }
  return KVX_OK;
}

// The packed image a Pack writes / an Unpack reads must be device memory of
// the synchronizer's device.
int CheckStaging(const kvx::WeightSynchronizer& w, uint64_t staging, int64_t staging_bytes) {
  if (staging_bytes < 0) return Fail(KVX_INVALID_ARGUMENT, "negative staging_bytes");
  const int64_t used = std::min<int64_t>(staging_bytes, w.total_bytes());
  kvx::Status st = kvx::CheckDeviceRange(w.device(), staging, static_cast<uint64_t>(used),
                                         "staging");
  return st.ok() ? KVX_OK : Fail(st);
}

int TileCall(int32_t device, const kvx_tiled_layout* layout, uint64_t linear, uint64_t tiled,
             bool tile, void* stream, kvx_future** out) {
  if (out == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null output");
  kvx::TiledLayout l;
  const int rc = ToLayout(layout, &l);
  if (rc != KVX_OK) return rc;
  auto plan = kvx::PlanTiled(l);
  if (!plan.ok()) return Fail(plan.status());
  // Both buffers are device memory (the reference's TileBuffer / DetileBuffer
  // take host buffers; these run in HBM).
  kvx::DeviceRangeChecker ranges(device);
  kvx::Status st = ranges.Check(linear, static_cast<uint64_t>(plan->logical_bytes),
                                tile ? "src_linear" : "dst_linear");
  if (st.ok()) {
    st = ranges.Check(tiled, static_cast<uint64_t>(plan->tiled_bytes),
                      tile ? "dst_tiled" : "src_tiled");
  }
  if (!st.ok()) return Fail(st);
  return Emit(kvx::TileOnDevice(device, plan.value(), linear, tiled, tile,
                                static_cast<hipStream_t>(stream)),
              out);
}

}  // namespace

extern "C" {

int kvx_tiled_buffer_elements(const kvx_tiled_layout* layout, int64_t* out) {
  if (out == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null output");
  kvx::TiledLayout l;
  const int rc = ToLayout(layout, &l);
  if (rc != KVX_OK) return rc;
  auto n = kvx::TiledBufferElements(l);
  if (!n.ok()) return Fail(n.status());
  *out = n.value();
  return KVX_OK;
}

int kvx_tile_buffer(int32_t device, const kvx_tiled_layout* layout, uint64_t src_linear,
                    uint64_t dst_tiled, void* stream, kvx_future** out) {
  return TileCall(device, layout, src_linear, dst_tiled, true, stream, out);
}

int kvx_detile_buffer(int32_t device, const kvx_tiled_layout* layout, uint64_t src_tiled,
                      uint64_t dst_linear, void* stream, kvx_future** out) {
  return TileCall(device, layout, dst_linear, src_tiled, false, stream, out);
}

int kvx_weight_sync_create(const kvx_weight_sync_config* cfg, kvx_weight_sync** out) {
  if (cfg == nullptr || out == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null config or output");
  *out = nullptr;
  if (cfg->num_layers < 0 || cfg->num_shards <= 0) {
    return Fail(KVX_INVALID_ARGUMENT, "num_layers must be >= 0 and num_shards >= 1");
  }
  const int64_t n = cfg->num_layers * cfg->num_shards;
  if (BadArray(cfg->device_ptrs, n) || BadArray(cfg->device_bytes, n)) {
    return Fail(KVX_INVALID_ARGUMENT, "null device_ptrs or device_bytes");
  }
  kvx::WeightSyncConfig c;
  c.device = cfg->device;
  c.num_layers = cfg->num_layers;
  c.num_shards = cfg->num_shards;
  c.device_ptrs.assign(cfg->device_ptrs, cfg->device_ptrs + n);
  c.device_bytes.assign(cfg->device_bytes, cfg->device_bytes + n);
  kvx::DeviceRangeChecker ranges(cfg->device);
  for (int64_t k = 0; k < n; ++k) {
    if (c.device_bytes[k] < 0) return Fail(KVX_INVALID_ARGUMENT, "negative device_bytes");
    kvx::Status st = ranges.Check(c.device_ptrs[k], static_cast<uint64_t>(c.device_bytes[k]),
                                  ("device_ptrs[" + std::to_string(k) + "]").c_str());
    if (!st.ok()) return Fail(st);
  }
  if (cfg->host_alloc != KVX_HOST_PINNED && cfg->host_alloc != KVX_HOST_MALLOC) {
    return Fail(KVX_INVALID_ARGUMENT, "weight sync host memory must be pinned or malloc");
  }
  c.host_alloc = static_cast<kvx::HostAllocKind>(cfg->host_alloc);
  if (cfg->chunk_bytes > 0) c.chunk_bytes = cfg->chunk_bytes;
  if (cfg->staging_chunks > 0) c.staging_chunks = static_cast<int>(cfg->staging_chunks);
  c.profile_kernels = cfg->profile_kernels != 0;
  c.numa_local = cfg->numa_off == 0;
  if (cfg->layouts != nullptr) {
    c.tiled.resize(static_cast<size_t>(n));
    for (int64_t k = 0; k < n; ++k) {
      if (cfg->layouts[k].num_tiles == 0) continue;
      kvx::TiledLayout l;
      const int rc = ToLayout(&cfg->layouts[k], &l);
      if (rc != KVX_OK) return rc;
      auto plan = kvx::PlanTiled(l);
      if (!plan.ok()) return Fail(plan.status());
      c.tiled[static_cast<size_t>(k)] =
          std::make_shared<const kvx::TiledPlan>(std::move(plan).value());
    }
  }
  auto r = kvx::WeightSynchronizer::Create(std::move(c));
  if (!r.ok()) return Fail(r.status());
  *out = new kvx_weight_sync{std::move(r).value()};
  return KVX_OK;
}

void kvx_weight_sync_destroy(kvx_weight_sync* w) { delete w; }

int kvx_weight_sync_d2h(kvx_weight_sync* w, void* stream, kvx_future** out) {
  if (w == nullptr || out == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null handle or output");
  return Emit(w->impl->D2h(static_cast<hipStream_t>(stream)), out);
}

int kvx_weight_sync_h2d(kvx_weight_sync* w, void* stream, kvx_future** out) {
  if (w == nullptr || out == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null handle or output");
  return Emit(w->impl->H2d(static_cast<hipStream_t>(stream)), out);
}

int kvx_weight_sync_d2h_layer(kvx_weight_sync* w, int64_t layer, void* stream,
                              kvx_future** out) {
  if (w == nullptr || out == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null handle or output");
  return Emit(w->impl->D2hLayer(layer, static_cast<hipStream_t>(stream)), out);
}

int kvx_weight_sync_h2d_layer(kvx_weight_sync* w, int64_t layer, void* stream,
                              kvx_future** out) {
  if (w == nullptr || out == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null handle or output");
  return Emit(w->impl->H2dLayer(layer, static_cast<hipStream_t>(stream)), out);
}

int kvx_weight_sync_pack(kvx_weight_sync* w, uint64_t staging, int64_t staging_bytes,
                         void* stream, kvx_future** out) {
  if (w == nullptr || out == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null handle or output");
  if (const int rc = CheckStaging(*w->impl, staging, staging_bytes); rc != KVX_OK) return rc;
  return Emit(w->impl->Pack(staging, staging_bytes, static_cast<hipStream_t>(stream)), out);
}

int kvx_weight_sync_unpack(kvx_weight_sync* w, uint64_t staging, int64_t staging_bytes,
                           void* stream, kvx_future** out) {
  if (w == nullptr || out == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null handle or output");
  if (const int rc = CheckStaging(*w->impl, staging, staging_bytes); rc != KVX_OK) return rc;
  return Emit(w->impl->Unpack(staging, staging_bytes, static_cast<hipStream_t>(stream)), out);
}

int64_t kvx_weight_sync_total_bytes(const kvx_weight_sync* w) {
  return w == nullptr ? 0 : w->impl->total_bytes();
}

int kvx_weight_sync_host_buffer(kvx_weight_sync* w, int64_t layer, int64_t shard,
                                uint64_t* out_ptr, int64_t* out_bytes, int64_t* out_offset) {
  if (w == nullptr || out_ptr == nullptr || out_bytes == nullptr || out_offset == nullptr) {
    return Fail(KVX_INVALID_ARGUMENT, "null handle or output");
  }
  if (layer < 0 || layer >= w->impl->num_layers() || shard < 0 ||
      shard >= w->impl->num_shards()) {
    return Fail(KVX_OUT_OF_RANGE, "layer or shard index out of range");
  }
  *out_offset = w->impl->offset(layer, shard);
  *out_ptr = reinterpret_cast<uint64_t>(w->impl->host_base() + *out_offset);
  *out_bytes = w->impl->size(layer, shard);
  return KVX_OK;
}

uint64_t kvx_weight_sync_host_base(const kvx_weight_sync* w) {
  return w == nullptr ? 0 : reinterpret_cast<uint64_t>(w->impl->host_base());
}

int kvx_weight_sync_wait(kvx_weight_sync* w) {
  if (w == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null handle");
  return Done(w->impl->Synchronize());
}

int kvx_weight_sync_kernel_times(kvx_weight_sync* w, int32_t pack, int32_t reset,
                                 int64_t* out_launches, double* out_ms, int64_t* out_bytes) {
  if (w == nullptr || out_launches == nullptr || out_ms == nullptr || out_bytes == nullptr) {
    return Fail(KVX_INVALID_ARGUMENT, "null handle or output");
  }
  return Done(w->impl->KernelTimes(pack != 0, reset != 0, out_launches, out_ms, out_bytes));
}

int kvx_copy_strided(int32_t device, const kvx_strided_entry* entries, int64_t n,
                     void* stream, kvx_future** out) {
  if (out == nullptr) return Fail(KVX_INVALID_ARGUMENT, "bad arguments");
  std::vector<kvx::StridedCopy> copies;
  const int rc = ToCopies(device, entries, n, &copies);
  if (rc != KVX_OK) return rc;
  return Emit(kvx::CopyStridedOnDevice(device, copies, static_cast<hipStream_t>(stream)), out);
}

int kvx_strided_plan_create(int32_t device, const kvx_strided_entry* entries, int64_t n,
                            kvx_strided_plan** out) {
  if (out == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null output");
  *out = nullptr;
  std::vector<kvx::StridedCopy> copies;
  const int rc = ToCopies(device, entries, n, &copies);
  if (rc != KVX_OK) return rc;
  auto p = kvx::StridedCopyPlan::Create(device, copies);
  if (!p.ok()) return Fail(p.status());
  *out = new kvx_strided_plan{std::move(p).value()};
  return KVX_OK;
}

int kvx_strided_plan_run(kvx_strided_plan* p, void* stream, kvx_future** out) {
  if (p == nullptr || out == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null handle or output");
  return Emit(p->impl->Run(static_cast<hipStream_t>(stream)), out);
}

void kvx_strided_plan_destroy(kvx_strided_plan* p) { delete p; }

int kvx_strided_plan_profile(kvx_strided_plan* p, int32_t on) {
  if (p == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null handle");
  p->impl->SetProfiling(on != 0);
  return KVX_OK;
}

int kvx_strided_plan_kernel_times(kvx_strided_plan* p, int32_t reset, int64_t* out_launches,
                                  double* out_total_ms, int64_t* out_bytes) {
  if (p == nullptr || out_launches == nullptr || out_total_ms == nullptr || out_bytes == nullptr) {
    return Fail(KVX_INVALID_ARGUMENT, "null handle or output");
  }
  return Done(p->impl->KernelTimes(reset != 0, out_launches, out_total_ms, out_bytes));
}

}  // extern "C"
