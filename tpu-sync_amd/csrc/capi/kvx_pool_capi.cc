// extern "C" surface of the block-pool geometry and the manager's pool table
// (declared in include/kvx.h).
#include <cstdint>
#include <limits>
#include <optional>
#include <string>
#include <vector>

#include "../host/pool_layout.h"
#include "capi_internal.h"

using kvx_capi::BadArray;
using kvx_capi::Done;
using kvx_capi::Fail;

namespace {

kvx::Status ToPool(const kvx_pool_spec* in, kvx::PoolSpec* out) {
  if (in == nullptr) return kvx::InvalidArgumentError("null pool spec");
  if (BadArray(in->regions, in->num_regions)) {
    return kvx::InvalidArgumentError("null regions with a positive count");
  }
  if (in->storage_index < 0) {
    return kvx::InvalidArgumentError("pool " + std::string(in->tag ? in->tag : "") +
                                     " storage_index must be non-negative");
  }
  out->tag = in->tag ? in->tag : "";
  out->storage_index = static_cast<size_t>(in->storage_index);
  out->base_offset_bytes = in->base_offset_bytes;
  out->block_stride_bytes = in->block_stride_bytes;
  out->num_blocks = in->num_blocks;
  out->dtype_tag = in->dtype_tag ? in->dtype_tag : "";
  out->regions.clear();
  for (int64_t i = 0; i < in->num_regions; ++i) {
    const kvx_region_spec& r = in->regions[i];
    kvx::RegionSpec s;
    s.name = r.name ? r.name : "";
    s.offset_bytes = r.offset_bytes;
    s.stride_bytes = r.stride_bytes;
    s.unit_bytes = r.unit_bytes;
    s.num_units = r.num_units;
    s.units_per_stride = r.units_per_stride;
    out->regions.push_back(std::move(s));
  }
  return kvx::OkStatus();
}

template <typename T, typename F>
int Emit(const std::vector<T>& items, int per, int64_t* out, int64_t cap, int64_t* n_out,
         F fields) {
  if (n_out == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null count output");
  if (cap < 0 || (cap > 0 && out == nullptr)) {
    return Fail(KVX_INVALID_ARGUMENT, "null output with a positive capacity");
  }
  *n_out = static_cast<int64_t>(items.size());
  for (size_t i = 0; i < items.size() && static_cast<int64_t>(i) < cap; ++i) {
    fields(items[i], out + per * i);
  }
  return KVX_OK;
}

}  // namespace

extern "C" {

int kvx_pool_validate(const kvx_pool_spec* pool, int64_t storage_bytes) {
  kvx::PoolSpec p;
  kvx::Status st = ToPool(pool, &p);
  if (!st.ok()) return Fail(st);
  return Done(p.Validate(storage_bytes));
}

int64_t kvx_pool_storage_extent_end(const kvx_pool_spec* pool) {
  kvx::PoolSpec p;
  if (!ToPool(pool, &p).ok()) return std::numeric_limits<int64_t>::max();
  return p.storage_extent_end_bytes();
}

int kvx_pool_copy_extents(const kvx_pool_spec* pool, const int64_t* block_ids, int64_t n,
                          int64_t* out, int64_t cap, int64_t* n_out) {
  if (BadArray(block_ids, n)) return Fail(KVX_INVALID_ARGUMENT, "null block ids");
  kvx::PoolSpec p;
  kvx::Status st = ToPool(pool, &p);
  if (!st.ok()) return Fail(st);
  auto r = kvx::ComputePoolBlockCopyExtents(p, std::vector<int64_t>(block_ids, block_ids + n));
  if (!r.ok()) return Fail(r.status());
  return Emit(*r, 2, out, cap, n_out, [](const kvx::PoolBlockCopyExtent& e, int64_t* o) {
    o[0] = e.offset_bytes;
    o[1] = e.size_bytes;
  });
}

int kvx_pool_live_segments(const kvx_pool_spec* pool, int64_t* out, int64_t cap,
                           int64_t* n_out) {
  kvx::PoolSpec p;
  kvx::Status st = ToPool(pool, &p);
  if (!st.ok()) return Fail(st);
  auto r = kvx::ExpandPoolLiveSegments(p);
  if (!r.ok()) return Fail(r.status());
  return Emit(*r, 3, out, cap, n_out, [](const kvx::PoolLiveSegment& s, int64_t* o) {
    o[0] = s.logical_offset;
    o[1] = s.physical_offset;
    o[2] = s.size;
  });
}

int kvx_pool_physical_to_logical(const kvx_pool_spec* pool, int64_t physical_offset,
                                 int64_t size, int64_t* out_begin, int64_t* out_end) {
  if (out_begin == nullptr || out_end == nullptr) {
    return Fail(KVX_INVALID_ARGUMENT, "null output");
  }
  kvx::PoolSpec p;
  kvx::Status st = ToPool(pool, &p);
  if (!st.ok()) return Fail(st);
  auto segs = kvx::ExpandPoolLiveSegments(p);
  if (!segs.ok()) return Fail(segs.status());
  auto r = kvx::PhysicalLiveRangeToLogical(*segs, physical_offset, size);
  if (!r.ok()) return Fail(r.status());
  *out_begin = r->first;
  *out_end = r->second;
  return KVX_OK;
}

int kvx_pool_translate_live_copy(const kvx_pool_spec* src, const kvx_pool_spec* dst,
                                 int64_t src_offset, int64_t dst_offset, int64_t size,
                                 int64_t* out, int64_t cap, int64_t* n_out) {
  kvx::PoolSpec ps, pd;
  kvx::Status st = ToPool(src, &ps);
  if (st.ok()) st = ToPool(dst, &pd);
  if (!st.ok()) return Fail(st);
  auto ss = kvx::ExpandPoolLiveSegments(ps);
  if (!ss.ok()) return Fail(ss.status());
  auto ds = kvx::ExpandPoolLiveSegments(pd);
  if (!ds.ok()) return Fail(ds.status());
  auto r = kvx::TranslateLiveCopy(*ss, *ds, src_offset, dst_offset, size);
  if (!r.ok()) return Fail(r.status());
  return Emit(*r, 3, out, cap, n_out, [](const kvx::LiveCopyChunk& c, int64_t* o) {
    o[0] = c.src_physical;
    o[1] = c.dst_physical;
    o[2] = c.size;
  });
}

int32_t kvx_regions_cover_range(const kvx_region_spec* regions, int64_t n, int64_t start,
                                int64_t end) {
  if (BadArray(regions, n) || start < 0 || end < 0) return 0;
  kvx_pool_spec tmp{"", 0, 0, 0, 0, regions, n, ""};
  kvx::PoolSpec p;
  if (!ToPool(&tmp, &p).ok()) return 0;
  return kvx::RegionsCoverRange(p.regions, static_cast<size_t>(start),
                                static_cast<size_t>(end))
             ? 1
             : 0;
}

int kvx_manager_register_pools(kvx_manager* m, const kvx_pool_spec* pools, int64_t n) {
  if (m == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null manager");
  if (BadArray(pools, n)) return Fail(KVX_INVALID_ARGUMENT, "null pools");
  std::vector<kvx::PoolSpec> v(static_cast<size_t>(n));
  for (int64_t i = 0; i < n; ++i) {
    kvx::Status st = ToPool(&pools[i], &v[static_cast<size_t>(i)]);
    if (!st.ok()) return Fail(st);
  }
  return Done(m->impl->RegisterPools(std::move(v)));
}

int64_t kvx_manager_num_pools(kvx_manager* m) {
  return m == nullptr ? -1 : static_cast<int64_t>(m->impl->num_pools());
}

int32_t kvx_manager_has_explicit_pools(kvx_manager* m) {
  return m != nullptr && m->impl->has_explicit_pools() ? 1 : 0;
}

int kvx_manager_pool_indices_with_tag(kvx_manager* m, const char* tag, int64_t* out,
                                      int64_t cap, int64_t* n_out) {
  if (m == nullptr || tag == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null argument");
  std::vector<size_t> ids = m->impl->PoolIndicesWithTag(tag);
  return Emit(ids, 1, out, cap, n_out,
              [](size_t i, int64_t* o) { o[0] = static_cast<int64_t>(i); });
}

int kvx_manager_pool_spec(kvx_manager* m, int64_t pool_idx, kvx_pool_spec* out,
                          kvx_region_spec* regions, int64_t cap, int64_t* out_num_regions,
                          kvx_strings** out_names) {
  if (m == nullptr || out == nullptr || out_num_regions == nullptr || out_names == nullptr) {
    return Fail(KVX_INVALID_ARGUMENT, "null argument");
  }
  if (cap < 0 || (cap > 0 && regions == nullptr)) {
    return Fail(KVX_INVALID_ARGUMENT, "null regions with a positive capacity");
  }
  if (pool_idx < 0) return Fail(KVX_OUT_OF_RANGE, "pool index out of range");
  auto r = m->impl->pool_spec(static_cast<size_t>(pool_idx));
  if (!r.ok()) return Fail(r.status());
  const kvx::PoolSpec& p = *r;
  *out = kvx_pool_spec{nullptr,
                       static_cast<int64_t>(p.storage_index),
                       p.base_offset_bytes,
                       p.block_stride_bytes,
                       p.num_blocks,
                       nullptr,
                       static_cast<int64_t>(p.regions.size()),
                       nullptr};
  *out_num_regions = static_cast<int64_t>(p.regions.size());
  auto* names = new kvx_strings();
  names->items.push_back(p.tag);
  names->items.push_back(p.dtype_tag);
  for (size_t i = 0; i < p.regions.size(); ++i) {
    const kvx::RegionSpec& s = p.regions[i];
    names->items.push_back(s.name);
    if (static_cast<int64_t>(i) < cap) {
      regions[i] = kvx_region_spec{nullptr,      s.offset_bytes, s.stride_bytes,
                                   s.unit_bytes, s.num_units,    s.units_per_stride};
    }
  }
  *out_names = names;
  return KVX_OK;
}

int kvx_manager_pool_block_ref(kvx_manager* m, int64_t pool_idx, int64_t shard_idx,
                               int64_t block_id, uint64_t* out_ptr,
                               int64_t* out_block_stride_bytes) {
  if (m == nullptr || out_ptr == nullptr || out_block_stride_bytes == nullptr) {
    return Fail(KVX_INVALID_ARGUMENT, "null argument");
  }
  if (pool_idx < 0 || shard_idx < 0) {
    return Fail(KVX_OUT_OF_RANGE, "pool or shard index out of range");
  }
  auto r = m->impl->GetPoolBlockRef(static_cast<size_t>(pool_idx),
                                    static_cast<size_t>(shard_idx), block_id);
  if (!r.ok()) return Fail(r.status());
  *out_ptr = reinterpret_cast<uint64_t>(r->ptr);
  *out_block_stride_bytes = r->block_stride_bytes;
  return KVX_OK;
}

static int PoolCopy(bool d2h, kvx_manager* m, int64_t pool_idx, const int64_t* block_ids,
                    int64_t n, int64_t shard_idx, void* stream, kvx_future** out) {
  if (m == nullptr || out == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null manager or output");
  if (BadArray(block_ids, n)) return Fail(KVX_INVALID_ARGUMENT, "null block ids");
  if (pool_idx < 0) return Fail(KVX_OUT_OF_RANGE, "pool index out of range");
  std::optional<size_t> shard;
  if (shard_idx >= 0) shard = static_cast<size_t>(shard_idx);
  std::vector<int64_t> ids(block_ids, block_ids + n);
  auto r = d2h ? m->impl->D2hPoolBlocks(static_cast<size_t>(pool_idx), ids, shard,
                                        static_cast<hipStream_t>(stream))
               : m->impl->H2dPoolBlocks(static_cast<size_t>(pool_idx), ids, shard,
                                        static_cast<hipStream_t>(stream));
  if (!r.ok()) return Fail(r.status());
  *out = new kvx_future{std::move(*r)};
  return KVX_OK;
}

int kvx_manager_d2h_pool_blocks(kvx_manager* m, int64_t pool_idx, const int64_t* block_ids,
                                int64_t n, int64_t shard_idx, void* stream,
                                kvx_future** out) {
  return PoolCopy(true, m, pool_idx, block_ids, n, shard_idx, stream, out);
}

int kvx_manager_h2d_pool_blocks(kvx_manager* m, int64_t pool_idx, const int64_t* block_ids,
                                int64_t n, int64_t shard_idx, void* stream,
                                kvx_future** out) {
  return PoolCopy(false, m, pool_idx, block_ids, n, shard_idx, stream, out);
}

}  // extern "C"
