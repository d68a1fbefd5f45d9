// extern "C" surface of the transport framing (declared in include/kvx.h).
#include <cstdint>
#include <cstring>
#include <vector>

#include "../host/chunk_wire.h"
#include "capi_internal.h"

using kvx_capi::BadArray;
using kvx_capi::Fail;

namespace {

kvx::ChunkHeader FromC(const kvx_chunk_header& c) {
  kvx::ChunkHeader h;
  h.version = c.version;
  h.op = c.op;
  h.flags = c.flags;
  h.buffer_id = c.buffer_id;
  h.reserved = c.reserved;
  h.metadata_size = c.metadata_size;
  h.remote_id = c.remote_id;
  h.local_id = c.local_id;
  h.count_or_size = c.count_or_size;
  h.uuid = c.uuid;
  return h;
}

kvx_chunk_header ToC(const kvx::ChunkHeader& h) {
  return kvx_chunk_header{h.version,   h.op,        h.flags,         h.buffer_id, h.reserved,
                          h.metadata_size, h.remote_id, h.local_id, h.count_or_size, h.uuid};
}

std::vector<int64_t> ArrayBlockBytes(kvx_manager* m) {
  std::vector<int64_t> bb;
  for (size_t l = 0; l < m->impl->num_layers(); ++l) bb.push_back(m->impl->LayerBlockByteSize(l));
  return bb;
}

}  // namespace

extern "C" {

void kvx_chunk_header_serialize(const kvx_chunk_header* h, uint8_t* out64) {
  if (h == nullptr || out64 == nullptr) return;
  const auto b = kvx::SerializeChunkHeader(FromC(*h));
  std::memcpy(out64, b.data(), b.size());
}

int kvx_chunk_header_deserialize(const uint8_t* bytes, int64_t n, kvx_chunk_header* out) {
  if (out == nullptr || n < 0) return Fail(KVX_INVALID_ARGUMENT, "null output");
  auto r = kvx::DeserializeChunkHeader(bytes, static_cast<size_t>(n));
  if (!r.ok()) return Fail(r.status());
  *out = ToC(*r);
  return KVX_OK;
}

void kvx_chunk_metadata_serialize(const kvx_chunk_metadata* m, uint8_t* out24) {
  if (m == nullptr || out24 == nullptr) return;
  kvx::ChunkMetadata md;
  md.layer_idx = m->layer_idx;
  md.dst_shard_idx = m->dst_shard_idx;
  md.dst_offset_bytes = m->dst_offset_bytes;
  md.size_bytes = m->size_bytes;
  const auto b = kvx::SerializeChunkMetadata(md);
  std::memcpy(out24, b.data(), b.size());
}

int kvx_chunk_metadata_deserialize(const uint8_t* bytes, int64_t n, int32_t version,
                                   kvx_chunk_metadata* out) {
  if (out == nullptr || n < 0) return Fail(KVX_INVALID_ARGUMENT, "null output");
  auto r = kvx::DeserializeChunkMetadata(bytes, static_cast<size_t>(n),
                                         static_cast<uint16_t>(version));
  if (!r.ok()) return Fail(r.status());
  *out = kvx_chunk_metadata{r->layer_idx, r->dst_shard_idx, r->dst_offset_bytes, r->size_bytes};
  return KVX_OK;
}

void kvx_block_ids_serialize(const int64_t* ids, int64_t n, uint8_t* out) {
  if (BadArray(ids, n) || BadArray(out, n)) return;
  const auto b = kvx::SerializeBlockIds(std::vector<int64_t>(ids, ids + n));
  if (!b.empty()) std::memcpy(out, b.data(), b.size());
}

void kvx_block_ids_deserialize(const uint8_t* bytes, int64_t n_bytes, int64_t* out) {
  if (BadArray(bytes, n_bytes) || BadArray(out, n_bytes / 4)) return;
  const auto ids = kvx::DeserializeBlockIds(bytes, static_cast<size_t>(n_bytes));
  for (size_t i = 0; i < ids.size(); ++i) out[i] = ids[i];
}

int kvx_manager_build_push_frame(kvx_manager* m, uint64_t uuid, uint32_t node_id,
                                 int64_t layer_idx, int32_t parallelism, int32_t major_order,
                                 const int64_t* src_ids, const int64_t* dst_ids, int64_t n,
                                 uint8_t* out_header64, uint8_t* out_dst_ids,
                                 uint8_t* out_src_ids, kvx_push_item* out_items,
                                 int64_t items_cap, int64_t* out_n_items,
                                 int64_t* out_staging_bytes) {
  if (m == nullptr || out_header64 == nullptr || out_n_items == nullptr ||
      out_staging_bytes == nullptr || BadArray(src_ids, n) || BadArray(out_items, items_cap)) {
    return Fail(KVX_INVALID_ARGUMENT, "null argument");
  }
  if (dst_ids != nullptr && (BadArray(out_dst_ids, n) || BadArray(out_src_ids, n))) {
    return Fail(KVX_INVALID_ARGUMENT, "null id outputs for an explicit-destination push");
  }
  if (major_order != KVX_LAYER_MAJOR && major_order != KVX_BLOCK_MAJOR) {
    return Fail(KVX_INVALID_ARGUMENT, "unknown major order");
  }
  if (parallelism < 0 || parallelism > 0xFFFF) {
    return Fail(KVX_INVALID_ARGUMENT, "parallelism does not fit the header");
  }
  kvx::BlockPushSpec spec;
  spec.uuid = uuid;
  spec.node_id = node_id;
  spec.layer_idx = layer_idx;
  spec.parallelism = static_cast<uint16_t>(parallelism);
  spec.order = static_cast<kvx::MajorOrder>(major_order);
  spec.src_block_ids.assign(src_ids, src_ids + n);
  if (dst_ids != nullptr) spec.dst_block_ids.assign(dst_ids, dst_ids + n);
  spec.array_block_bytes = ArrayBlockBytes(m);
  spec.num_shards = static_cast<int64_t>(m->impl->num_shards());
  auto r = kvx::BuildBlockPushFrame(spec);
  if (!r.ok()) return Fail(r.status());
  std::memcpy(out_header64, r->header.data(), r->header.size());
  if (dst_ids != nullptr && n > 0) {
    std::memcpy(out_dst_ids, r->dst_ids.data(), r->dst_ids.size());
    std::memcpy(out_src_ids, r->src_ids.data(), r->src_ids.size());
  }
  *out_n_items = static_cast<int64_t>(r->items.size());
  for (int64_t i = 0; i < *out_n_items && i < items_cap; ++i) {
    const kvx::PushItem& it = r->items[static_cast<size_t>(i)];
    out_items[i] = kvx_push_item{it.layer, it.shard, it.k, it.staging_offset, it.size};
  }
  *out_staging_bytes = r->staging_bytes;
  return KVX_OK;
}

int kvx_manager_parse_push_stream(kvx_manager* m, const uint8_t* stream, int64_t n,
                                  uint8_t* staging, int64_t staging_cap,
                                  kvx_chunk_header* out_header, int64_t* out_layer_idx,
                                  int32_t* out_major_order, int64_t* out_dst_ids,
                                  int64_t* out_src_ids, int64_t ids_cap, int64_t* out_count,
                                  int64_t* out_staging_bytes) {
  if (m == nullptr || out_header == nullptr || out_layer_idx == nullptr ||
      out_major_order == nullptr || out_count == nullptr || out_staging_bytes == nullptr ||
      BadArray(stream, n) || BadArray(out_dst_ids, ids_cap) || BadArray(out_src_ids, ids_cap) ||
      staging_cap < 0) {
    return Fail(KVX_INVALID_ARGUMENT, "null argument");
  }
  auto r = kvx::ParseBlockPushStream(stream, static_cast<size_t>(n), ArrayBlockBytes(m),
                                     static_cast<int64_t>(m->impl->num_shards()), staging,
                                     static_cast<size_t>(staging_cap));
  if (!r.ok()) return Fail(r.status());
  *out_header = ToC(r->header);
  *out_layer_idx = r->layer_idx;
  *out_major_order = static_cast<int32_t>(r->order);
  *out_count = static_cast<int64_t>(r->dst_block_ids.size());
  for (int64_t i = 0; i < *out_count && i < ids_cap; ++i) {
    out_dst_ids[i] = r->dst_block_ids[static_cast<size_t>(i)];
    out_src_ids[i] = r->src_block_ids[static_cast<size_t>(i)];
  }
  *out_staging_bytes = r->staging_bytes;
  return KVX_OK;
}

}  // extern "C"
