#include "chunk_wire.h"

#include <cstring>
#include <limits>
#include <string>

#include "transfer_engine.h"

namespace kvx {
namespace {

template <typename T>
void Put(uint8_t* p, T v) {
  for (size_t i = 0; i < sizeof(T); ++i) p[i] = static_cast<uint8_t>(static_cast<uint64_t>(v) >> (8 * i));
}

template <typename T>
T Get(const uint8_t* p) {
  uint64_t v = 0;
  for (size_t i = 0; i < sizeof(T); ++i) v |= static_cast<uint64_t>(p[i]) << (8 * i);
  return static_cast<T>(v);
}

// Calls fn(layer, shard, k) in the payload sequence of `order`.
template <typename Fn>
Status ForEachItem(MajorOrder order, const std::vector<int64_t>& layers, int64_t shards,
                   int64_t blocks, Fn fn) {
  if (order == MajorOrder::kLayerMajor) {
    for (int64_t l : layers)
      for (int64_t s = 0; s < shards; ++s)
        for (int64_t k = 0; k < blocks; ++k) KVX_RETURN_IF_ERROR(fn(l, s, k));
  } else {
    for (int64_t k = 0; k < blocks; ++k)
      for (int64_t l : layers)
        for (int64_t s = 0; s < shards; ++s) KVX_RETURN_IF_ERROR(fn(l, s, k));
  }
  return OkStatus();
}

StatusOr<std::vector<int64_t>> TargetLayers(int64_t layer_idx, size_t arrays) {
  std::vector<int64_t> layers;
  if (layer_idx < 0) {
    for (size_t l = 0; l < arrays; ++l) layers.push_back(static_cast<int64_t>(l));
  } else if (static_cast<size_t>(layer_idx) >= arrays) {
    return OutOfRangeError("push block-array index " + std::to_string(layer_idx) +
                           " out of range: " + std::to_string(arrays));
  } else {
    layers.push_back(layer_idx);
  }
  return layers;
}

// Staging layout of the (layer, shard) storages in layer-major storage order.
StatusOr<StagingLayout> LayoutFor(const std::vector<int64_t>& layers,
                                  const std::vector<int64_t>& array_bytes, int64_t shards,
                                  int64_t n, MajorOrder order) {
  std::vector<int64_t> bb;
  for (int64_t l : layers)
    for (int64_t s = 0; s < shards; ++s) bb.push_back(array_bytes[static_cast<size_t>(l)]);
  return DeviceStagingLayout(bb, n, order == MajorOrder::kBlockMajor);
}

}  // namespace

std::array<uint8_t, kChunkHeaderBytes> SerializeChunkHeader(const ChunkHeader& h) {
  std::array<uint8_t, kChunkHeaderBytes> b{};
  Put<uint16_t>(&b[0], kChunkMagic);
  Put<uint16_t>(&b[2], 1);  // the only version this serializer writes
  b[4] = h.op;
  b[5] = h.flags;
  Put<uint16_t>(&b[6], h.buffer_id);
  Put<uint16_t>(&b[8], h.reserved);
  Put<uint16_t>(&b[10], h.metadata_size);
  Put<uint32_t>(&b[12], h.remote_id);
  Put<uint32_t>(&b[16], h.local_id);
  Put<uint32_t>(&b[20], h.count_or_size);
  Put<uint64_t>(&b[24], h.uuid);
  return b;
}

StatusOr<ChunkHeader> DeserializeChunkHeader(const uint8_t* p, size_t n) {
  if (p == nullptr || n != kChunkHeaderBytes) {
    return InvalidArgumentError("Invalid chunk header size");
  }
  const uint16_t magic = Get<uint16_t>(p);
  if (magic != kChunkMagic) {
    return InvalidArgumentError("Chunk header magic mismatch: expected " +
                                std::to_string(kChunkMagic) + ", got " + std::to_string(magic));
  }
  const uint16_t ver = Get<uint16_t>(p + 2);
  if (ver != 1) {
    return FailedPreconditionError("Unsupported chunk header flatbuf version: " +
                                   std::to_string(ver));
  }
  ChunkHeader h;
  h.version = ver;
  h.op = p[4];
  h.flags = p[5];
  h.buffer_id = Get<uint16_t>(p + 6);
  h.reserved = Get<uint16_t>(p + 8);
  h.metadata_size = Get<uint16_t>(p + 10);
  h.remote_id = Get<uint32_t>(p + 12);
  h.local_id = Get<uint32_t>(p + 16);
  h.count_or_size = Get<uint32_t>(p + 20);
  h.uuid = Get<uint64_t>(p + 24);
  return h;
}

std::array<uint8_t, kChunkMetadataBytes> SerializeChunkMetadata(const ChunkMetadata& m) {
  std::array<uint8_t, kChunkMetadataBytes> b{};
  Put<uint32_t>(&b[0], m.layer_idx);
  Put<uint32_t>(&b[4], m.dst_shard_idx);
  Put<uint64_t>(&b[8], m.dst_offset_bytes);
  Put<uint64_t>(&b[16], m.size_bytes);
  return b;
}

StatusOr<ChunkMetadata> DeserializeChunkMetadata(const uint8_t* p, size_t n, uint16_t ver) {
  const size_t want = ver == 1 ? kChunkMetadataBytes : 0;
  if (p == nullptr || n != want) return InvalidArgumentError("Invalid chunk metadata size");
  ChunkMetadata m;
  m.layer_idx = Get<uint32_t>(p);
  m.dst_shard_idx = Get<uint32_t>(p + 4);
  m.dst_offset_bytes = Get<uint64_t>(p + 8);
  m.size_bytes = Get<uint64_t>(p + 16);
  return m;
}

std::vector<uint8_t> SerializeBlockIds(const std::vector<int64_t>& ids) {
  std::vector<uint8_t> b(ids.size() * 4);
  for (size_t i = 0; i < ids.size(); ++i) Put<uint32_t>(&b[4 * i], static_cast<uint32_t>(ids[i]));
  return b;
}

std::vector<int64_t> DeserializeBlockIds(const uint8_t* p, size_t n) {
  std::vector<int64_t> ids(n / 4);
  for (size_t i = 0; i < ids.size(); ++i) {
    ids[i] = static_cast<int32_t>(Get<uint32_t>(p + 4 * i));  // ids are ints on the wire
  }
  return ids;
}

std::array<uint8_t, kChunkSizeFieldBytes> SerializeChunkSize(uint32_t size) {
  std::array<uint8_t, kChunkSizeFieldBytes> b{};
  Put<uint32_t>(&b[0], size);
  return b;
}

uint32_t DeserializeChunkSize(const uint8_t* p) { return Get<uint32_t>(p); }

StatusOr<MajorOrder> ParseMajorOrder(uint8_t flags) {
  const uint8_t v = flags & static_cast<uint8_t>(~kUseBlockChunksFlag);
  if (v == 0) return MajorOrder::kLayerMajor;
  if (v == 1) return MajorOrder::kBlockMajor;
  return InvalidArgumentError("Unknown block transport major order: " + std::to_string(flags));
}

StatusOr<BlockPushFrame> BuildBlockPushFrame(const BlockPushSpec& spec) {
  const int64_t n = static_cast<int64_t>(spec.src_block_ids.size());
  if (!spec.dst_block_ids.empty() && spec.dst_block_ids.size() != spec.src_block_ids.size()) {
    return InvalidArgumentError("src and dst block lists must have same length");
  }
  if (n > static_cast<int64_t>(std::numeric_limits<uint32_t>::max())) {
    return OutOfRangeError("Block count exceeds uint32");
  }
  if (spec.num_shards <= 0) return InvalidArgumentError("num_shards must be positive");
  for (const std::vector<int64_t>* ids : {&spec.src_block_ids, &spec.dst_block_ids}) {
    for (int64_t id : *ids) {
      if (id < 0 || id > std::numeric_limits<int32_t>::max()) {
        return OutOfRangeError("block id " + std::to_string(id) + " does not fit the wire format");
      }
    }
  }
  KVX_ASSIGN_OR_RETURN(std::vector<int64_t> layers,
                       TargetLayers(spec.layer_idx, spec.array_block_bytes.size()));
  for (int64_t l : layers) {
    const int64_t bb = spec.array_block_bytes[static_cast<size_t>(l)];
    if (bb <= 0 || bb > static_cast<int64_t>(std::numeric_limits<uint32_t>::max())) {
      return InvalidArgumentError("block bytes of block array " + std::to_string(l) +
                                  " do not fit a chunk size field");
    }
  }
  KVX_ASSIGN_OR_RETURN(StagingLayout lay, LayoutFor(layers, spec.array_block_bytes,
                                                    spec.num_shards, n, spec.order));
  BlockPushFrame f;
  ChunkHeader h;
  h.op = spec.dst_block_ids.empty() ? kOpBlockPushAllocate : kOpBlockPushExplicit;
  h.flags = static_cast<uint8_t>(spec.order);
  h.reserved = spec.parallelism;
  h.remote_id = spec.node_id;
  h.local_id = spec.layer_idx < 0 ? kAllBlockArrays : static_cast<uint32_t>(spec.layer_idx);
  h.count_or_size = static_cast<uint32_t>(n);
  h.uuid = spec.uuid;
  f.header = SerializeChunkHeader(h);
  if (!spec.dst_block_ids.empty()) {
    f.dst_ids = SerializeBlockIds(spec.dst_block_ids);
    f.src_ids = SerializeBlockIds(spec.src_block_ids);
  }
  f.staging_bytes = lay.total_bytes;
  // Storage index of (layer position, shard) in the layout.
  std::vector<int64_t> layer_pos(spec.array_block_bytes.size(), 0);
  for (size_t i = 0; i < layers.size(); ++i) layer_pos[static_cast<size_t>(layers[i])] = static_cast<int64_t>(i);
  KVX_RETURN_IF_ERROR(ForEachItem(spec.order, layers, spec.num_shards, n,
                                  [&](int64_t l, int64_t s, int64_t k) -> Status {
                                    const size_t w = static_cast<size_t>(
                                        layer_pos[static_cast<size_t>(l)] * spec.num_shards + s);
                                    f.items.push_back(PushItem{
                                        l, s, k, lay.base[w] + k * lay.stride_k[w],
                                        spec.array_block_bytes[static_cast<size_t>(l)]});
                                    return OkStatus();
                                  }));
  return f;
}

StatusOr<ParsedBlockPush> ParseBlockPushStream(const uint8_t* stream, size_t n,
                                               const std::vector<int64_t>& array_bytes,
                                               int64_t num_shards, uint8_t* staging,
                                               size_t staging_capacity) {
  if (stream == nullptr || n < kChunkHeaderBytes) {
    return InvalidArgumentError("stream shorter than a chunk header");
  }
  if (num_shards <= 0) return InvalidArgumentError("num_shards must be positive");
  ParsedBlockPush out;
  KVX_ASSIGN_OR_RETURN(out.header, DeserializeChunkHeader(stream, kChunkHeaderBytes));
  if (out.header.op == kOpBlockPushAllocate) {
    return UnimplementedError("allocate-on-receive pushes need the receiver's id reply");
  }
  if (out.header.op != kOpBlockPushExplicit) {
    return InvalidArgumentError("not a block push: op " + std::to_string(out.header.op));
  }
  KVX_ASSIGN_OR_RETURN(out.order, ParseMajorOrder(out.header.flags));
  out.layer_idx = out.header.local_id == kAllBlockArrays
                      ? -1
                      : static_cast<int64_t>(out.header.local_id);
  KVX_ASSIGN_OR_RETURN(std::vector<int64_t> layers, TargetLayers(out.layer_idx, array_bytes.size()));
  const int64_t count = out.header.count_or_size;
  size_t pos = kChunkHeaderBytes;
  const size_t ids_bytes = static_cast<size_t>(count) * 4;
  if (n - pos < 2 * ids_bytes) return InvalidArgumentError("stream ends inside the block ids");
  out.dst_block_ids = DeserializeBlockIds(stream + pos, ids_bytes);
  pos += ids_bytes;
  out.src_block_ids = DeserializeBlockIds(stream + pos, ids_bytes);
  pos += ids_bytes;
  KVX_ASSIGN_OR_RETURN(StagingLayout lay, LayoutFor(layers, array_bytes, num_shards, count,
                                                    out.order));
  out.staging_bytes = lay.total_bytes;
  if (staging == nullptr || staging_capacity < static_cast<size_t>(lay.total_bytes)) {
    return InvalidArgumentError("staging buffer of " + std::to_string(staging_capacity) +
                                " bytes is smaller than the push payload " +
                                std::to_string(lay.total_bytes));
  }
  std::vector<int64_t> layer_pos(array_bytes.size(), 0);
  for (size_t i = 0; i < layers.size(); ++i) layer_pos[static_cast<size_t>(layers[i])] = static_cast<int64_t>(i);
  KVX_RETURN_IF_ERROR(ForEachItem(
      out.order, layers, num_shards, count, [&](int64_t l, int64_t s, int64_t k) -> Status {
        if (n - pos < kChunkSizeFieldBytes) {
          return InvalidArgumentError("stream ends before the chunk size of block " +
                                      std::to_string(k));
        }
        const uint32_t size = DeserializeChunkSize(stream + pos);
        pos += kChunkSizeFieldBytes;
        const int64_t bb = array_bytes[static_cast<size_t>(l)];
        if (static_cast<int64_t>(size) != bb) {
          return InvalidArgumentError("chunk size " + std::to_string(size) +
                                      " does not match block bytes " + std::to_string(bb) +
                                      " of block array " + std::to_string(l));
        }
        if (n - pos < size) return InvalidArgumentError("stream ends inside a payload");
        const size_t w = static_cast<size_t>(layer_pos[static_cast<size_t>(l)] * num_shards + s);
        std::memcpy(staging + lay.base[w] + k * lay.stride_k[w], stream + pos, size);
        pos += size;
        return OkStatus();
      }));
  if (pos != n) {
    return InvalidArgumentError(std::to_string(n - pos) + " trailing bytes after the push");
  }
  return out;
}

}  // namespace kvx
