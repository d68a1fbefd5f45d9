// Wire framing of block pushes, so a device-staged (gathered) buffer feeds a
// network push without re-packing.
//
// Byte formats follow the reference exactly (other peers parse them):
//   ChunkHeader  64-byte little-endian record {magic 0x4452 "RD", ver 1, op,
//                flags, buffer_id, reserved, metadata_size, remote_id,
//                local_id, count_or_size, uuid, 32 zero bytes}
//                (tpu_sync/transport/lib/chunk.fbs, chunk_serializer.cc:35-112);
//   ChunkMetadata 24 bytes {layer_idx u32, dst_shard_idx u32,
//                dst_offset_bytes u64, size_bytes u64};
//   block ids    u32 little-endian each; chunk size  u32 little-endian.
// A block push (tpu_sync/transport/block_transport.cc:974-1175) is: the
// header (op 6 with explicit destinations, 1 to let the receiver allocate),
// for op 6 the destination then the source ids, then one item per
// (layer, shard, block) in the major order's sequence
// (block_transport.cc:166-190): a chunk-size field and the block's bytes.
// The gather kernel writes exactly that payload sequence, so each item's
// bytes are one slice of the staging buffer.
#ifndef KVX_HOST_CHUNK_WIRE_H_
#define KVX_HOST_CHUNK_WIRE_H_

#include <array>
#include <cstddef>
#include <cstdint>
#include <vector>

#include "status.h"

namespace kvx {

constexpr uint16_t kChunkMagic = 0x4452;
constexpr size_t kChunkHeaderBytes = 64;
constexpr size_t kChunkMetadataBytes = 24;
constexpr size_t kChunkSizeFieldBytes = 4;
constexpr uint8_t kOpBlockPushAllocate = 1;
constexpr uint8_t kOpBlockPushExplicit = 6;
constexpr uint8_t kUseBlockChunksFlag = 0x80;
constexpr uint32_t kAllBlockArrays = 0xFFFFFFFFu;

enum class MajorOrder : uint8_t { kLayerMajor = 0, kBlockMajor = 1 };

struct ChunkHeader {
  uint16_t version = 1;
  uint8_t op = 0;
  uint8_t flags = 0;
  uint16_t buffer_id = 0;
  uint16_t reserved = 0;
  uint16_t metadata_size = 0;
  uint32_t remote_id = 0;
  uint32_t local_id = 0;
  uint32_t count_or_size = 0;
  uint64_t uuid = 0;
};

struct ChunkMetadata {
  uint32_t layer_idx = 0;
  uint32_t dst_shard_idx = 0;
  uint64_t dst_offset_bytes = 0;
  uint64_t size_bytes = 0;
};

std::array<uint8_t, kChunkHeaderBytes> SerializeChunkHeader(const ChunkHeader& h);
// InvalidArgument for a wrong size or magic, FailedPrecondition for an
// unsupported version.
StatusOr<ChunkHeader> DeserializeChunkHeader(const uint8_t* bytes, size_t n);
std::array<uint8_t, kChunkMetadataBytes> SerializeChunkMetadata(const ChunkMetadata& m);
StatusOr<ChunkMetadata> DeserializeChunkMetadata(const uint8_t* bytes, size_t n, uint16_t ver);
std::vector<uint8_t> SerializeBlockIds(const std::vector<int64_t>& ids);
std::vector<int64_t> DeserializeBlockIds(const uint8_t* bytes, size_t n);
std::array<uint8_t, kChunkSizeFieldBytes> SerializeChunkSize(uint32_t size);
uint32_t DeserializeChunkSize(const uint8_t* bytes);
// The order bits of a header's flags (the block-chunks flag masked off).
StatusOr<MajorOrder> ParseMajorOrder(uint8_t flags);

struct BlockPushSpec {
  uint64_t uuid = 0;
  uint32_t node_id = 0;
  int64_t layer_idx = -1;  // one block array, or -1 for all
  uint16_t parallelism = 1;
  MajorOrder order = MajorOrder::kLayerMajor;
  std::vector<int64_t> src_block_ids;
  std::vector<int64_t> dst_block_ids;  // empty: the receiver allocates (op 1)
  std::vector<int64_t> array_block_bytes;  // per block array
  int64_t num_shards = 1;
};

// One payload item: block k of (layer, shard), `size` bytes at
// `staging_offset` of the gathered staging buffer.
struct PushItem {
  int64_t layer = 0;
  int64_t shard = 0;
  int64_t k = 0;
  int64_t staging_offset = 0;
  int64_t size = 0;
};

struct BlockPushFrame {
  std::array<uint8_t, kChunkHeaderBytes> header{};
  std::vector<uint8_t> dst_ids;  // op 6 only
  std::vector<uint8_t> src_ids;  // op 6 only
  std::vector<PushItem> items;   // payload sequence
  int64_t staging_bytes = 0;     // size of the gathered staging buffer
};

StatusOr<BlockPushFrame> BuildBlockPushFrame(const BlockPushSpec& spec);

// Receiver side of an op-6 push whose whole byte stream (header, ids, items)
// is in `stream`: checks the header and every item's size against the block
// arrays, and copies the payload into `staging` (laid out as the gather
// would, for the arrays the header names) ready for the scatter.
struct ParsedBlockPush {
  ChunkHeader header;
  MajorOrder order = MajorOrder::kLayerMajor;
  int64_t layer_idx = -1;
  std::vector<int64_t> dst_block_ids;
  std::vector<int64_t> src_block_ids;
  int64_t staging_bytes = 0;
};
StatusOr<ParsedBlockPush> ParseBlockPushStream(const uint8_t* stream, size_t n,
                                               const std::vector<int64_t>& array_block_bytes,
                                               int64_t num_shards, uint8_t* staging,
                                               size_t staging_capacity);

}  // namespace kvx

#endif  // KVX_HOST_CHUNK_WIRE_H_
