"""ORACLE -- test infrastructure only.

Python restatement of the transport framing of a block push:

  header            the 64-byte little-endian flatbuffer struct of
                    tpu_sync/transport/lib/chunk.fbs (magic u16 0x4452, ver
                    u16, op u8, flags u8, buffer_id u16, reserved u16,
                    metadata_size u16, remote_id u32, local_id u32,
                    count_or_size u32, uuid u64, 4 x u64 padding), written
                    by chunk_serializer.cc:35-112 with struct.pack;
  metadata          the 24-byte ChunkMetadata (chunk.fbs);
  block_ids         u32 little-endian per id (chunk_serializer.cc:132-152);
  payload_order     ForEachPayload (tpu_sync/transport/block_transport.cc:
                    166-190): layer-major = for layer, shard, block;
                    block-major = for block, layer, shard;
  push_stream       BuildBlockRequests + ProcessSocketPush
                    (block_transport.cc:974-1175) without the handshake
                    bytes: header (op 6 with destinations, else 1;
                    flags = order; reserved = parallelism; remote_id =
                    node id; local_id = layer or 0xFFFFFFFF), destination
                    and source ids (op 6), then per item a u32 size and the
                    block's bytes.

Parity status: header / metadata / block ids are pinned by the byte
vectors of the reference's chunk_serializer_test.cc
(tests/golden/wire_cases.json); payload_order and push_stream by their
definitions and by the round trip through the product's parser, with a
byte-level check that every item carries the block the order names
(tests/test_transport.py, tests/test_gpu_transport.py).
"""
import struct

_HEADER = struct.Struct("<HHBBHHHIIIQ32x")
_META = struct.Struct("<IIQQ")


def header(op, flags, buffer_id, reserved, metadata_size, remote_id, local_id, count_or_size,
           uuid, version=1):
    return _HEADER.pack(0x4452, version, op, flags, buffer_id, reserved, metadata_size,
                        remote_id, local_id, count_or_size, uuid)


def parse_header(b):
    magic, ver, op, flags, bid, res, ms, rid, lid, cnt, uuid = _HEADER.unpack(b)
    return {"magic": magic, "version": ver, "op": op, "flags": flags, "buffer_id": bid,
            "reserved": res, "metadata_size": ms, "remote_id": rid, "local_id": lid,
            "count_or_size": cnt, "uuid": uuid}


def metadata(layer_idx, dst_shard_idx, dst_offset_bytes, size_bytes):
    return _META.pack(layer_idx, dst_shard_idx, dst_offset_bytes, size_bytes)


def block_ids(ids):
    return b"".join(struct.pack("<I", i & 0xFFFFFFFF) for i in ids)


def payload_order(order, layers, shards, blocks):
    if order == 0:
        return [(l, s, k) for l in layers for s in range(shards) for k in range(blocks)]
    return [(l, s, k) for k in range(blocks) for l in layers for s in range(shards)]


def push_stream(block_of, order, layers, shards, src, dst=None, uuid=0, node_id=0,
                layer_idx=-1, parallelism=1):
    """block_of(layer, shard, src_id) -> bytes of that block on the sender."""
    op = 6 if dst is not None else 1
    local = 0xFFFFFFFF if layer_idx < 0 else layer_idx
    out = [header(op, order, 0, parallelism, 0, node_id, local, len(src), uuid)]
    if dst is not None:
        out += [block_ids(dst), block_ids(src)]
    for l, s, k in payload_order(order, layers, shards, len(src)):
        b = block_of(l, s, src[k])
        out += [struct.pack("<I", len(b)), b]
    return b"".join(out)
