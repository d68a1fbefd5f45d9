"""Transport framing of block pushes: the reference's ChunkHeader /
ChunkMetadata / block-id / chunk-size wire forms
(tpu_sync/transport/lib/chunk.h:22-59, chunk_serializer.cc:35-182) and the
block-push byte stream (tpu_sync/transport/block_transport.cc:974-1175), built
and parsed by the library. Payload items are slices of the buffer
``KVCacheManager.gather`` writes (same major order), so a push needs no
re-packing; there is no network in this package."""
from __future__ import annotations

import ctypes
import dataclasses
from typing import List, Optional, Sequence

from . import _capi

LAYER_MAJOR, BLOCK_MAJOR = 0, 1
OP_BLOCK_PUSH_ALLOCATE, OP_BLOCK_PUSH_EXPLICIT = 1, 6
ALL_BLOCK_ARRAYS = 0xFFFFFFFF


@dataclasses.dataclass
class ChunkHeader:
    version: int = 1
    op: int = 0
    flags: int = 0
    buffer_id: int = 0
    reserved: int = 0
    metadata_size: int = 0
    remote_id: int = 0
    local_id: int = 0
    count_or_size: int = 0
    uuid: int = 0

    def serialize(self) -> bytes:
        c = _capi.ChunkHeaderC(*dataclasses.astuple(self))
        out = ctypes.create_string_buffer(64)
        _capi.load().kvx_chunk_header_serialize(ctypes.byref(c), out)
        return out.raw

    @classmethod
    def deserialize(cls, data: bytes) -> "ChunkHeader":
        c = _capi.ChunkHeaderC()
        _capi.check(_capi.load().kvx_chunk_header_deserialize(bytes(data), len(data),
                                                              ctypes.byref(c)),
                    "DeserializeChunkHeader")
        return cls(*[getattr(c, f.name) for f in dataclasses.fields(cls)])


@dataclasses.dataclass
class ChunkMetadata:
    layer_idx: int = 0
    dst_shard_idx: int = 0
    dst_offset_bytes: int = 0
    size_bytes: int = 0

    def serialize(self) -> bytes:
        c = _capi.ChunkMetadataC(*dataclasses.astuple(self))
        out = ctypes.create_string_buffer(24)
        _capi.load().kvx_chunk_metadata_serialize(ctypes.byref(c), out)
        return out.raw

    @classmethod
    def deserialize(cls, data: bytes, version: int = 1) -> "ChunkMetadata":
        c = _capi.ChunkMetadataC()
        _capi.check(_capi.load().kvx_chunk_metadata_deserialize(bytes(data), len(data), version,
                                                                ctypes.byref(c)),
                    "DeserializeChunkMetadata")
        return cls(*[getattr(c, f.name) for f in dataclasses.fields(cls)])


def serialize_block_ids(ids: Sequence[int]) -> bytes:
    arr, n = _capi.i64_array(ids)
    out = ctypes.create_string_buffer(max(4 * n, 1))
    _capi.load().kvx_block_ids_serialize(arr, n, out)
    return out.raw[:4 * n]


def deserialize_block_ids(data: bytes) -> List[int]:
    n = len(data) // 4
    out = (ctypes.c_int64 * max(n, 1))()
    _capi.load().kvx_block_ids_deserialize(bytes(data), len(data), out)
    return list(out[:n])


def serialize_chunk_size(size: int) -> bytes:
    return int(size).to_bytes(4, "little")


def push_frame(mgr, src_block_ids: Sequence[int], dst_block_ids: Optional[Sequence[int]] = None,
               *, uuid: int = 0, node_id: int = 0, layer_idx: int = -1, parallelism: int = 1,
               major_order: int = LAYER_MAJOR) -> dict:
    """The sender's bytes of one block push over ``mgr``'s arrays: header,
    id arrays (explicit destinations only) and the payload items
    (layer, shard, k, staging_offset, size) in stream order."""
    src, n = _capi.i64_array(src_block_ids)
    dst = None
    if dst_block_ids is not None:
        dst, nd = _capi.i64_array(dst_block_ids)
        if nd != n:
            raise _capi.KvxError(3, "src and dst block lists must have same length", "push")
    header = ctypes.create_string_buffer(64)
    ids_d = ctypes.create_string_buffer(max(4 * n, 1))
    ids_s = ctypes.create_string_buffer(max(4 * n, 1))
    lib = _capi.load()
    cap = 1024
    while True:
        items = (_capi.PushItemC * cap)()
        n_items, staging = ctypes.c_int64(), ctypes.c_int64()
        _capi.check(lib.kvx_manager_build_push_frame(
            mgr._h, uuid, node_id, layer_idx, parallelism, major_order, src, dst, n, header,
            ids_d if dst is not None else None, ids_s if dst is not None else None, items, cap,
            ctypes.byref(n_items), ctypes.byref(staging)), "BuildBlockPushFrame")
        if n_items.value <= cap:
            break
        cap = n_items.value
    return {"header": header.raw,
            "dst_ids": ids_d.raw[:4 * n] if dst is not None else b"",
            "src_ids": ids_s.raw[:4 * n] if dst is not None else b"",
            "items": [(it.layer, it.shard, it.k, it.staging_offset, it.size)
                      for it in items[:n_items.value]],
            "staging_bytes": staging.value}


def assemble_stream(frame: dict, staging: bytes) -> bytes:
    """Concatenates what a sender writes for `frame` (no handshake bytes):
    header, ids, then a chunk-size field and the staged bytes per item."""
    parts = [frame["header"], frame["dst_ids"], frame["src_ids"]]
    mv = memoryview(staging)
    for _, _, _, off, size in frame["items"]:
        parts.append(serialize_chunk_size(size))
        parts.append(mv[off:off + size].tobytes())
    return b"".join(parts)


def parse_push_stream(mgr, stream: bytes, staging_ptr: int, staging_capacity: int) -> dict:
    """Receiver side of a whole explicit-destination push stream: the payload
    lands at ``staging_ptr`` (host memory) in the gather's layout."""
    data = bytes(stream)
    h = _capi.ChunkHeaderC()
    layer, order = ctypes.c_int64(), ctypes.c_int32()
    cap = max(len(data) // 8, 1)
    dst, src = (ctypes.c_int64 * cap)(), (ctypes.c_int64 * cap)()
    count, nbytes = ctypes.c_int64(), ctypes.c_int64()
    _capi.check(_capi.load().kvx_manager_parse_push_stream(
        mgr._h, data, len(data), ctypes.c_void_p(staging_ptr), staging_capacity, ctypes.byref(h),
        ctypes.byref(layer), ctypes.byref(order), dst, src, cap, ctypes.byref(count),
        ctypes.byref(nbytes)), "ParseBlockPushStream")
    return {"header": ChunkHeader(*[getattr(h, f.name) for f in dataclasses.fields(ChunkHeader)]),
            "layer_idx": layer.value, "major_order": order.value,
            "dst_block_ids": list(dst[:count.value]), "src_block_ids": list(src[:count.value]),
            "staging_bytes": nbytes.value}
