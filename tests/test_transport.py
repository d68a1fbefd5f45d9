"""Transport framing on the CPU: header / metadata / block-id / chunk-size
wire bytes against the reference's chunk_serializer_test.cc vectors (product
and oracle), push frames of host-only managers against the oracle's stream,
and the receiver's parser: round trips and every rejection."""
import json
import os

import numpy as np
import pytest

from oracle import wire as O

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "wire_cases.json")))


def test_wire_bytes_match_reference_vectors(kvx):
    T = kvx.transport
    f = GOLD["header_fields"]
    h = T.ChunkHeader(**f)
    b = h.serialize()
    assert len(b) == 64
    assert b[:32].hex() == GOLD["header_wire_prefix"] and b[32:] == bytes(32)
    assert b[:2] == b"RD"
    assert T.ChunkHeader.deserialize(b) == h
    ob = O.header(f["op"], f["flags"], f["buffer_id"], f["reserved"], f["metadata_size"],
                  f["remote_id"], f["local_id"], f["count_or_size"], f["uuid"])
    assert ob == b
    m = T.ChunkMetadata(**GOLD["metadata_fields"])
    assert m.serialize().hex() == GOLD["metadata_wire"]
    assert O.metadata(*GOLD["metadata_fields"].values()).hex() == GOLD["metadata_wire"]
    assert T.ChunkMetadata.deserialize(m.serialize()) == m
    assert T.serialize_block_ids(GOLD["block_ids"]).hex() == GOLD["block_ids_wire"]
    assert O.block_ids(GOLD["block_ids"]).hex() == GOLD["block_ids_wire"]
    ids = GOLD["block_ids_roundtrip"]
    assert T.deserialize_block_ids(T.serialize_block_ids(ids)) == ids
    assert T.serialize_chunk_size(GOLD["chunk_size"]).hex() == GOLD["chunk_size_wire"]


def test_header_rejections(kvx):
    T = kvx.transport
    b = bytearray(T.ChunkHeader(op=6).serialize())
    bad = bytearray(b)
    bad[0] ^= 0xFF
    with pytest.raises(kvx.KvxError) as e:
        T.ChunkHeader.deserialize(bytes(bad))
    assert e.value.code == 3
    bad = bytearray(b)
    bad[2:4] = b"\x02\x00"
    with pytest.raises(kvx.KvxError) as e:
        T.ChunkHeader.deserialize(bytes(bad))
    assert e.value.code == 9
    with pytest.raises(kvx.KvxError) as e:
        T.ChunkHeader.deserialize(bytes(b[:63]))
    assert e.value.code == 3
    with pytest.raises(kvx.KvxError):
        T.ChunkMetadata.deserialize(bytes(23))


def host_mgr(kvx, layers, shards, block):
    return kvx.KVCacheManager.create_host_only_for_testing(
        num_layers=layers, num_shards=shards, slice_byte_size=block, host_blocks=8)


@pytest.mark.parametrize("order", [0, 1])
@pytest.mark.parametrize("layer_idx", [-1, 2])
def test_push_frame_and_parse_round_trip(kvx, order, layer_idx):
    """A frame's items over a synthetic gathered staging buffer assemble into
    exactly the oracle's stream; parsing it restores the staging bytes."""
    T = kvx.transport
    L, S, B = 3, 2, 48
    mgr = host_mgr(kvx, L, S, B)
    rng = np.random.default_rng(order * 10 + layer_idx + 5)
    pool = rng.integers(0, 256, (L, S, 40, B), dtype=np.uint8)
    src = [7, 3, 3, 39, 0]
    dst = [1, 2, 5, 6, 0]
    fr = T.push_frame(mgr, src, dst, uuid=0xABCDEF, node_id=9, layer_idx=layer_idx,
                      parallelism=4, major_order=order)
    layers = list(range(L)) if layer_idx < 0 else [layer_idx]
    n = len(src)
    # The gather's staging for these storages and this order.
    if order == 0:
        staging = np.concatenate([pool[l, s][src].reshape(-1) for l in layers for s in range(S)])
    else:
        staging = np.concatenate([pool[l, s][src[k]] for k in range(n) for l in layers
                                  for s in range(S)])
    assert fr["staging_bytes"] == staging.size
    stream = T.assemble_stream(fr, staging.tobytes())
    want = O.push_stream(lambda l, s, i: pool[l, s, i].tobytes(), order, layers, S, src, dst,
                         uuid=0xABCDEF, node_id=9, layer_idx=layer_idx, parallelism=4)
    assert stream == want
    h = O.parse_header(fr["header"])
    assert (h["op"], h["flags"], h["reserved"], h["remote_id"], h["count_or_size"]) == \
        (6, order, 4, 9, n)
    assert h["local_id"] == (0xFFFFFFFF if layer_idx < 0 else layer_idx)
    assert [it[:3] for it in fr["items"]] == O.payload_order(order, layers, S, n)
    out = np.zeros(staging.size, np.uint8)
    r = T.parse_push_stream(host_mgr(kvx, L, S, B), stream, out.ctypes.data, out.size)
    assert np.array_equal(out, staging)
    assert r["dst_block_ids"] == dst and r["src_block_ids"] == src
    assert r["layer_idx"] == layer_idx and r["major_order"] == order
    assert r["header"].uuid == 0xABCDEF


def test_parse_rejections(kvx):
    T = kvx.transport
    mgr = host_mgr(kvx, 2, 1, 16)
    fr = T.push_frame(mgr, [1, 2], [3, 4])
    staging = bytes(range(fr["staging_bytes"]))
    stream = T.assemble_stream(fr, staging)
    out = np.zeros(fr["staging_bytes"], np.uint8)

    def parse(s, cap=out.size, m=mgr):
        return T.parse_push_stream(m, s, out.ctypes.data, cap)

    parse(stream)
    with pytest.raises(kvx.KvxError, match="trailing bytes"):
        parse(stream + b"x")
    with pytest.raises(kvx.KvxError, match="stream ends"):
        parse(stream[:-1])
    with pytest.raises(kvx.KvxError, match="smaller than the push payload"):
        parse(stream, cap=out.size - 1)
    big = np.zeros(4 * out.size, np.uint8)
    with pytest.raises(kvx.KvxError, match="does not match block bytes"):
        T.parse_push_stream(host_mgr(kvx, 2, 1, 32), stream, big.ctypes.data, big.size)
    bad = bytearray(stream)
    bad[5] = 3  # unknown major order
    with pytest.raises(kvx.KvxError, match="major order"):
        parse(bytes(bad))
    bad = bytearray(stream)
    bad[16:20] = (7).to_bytes(4, "little")  # block array 7 of 2
    with pytest.raises(kvx.KvxError) as e:
        parse(bytes(bad))
    assert e.value.code == 11
    alloc = T.push_frame(mgr, [1, 2])  # op 1: the receiver would allocate
    assert O.parse_header(alloc["header"])["op"] == 1 and alloc["dst_ids"] == b""
    with pytest.raises(kvx.KvxError) as e:
        parse(T.assemble_stream(alloc, staging))
    assert e.value.code == 12
    with pytest.raises(kvx.KvxError) as e:
        T.push_frame(mgr, [1, -2], [3, 4])
    assert e.value.code == 11
    with pytest.raises(kvx.KvxError) as e:
        T.push_frame(mgr, [1], [3], layer_idx=5)
    assert e.value.code == 11
