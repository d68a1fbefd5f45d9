"""GPU: a block push through the wire framing with the real kernels. The
sender gathers the source blocks on the device (the staging is the push
payload in the frame's order), the stream is assembled from that staging,
the receiver parses it into its own staging and scatters it into its pool.
Every destination block must equal the sender's source block, byte for
byte, against the oracle's stream and numpy indexing; other blocks stay
untouched. Covers both major orders, one block array, and fp8 payload plus
scale tables (mixed block sizes, layer-major)."""
import numpy as np
import pytest

from oracle import wire as O

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


def u8(t):
    torch.cuda.synchronize()
    return t.detach().cpu().contiguous().view(torch.uint8).numpy().reshape(t.shape[0], -1).copy()


def pools(cuda, rng, sizes, blocks):
    host = [rng.integers(0, 256, (blocks, b), dtype=np.uint8) for b in sizes]
    return host, [torch.from_numpy(h).to(cuda) for h in host]


def push(kvx, cuda, src_mgr, dst_mgr, src, dst, order, layer_idx=-1):
    T = kvx.transport
    fr = T.push_frame(src_mgr, src, dst, uuid=77, node_id=3, layer_idx=layer_idx,
                      major_order=order)
    staging = torch.empty(fr["staging_bytes"], dtype=torch.uint8, device=cuda)
    src_mgr.gather(src, staging, block_major=bool(order),
                   layer_idx=None if layer_idx < 0 else layer_idx).Await()
    stream = T.assemble_stream(fr, staging.cpu().numpy().tobytes())
    recv = np.zeros(fr["staging_bytes"], np.uint8)
    r = T.parse_push_stream(dst_mgr, stream, recv.ctypes.data, recv.size)
    assert r["dst_block_ids"] == list(dst) and r["src_block_ids"] == list(src)
    dev = torch.from_numpy(recv).to(cuda)
    dst_mgr.scatter(r["dst_block_ids"], dev, block_major=bool(r["major_order"]),
                    layer_idx=None if r["layer_idx"] < 0 else r["layer_idx"]).Await()
    return stream


@pytest.mark.parametrize("order", [0, 1])
def test_push_through_gather_stream_scatter(kvx, cuda, order):
    rng = np.random.default_rng(31 + order)
    L, P, B = 6, 128, 8192
    send_np, send = pools(cuda, rng, [B] * L, P)
    _, recv = pools(cuda, rng, [B] * L, P)
    recv_before = [u8(t) for t in recv]
    a = kvx.KVCacheManager(send, host_blocks_to_allocate=8)
    b = kvx.KVCacheManager(recv, host_blocks_to_allocate=8)
    src = [int(x) for x in rng.choice(P, 37, replace=False)]
    dst = [int(x) for x in rng.choice(P, 37, replace=False)]
    stream = push(kvx, cuda, a, b, src, dst, order)
    want = O.push_stream(lambda l, s, i: send_np[l][i].tobytes(), order, list(range(L)), 1,
                         src, dst, uuid=77, node_id=3)
    assert stream == want
    for l in range(L):
        exp = recv_before[l].copy()
        exp[dst] = send_np[l][src]
        assert np.array_equal(u8(recv[l]), exp), l
    a.close()
    b.close()


def test_push_of_one_block_array(kvx, cuda):
    rng = np.random.default_rng(33)
    send_np, send = pools(cuda, rng, [4096] * 4, 64)
    _, recv = pools(cuda, rng, [4096] * 4, 64)
    before = [u8(t) for t in recv]
    a = kvx.KVCacheManager(send, host_blocks_to_allocate=4)
    b = kvx.KVCacheManager(recv, host_blocks_to_allocate=4)
    src, dst = [5, 6, 7, 60], [0, 1, 2, 3]
    push(kvx, cuda, a, b, src, dst, 0, layer_idx=2)
    for l in range(4):
        exp = before[l].copy()
        if l == 2:
            exp[dst] = send_np[2][src]
        assert np.array_equal(u8(recv[l]), exp), l


def test_push_fp8_payload_with_scale_tables(kvx, cuda):
    """Payload (16 KiB fp8 blocks) and scales (8 heads x 4 B) in one push:
    mixed block sizes, layer-major, the staging groups payload then scales."""
    rng = np.random.default_rng(34)
    layers, P, H = 4, 96, 8
    kv_np, kv = pools(cuda, rng, [16384] * (2 * layers), P)
    sc_np, sc = pools(cuda, rng, [4 * H] * layers, P)
    _, kv2 = pools(cuda, rng, [16384] * (2 * layers), P)
    _, sc2 = pools(cuda, rng, [4 * H] * layers, P)
    before = [u8(t) for t in kv2 + sc2]
    a = kvx.KVCacheManager(kv, host_blocks_to_allocate=4, scale_tables=sc)
    b = kvx.KVCacheManager(kv2, host_blocks_to_allocate=4, scale_tables=sc2)
    src = [int(x) for x in rng.choice(P, 20, replace=False)]
    dst = [int(x) for x in rng.choice(P, 20, replace=False)]
    push(kvx, cuda, a, b, src, dst, 0)
    allsrc = kv_np + sc_np
    for w, t in enumerate(kv2 + sc2):
        exp = before[w].copy()
        exp[dst] = allsrc[w][src]
        assert np.array_equal(u8(t), exp), w
    with pytest.raises(kvx.KvxError, match="block-major staging needs one block size"):
        kvx.transport.push_frame(a, src, dst, major_order=1)
