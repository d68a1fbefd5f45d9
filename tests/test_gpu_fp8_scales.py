"""GPU: fp8 KV cache with a per-(layer, block, head) fp32 scale side table.

The payload is e4m3 bytes and the scales are fp32 words, both with NaN and
denormal bit patterns injected at a 0.1 % rate; payload and scales of the
same block ids move together (one kernel launch per staging chunk or device
gather) and must round-trip byte-exact. The reference has no scale table
(fp8 moves as opaque bytes there), so the oracle is the closed form: block
identity per storage under the id map (oracle.transfer / oracle.extract).
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

E4M3_SPECIAL = np.array([0x7F, 0xFF, 0x01, 0x02, 0x07, 0x81, 0x85, 0x87], np.uint8)
F32_SPECIAL = np.array([0x7FC00000, 0xFFC00001, 0x7F800001, 0x00000001, 0x807FFFFF,
                        0x00400000, 0x80000000], np.uint32)


def fp8_payload(rng, blocks, bb):
    raw = rng.integers(0, 256, (blocks, bb), dtype=np.uint8)
    mask = rng.random(raw.shape) < 1e-3
    raw[mask] = rng.choice(E4M3_SPECIAL, size=int(mask.sum()))
    return raw


def fp32_scales(rng, blocks, heads):
    s = rng.standard_normal((blocks, heads), dtype=np.float32).view(np.uint32)
    mask = rng.random(s.shape) < 1e-3
    mask[0, 0] = True  # at least one special word per table
    s[mask] = rng.choice(F32_SPECIAL, size=int(mask.sum()))
    return s.view(np.float32)


def build(rng, cuda, layers, blocks, heads=8, head_dim=128, tokens=16):
    bb = tokens * heads * head_dim  # fp8: one byte per element
    kv_np = [fp8_payload(rng, blocks, bb) for _ in range(2 * layers)]
    sc_np = [fp32_scales(rng, blocks, heads) for _ in range(layers)]
    kv = [torch.from_numpy(a).to(cuda) for a in kv_np]
    sc = [torch.from_numpy(a).to(cuda) for a in sc_np]
    return kv_np, sc_np, kv, sc, bb


def u8(a):
    return np.ascontiguousarray(a).view(np.uint8).reshape(-1)


@pytest.mark.parametrize("mode", ["staged", "zero_copy", "bounce"])
def test_fp8_payload_and_scales_round_trip_match_oracle(kvx, oracle, cuda, mode):
    """bounce: a pageable (malloc) mirror; payload and scales of a chunk still
    move in one launch, through the bounce lane."""
    rng = np.random.default_rng(40)
    layers, blocks, host_blocks = 4, 96, 64
    kv_np, sc_np, kv, sc, bb = build(rng, cuda, layers, blocks)
    kw = dict(host_alloc="malloc") if mode == "bounce" else dict(transfer_mode=mode)
    mgr = kvx.KVCacheManager(kv, host_blocks_to_allocate=host_blocks, scale_tables=sc, **kw)
    assert mgr.num_kv_layers == 2 * layers and mgr.num_layers == 3 * layers
    assert mgr.block_bytes(0) == bb and mgr.block_bytes(2 * layers) == 32
    dev = [u8(a).copy() for a in kv_np + sc_np]
    host = [np.zeros(host_blocks * (bb if k < 2 * layers else 32), np.uint8)
            for k in range(3 * layers)]
    bbs = [bb] * (2 * layers) + [32] * layers
    ids = rng.choice(blocks, 40, replace=False).tolist()
    slot = rng.choice(host_blocks, 40, replace=False).tolist()
    before = mgr.engine_stats()["kernel_launches"]
    mgr.d2h(ids, slot).Await()
    # Payload and scales of one chunk move in one launch.
    assert mgr.engine_stats()["kernel_launches"] - before == 1
    assert oracle.transfer(True, dev, host, bbs, [d.nbytes for d in dev], ids, slot,
                           [1] * 40) == 0
    for k in range(3 * layers):
        assert np.array_equal(mgr.host_view(k), host[k]), k
    back = rng.choice(blocks, 40, replace=False).tolist()
    mgr.h2d(slot, back).Await()
    assert oracle.transfer(False, dev, host, bbs, [d.nbytes for d in dev], slot, back,
                           [1] * 40) == 0
    torch.cuda.synchronize()
    for k, t in enumerate(kv + sc):
        assert np.array_equal(u8(t.cpu().numpy()), dev[k]), k
    # Round trip: the reloaded blocks hold the offloaded bytes, specials included.
    for k, a in enumerate(kv_np + sc_np):
        got = (kv + sc)[k].cpu().numpy()
        assert np.array_equal(u8(got[back]), u8(a[ids]))
    mgr.close()


def test_fp8_chunk_with_partial_payload_and_scales_matches_oracle(kvx, oracle, cuda):
    """1.5 MiB staging chunks over 8 payload storages x 40 ids of 16 KiB:
    three chunks of payload alone, then a chunk holding the last 32 payload
    blocks (starting inside a storage) together with every scale block, so
    one launch carries a payload piece that does not start at a storage
    boundary beside the scale piece, in both directions."""
    rng = np.random.default_rng(43)
    layers, blocks, host_blocks, n = 4, 96, 64, 40
    kv_np, sc_np, kv, sc, bb = build(rng, cuda, layers, blocks)
    mgr = kvx.KVCacheManager(kv, host_blocks_to_allocate=host_blocks, scale_tables=sc,
                             transfer_mode="staged", staging_chunk_bytes=96 * bb,
                             staging_chunks=2)
    dev = [u8(a).copy() for a in kv_np + sc_np]
    host = [np.zeros(host_blocks * (bb if k < 2 * layers else 32), np.uint8)
            for k in range(3 * layers)]
    bbs = [bb] * (2 * layers) + [32] * layers
    ids = rng.choice(blocks, n, replace=False).tolist()
    slot = rng.permutation(host_blocks)[:n].tolist()
    before = mgr.engine_stats()["kernel_launches"]
    mgr.d2h(ids, slot).Await()
    assert mgr.engine_stats()["kernel_launches"] - before == 4
    assert oracle.transfer(True, dev, host, bbs, [d.nbytes for d in dev], ids, slot,
                           [1] * n) == 0
    for k in range(3 * layers):
        assert np.array_equal(mgr.host_view(k), host[k]), k
    back = rng.choice(blocks, n, replace=False).tolist()
    mgr.h2d(slot, back).Await()
    assert oracle.transfer(False, dev, host, bbs, [d.nbytes for d in dev], slot, back,
                           [1] * n) == 0
    torch.cuda.synchronize()
    for k, t in enumerate(kv + sc):
        assert np.array_equal(u8(t.cpu().numpy()), dev[k]), k
    mgr.close()


@pytest.mark.parametrize("n", [20, 21, 23, 1])
def test_fp8_device_gather_moves_scales_in_the_same_launch(kvx, oracle, cuda, n):
    """Payload and scales of n ids in one launch (the fast kernel behind
    the scale piece), n from 1 to 23, byte for byte."""
    rng = np.random.default_rng(41 + n)
    layers, blocks = 3, 64
    kv_np, sc_np, kv, sc, bb = build(rng, cuda, layers, blocks)
    mgr = kvx.KVCacheManager(kv, host_blocks_to_allocate=4, scale_tables=sc)
    ids = rng.choice(blocks, n, replace=False).tolist()
    n = len(ids)
    staging = torch.zeros(2 * layers * n * bb + layers * n * 32, dtype=torch.uint8,
                          device=cuda)
    before = mgr.engine_stats()["kernel_launches"]
    mgr.gather(ids, staging).Await()
    assert mgr.engine_stats()["kernel_launches"] - before == 1
    rc, want_kv = oracle.extract(kv_np, bb, ids)
    assert rc == 0
    rc, want_sc = oracle.extract([u8(a) for a in sc_np], 32, ids)
    assert rc == 0
    got = staging.cpu().numpy()
    assert np.array_equal(got[:want_kv.size], want_kv)
    assert np.array_equal(got[want_kv.size:], want_sc)
    # Scatter the staging image into other blocks and compare.
    dst = [i for i in range(blocks) if i not in ids][:n]
    mgr.scatter(dst, staging).Await()
    torch.cuda.synchronize()
    for k, a in enumerate(kv_np + sc_np):
        assert np.array_equal(u8((kv + sc)[k].cpu().numpy()[dst]), u8(a[ids]))
    mgr.close()


@pytest.mark.parametrize("heads", [1, 5, 8])
def test_fp8_scale_rows_of_any_width(kvx, oracle, cuda, heads):
    """Scale rows of 4, 20 and 32 bytes: the launch's vector width follows
    the narrowest row (4-byte vectors for 4 and 20), payload included, and
    the scale piece still moves in the payload's launch."""
    rng = np.random.default_rng(44 + heads)
    layers, blocks, n = 2, 48, 17
    kv_np, sc_np, kv, sc, bb = build(rng, cuda, layers, blocks, heads=heads)
    mgr = kvx.KVCacheManager(kv, host_blocks_to_allocate=32, scale_tables=sc)
    assert mgr.block_bytes(2 * layers) == 4 * heads
    ids = rng.choice(blocks, n, replace=False).tolist()
    staging = torch.zeros(2 * layers * n * bb + layers * n * 4 * heads, dtype=torch.uint8,
                          device=cuda)
    before = mgr.engine_stats()["kernel_launches"]
    mgr.gather(ids, staging).Await()
    assert mgr.engine_stats()["kernel_launches"] - before == 1
    rc, want_kv = oracle.extract(kv_np, bb, ids)
    assert rc == 0
    rc, want_sc = oracle.extract([u8(a) for a in sc_np], 4 * heads, ids)
    assert rc == 0
    got = staging.cpu().numpy()
    assert np.array_equal(got[:want_kv.size], want_kv)
    assert np.array_equal(got[want_kv.size:], want_sc)
    dst = [i for i in range(blocks) if i not in ids][:n]
    mgr.scatter(dst, staging).Await()
    torch.cuda.synchronize()
    for k, a in enumerate(kv_np + sc_np):
        assert np.array_equal(u8((kv + sc)[k].cpu().numpy()[dst]), u8(a[ids])), k
    # Untouched blocks keep their bytes.
    rest = [i for i in range(blocks) if i not in dst]
    for k, a in enumerate(kv_np + sc_np):
        assert np.array_equal(u8((kv + sc)[k].cpu().numpy()[rest]), u8(a[rest])), k
    mgr.close()


@pytest.mark.parametrize("seed", range(6))
def test_payload_and_side_tables_of_random_shapes(kvx, oracle, cuda, seed):
    """Random payload block sizes (16-, 4- and 2-byte multiples, so every
    vector width of the one-launch kernel) with side tables of 1-64 fp32 per
    block, random ids and small staging chunks that cut payload pieces inside
    storages: staged offload + reload and device gather + scatter, all
    against the oracle."""
    rng = np.random.default_rng(900 + seed)
    layers = int(rng.integers(1, 4))
    blocks, n = 40, int(rng.integers(1, 24))
    bb = int(rng.choice([8192, 12992, 20000, 32768, 10002, 16388]))
    k = int(rng.integers(1, 65))
    kv_np = [rng.integers(0, 256, (blocks, bb), dtype=np.uint8) for _ in range(2 * layers)]
    sc_np = [fp32_scales(rng, blocks, k) for _ in range(layers)]
    kv = [torch.from_numpy(a).to(cuda) for a in kv_np]
    sc = [torch.from_numpy(a).to(cuda) for a in sc_np]
    chunk = int(rng.integers(2, 6)) * bb + int(rng.integers(0, bb))
    mgr = kvx.KVCacheManager(kv, host_blocks_to_allocate=32, scale_tables=sc,
                             transfer_mode="staged", staging_chunk_bytes=chunk, staging_chunks=2)
    dev = [u8(a).copy() for a in kv_np + sc_np]
    bbs = [bb] * (2 * layers) + [4 * k] * layers
    host = [np.zeros(32 * b, np.uint8) for b in bbs]
    ids = rng.choice(blocks, n, replace=False).tolist()
    slot = rng.permutation(32)[:n].tolist()
    mgr.d2h(ids, slot).Await()
    assert oracle.transfer(True, dev, host, bbs, [d.nbytes for d in dev], ids, slot,
                           [1] * n) == 0
    for i in range(3 * layers):
        assert np.array_equal(mgr.host_view(i), host[i]), i
    back = rng.choice(blocks, n, replace=False).tolist()
    mgr.h2d(slot, back).Await()
    assert oracle.transfer(False, dev, host, bbs, [d.nbytes for d in dev], slot, back,
                           [1] * n) == 0
    torch.cuda.synchronize()
    for i, t in enumerate(kv + sc):
        assert np.array_equal(u8(t.cpu().numpy()), dev[i]), i
    # Device gather and scatter of the same storages in one launch each.
    g_ids = rng.choice(blocks, n, replace=False).tolist()
    staging = torch.zeros(2 * layers * n * bb + layers * n * 4 * k, dtype=torch.uint8,
                          device=cuda)
    mgr.gather(g_ids, staging).Await()
    want = np.concatenate([u8(a.reshape(blocks, -1)[g_ids]) for a in
                           [d.reshape(blocks, -1) for d in dev]])
    assert np.array_equal(staging.cpu().numpy(), want)
    dst = rng.choice(blocks, n, replace=False).tolist()
    mgr.scatter(dst, staging).Await()
    torch.cuda.synchronize()
    for i, t in enumerate(kv + sc):
        rows = dev[i].reshape(blocks, -1)
        rows[dst] = staging.cpu().numpy()[
            sum(n * b for b in bbs[:i]):sum(n * b for b in bbs[:i + 1])].reshape(n, -1)
        assert np.array_equal(u8(t.cpu().numpy()), dev[i]), i
    mgr.close()


def test_fp8_llama3_8b_pool_full_size_round_trip(kvx, cuda):
    """32 layers x 16384 blocks of fp8 KV (16 GiB) plus 32 scale tables: a
    512-block offload into a host slot and a reload into 512 other random
    blocks, checked per block on the device."""
    layers, blocks, heads, bb, n = 32, 16384, 8, 16 * 8 * 128, 512
    gen = torch.Generator(device=cuda).manual_seed(4)
    kv = [torch.randint(0, 256, (blocks, bb), dtype=torch.uint8, device=cuda, generator=gen)
          for _ in range(2 * layers)]
    sc = [torch.randn(blocks, heads, device=cuda, generator=gen) for _ in range(layers)]
    # NaN / denormal words in every scale table.
    for t in sc:
        w = t.view(torch.int32)
        w[::997, 0] = 0x7FC00001
        w[5::991, 1] = 0x00000001
    mgr = kvx.KVCacheManager(kv, host_blocks_to_allocate=n, scale_tables=sc)
    perm = torch.randperm(blocks, generator=torch.Generator().manual_seed(5)).tolist()
    src, dst = perm[:n], perm[n:2 * n]
    src_t = torch.tensor(src, device=cuda)
    dst_t = torch.tensor(dst, device=cuda)
    saved = [t.index_select(0, src_t).clone() for t in kv + sc]
    mgr.d2h(src, list(range(n))).Await()
    mgr.h2d(list(range(n)), dst).Await()
    torch.cuda.synchronize()
    for k, t in enumerate(kv + sc):
        got = t.index_select(0, dst_t)
        assert torch.equal(got.view(torch.uint8), saved[k].view(torch.uint8)), k
    mgr.close()
