"""GPU parity: the HIP path (libkvx through its C-ABI) against the oracle on
the same seeded inputs, bit-exact. Covers the direct, staged (gather/scatter
kernel + pipelined DMA), zero-copy, bounce-lane (pageable mirrors) and
runtime-pageable paths, every vector width of the kernel and its tail,
layer/shard/slot restrictions, the reference's e2e known answers, device
gather/scatter, bad ids, empty copies, threads, the auto-mode choice and a
full-size Llama-3-8B pool round trip.
"""
import os
import threading

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


def dev_pools(rng, cuda, layers, shards, blocks, bb):
    host = [[rng.integers(0, 256, size=(blocks, bb), dtype=np.uint8) for _ in range(shards)]
            for _ in range(layers)]
    dev = [[torch.from_numpy(h).to(cuda) for h in row] for row in host]
    return host, dev


def dev_np(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def flat(rows):
    return [x for row in rows for x in row]


def make_mgr(kvx, dev, host_blocks, **kw):
    caches = [row if len(row) > 1 else row[0] for row in dev]
    return kvx.KVCacheManager(caches, host_blocks_to_allocate=host_blocks, **kw)


class Mirror:
    """Oracle-side copy of a manager's device pools and host mirror."""

    def __init__(self, host_pools, host_blocks):
        self.dev = [p.reshape(-1).copy() for p in flat(host_pools)]
        bb = host_pools[0][0].shape[1]
        self.bb = bb
        self.host = [np.zeros(host_blocks * bb, np.uint8) for _ in self.dev]
        self.layers = len(host_pools)
        self.shards = len(host_pools[0])

    def select(self, layer=None, shard=None):
        ks = [l * self.shards + s for l in range(self.layers) for s in range(self.shards)
              if (layer is None or l == layer) and (shard is None or s == shard)]
        return ks

    def transfer(self, d2h, src, dst, sizes, layer=None, shard=None, host_base=0,
                 host_len=None):
        ks = self.select(layer, shard)
        dev = [self.dev[k] for k in ks]
        host = [self.host[k][host_base:host_base + host_len] if host_len is not None
                else self.host[k] for k in ks]
        n = len(ks)
        return self._run(d2h, dev, host, n, src, dst, sizes)

    def _run(self, d2h, dev, host, n, src, dst, sizes):
        import oracle
        return oracle.transfer(d2h, dev, host, [self.bb] * n, [d.nbytes for d in dev],
                               src, dst, sizes)

    def check(self, mgr, dev):
        torch.cuda.synchronize()
        for k, t in enumerate(flat(dev)):
            assert np.array_equal(t.cpu().numpy().reshape(-1), self.dev[k]), f"device {k}"
        for l in range(self.layers):
            for s in range(self.shards):
                k = l * self.shards + s
                assert np.array_equal(mgr.host_view(l, s), self.host[k]), f"host {k}"


def random_spec(rng, blocks, host_blocks, max_entries=8, max_run=3):
    src, dst, sizes = [], [], []
    used_dst = set()
    for _ in range(int(rng.integers(1, max_entries + 1))):
        z = int(rng.integers(1, max_run + 1))
        s = int(rng.integers(0, blocks - z + 1))
        d = int(rng.integers(0, host_blocks - z + 1))
        if any(x in used_dst for x in range(d, d + z)):
            continue
        used_dst.update(range(d, d + z))
        src.append(s)
        dst.append(d)
        sizes.append(z)
    return src, dst, sizes


PATHS = {
    # Every run moves directly (staged mode: auto mode would move short runs
    # zero-copy when the other direction is idle).
    "direct": dict(direct_min_bytes=1, transfer_mode="staged"),
    "staged": dict(direct_min_bytes=1 << 40, staging_chunk_bytes=1 << 16, staging_chunks=2,
                   transfer_mode="staged"),
    "zero_copy": dict(direct_min_bytes=1 << 40, transfer_mode="zero_copy"),
    # Pageable mirror through the pinned bounce lanes: 2 slots of 64 KiB, so
    # slots are drained and refilled inside one copy; 3 host threads.
    "bounce": dict(direct_min_bytes=1 << 40, staging_chunk_bytes=1 << 16, staging_chunks=2,
                   host_alloc="malloc", host_copy_threads=3),
    # The same with the lanes' DMAs through hipMemcpyAsync (KVX_LANE_DMA=hip)
    # instead of fixed SDMA engines.
    "bounce_hip": dict(direct_min_bytes=1 << 40, staging_chunk_bytes=1 << 16, staging_chunks=2,
                       host_alloc="malloc", host_copy_threads=3),
    # A pinned mirror whose short runs also go through the bounce lanes.
    "lanes": dict(direct_min_bytes=1 << 40, staging_chunk_bytes=1 << 16, staging_chunks=2,
                  host_alloc="pinned", transfer_mode="lanes", host_copy_threads=3),
    # One-slot rings: every chunk refills the slot the previous chunk's
    # scatter (H2D) or host copy (D2H) still owns.
    "bounce_1slot": dict(direct_min_bytes=1 << 40, staging_chunk_bytes=1 << 16,
                         staging_chunks=1, host_alloc="malloc", host_copy_threads=3),
    "lanes_1slot": dict(direct_min_bytes=1 << 40, staging_chunk_bytes=1 << 16, staging_chunks=1,
                        host_alloc="pinned", transfer_mode="lanes", host_copy_threads=3),
    # Pageable mirror left to the runtime's per-run hipMemcpyAsync.
    "pageable": dict(direct_min_bytes=1 << 40, staging_chunk_bytes=1 << 16, staging_chunks=2,
                     host_alloc="malloc", host_copy_threads=-1),
    # Auto mode on a pinned mirror with 64 KiB chunks: copies of more than
    # 32 chunks (2 MiB) go through the lanes, shorter ones zero-copy.
    "auto": dict(direct_min_bytes=1 << 40, staging_chunk_bytes=1 << 16, staging_chunks=2,
                 host_copy_threads=3),
}
MODES = ["staged", "zero_copy"]


@pytest.mark.parametrize("path", ["direct", "staged", "zero_copy", "bounce", "bounce_hip",
                                  "bounce_1slot", "lanes", "lanes_1slot", "pageable", "auto"])
@pytest.mark.parametrize("bb", [32768, 61424, 12992, 1024, 48, 36, 3])
def test_random_d2h_h2d_match_oracle(kvx, oracle, cuda, monkeypatch, path, bb):
    if path == "bounce_hip":
        monkeypatch.setenv("KVX_LANE_DMA", "hip")
    rng = np.random.default_rng(bb * 7 + len(path))
    layers, shards, blocks, hb = 3, 2, 40, 30
    host, dev = dev_pools(rng, cuda, layers, shards, blocks, bb)
    mgr = make_mgr(kvx, dev, hb, **PATHS[path])
    mir = Mirror(host, hb)
    for step in range(12):
        d2h = step % 2 == 0
        if d2h:
            src, dst, sizes = random_spec(rng, blocks, hb)
        else:
            dst, src, sizes = random_spec(rng, blocks, hb)
        layer = int(rng.integers(0, layers)) if step % 5 == 3 else None
        shard = int(rng.integers(0, shards)) if step % 7 == 4 else None
        fn = mgr.d2h if d2h else mgr.h2d
        print(f"path={path} bb={bb} step={step} d2h={d2h} spec={src},{dst},{sizes} "
              f"layer={layer} shard={shard}", flush=True)
        fn(src, dst, sizes, layer_idx=layer, shard_idx=shard).Await()
        assert mir.transfer(d2h, src, dst, sizes, layer, shard) == 0
        mir.check(mgr, dev)
    stats = mgr.engine_stats()
    if path in ("staged", "bounce", "bounce_hip", "bounce_1slot", "lanes", "lanes_1slot",
                "pageable"):
        assert stats["direct_copies"] == 0 and stats["staged_copies"] == 12
        assert stats["chunks"] > 12 or bb < 1024
        lanes = path.startswith("bounce") or path.startswith("lanes")
        assert stats["bounce_copies"] == (12 if lanes else 0)
    elif path == "zero_copy":
        assert stats["zero_copy_copies"] == 12 and stats["memcpy_calls"] == 0
    elif path == "auto":
        # Every copy is zero-copy or (past 32 chunks) a lane copy.
        assert stats["zero_copy_copies"] + stats["bounce_copies"] == 12, stats
        assert stats["staged_copies"] == stats["bounce_copies"], stats
        if bb >= 32768:
            assert stats["bounce_copies"] > 0, stats
    else:
        assert stats["staged_copies"] == 0 and stats["zero_copy_copies"] == 0
    # The lanes' DMAs: one SDMA engine bit per direction, or hipMemcpyAsync.
    if path in ("bounce", "bounce_1slot", "lanes", "lanes_1slot"):
        engines = mgr.lane_dma_engines
        assert engines is not None and all(e and e & (e - 1) == 0 for e in engines), engines
    elif path == "bounce_hip":
        assert mgr.lane_dma_engines is None
    mgr.close()


@pytest.mark.parametrize("mode", MODES)
def test_scattered_ids_match_oracle_many_chunks(kvx, cuda, mode):
    """512 random single-block ids over 8 storages (staged: through a 2-chunk
    ring of 256 KiB, so chunk boundaries fall inside a storage and the ring is
    reused across calls; zero-copy: one kernel per call)."""
    rng = np.random.default_rng(21)
    layers, blocks, hb, bb = 8, 1024, 600, 4096
    host, dev = dev_pools(rng, cuda, layers, 1, blocks, bb)
    mgr = make_mgr(kvx, dev, hb, staging_chunk_bytes=256 << 10, staging_chunks=2,
                   transfer_mode=mode)
    mir = Mirror(host, hb)
    for rep in range(3):
        ids = rng.choice(blocks, size=512, replace=False).tolist()
        hids = rng.choice(hb, size=512, replace=False).tolist()
        print(f"rep={rep} offload 512 ids", flush=True)
        mgr.d2h(ids, hids).Await()
        assert mir.transfer(True, ids, hids, []) == 0
        mir.check(mgr, dev)
        back = rng.choice(blocks, size=512, replace=False).tolist()
        mgr.h2d(hids, back).Await()
        assert mir.transfer(False, hids, back, []) == 0
        mir.check(mgr, dev)
    mgr.close()


def test_auto_moves_long_pinned_copies_through_the_lanes(kvx, cuda):
    """Auto mode on a pinned mirror: a copy of more than 32 staging chunks
    goes through the lanes (issued chunk by chunk), a shorter one stays on
    the stream-ordered paths (zero-copy here: its host runs are shorter than
    4 MiB); every copy, and a load and a save in flight together, byte for
    byte the oracle's. 8 storages x 4 KiB blocks, 64 KiB chunks: 32 chunks
    are 64 blocks."""
    rng = np.random.default_rng(41)
    layers, blocks, hb, bb = 8, 1024, 700, 4096
    host, dev = dev_pools(rng, cuda, layers, 1, blocks, bb)
    mgr = make_mgr(kvx, dev, hb, staging_chunk_bytes=1 << 16, staging_chunks=2,
                   direct_min_bytes=1 << 40, host_copy_threads=3)
    mir = Mirror(host, hb)
    want = {"bounce_copies": 0, "zero_copy_copies": 0, "staged_copies": 0}
    for n, scattered, path in ((64, True, "zero_copy_copies"), (65, True, "bounce_copies"),
                               (300, True, "bounce_copies"), (300, False, "bounce_copies"),
                               (48, False, "zero_copy_copies")):
        ids = rng.choice(blocks, size=n, replace=False).tolist()
        hids = (rng.choice(hb, size=n, replace=False) if scattered
                else np.arange(n) + int(rng.integers(0, hb - n))).tolist()
        print(f"n={n} scattered={scattered} expect {path}", flush=True)
        mgr.d2h(ids, hids).Await()
        assert mir.transfer(True, ids, hids, []) == 0
        mir.check(mgr, dev)
        back = rng.choice(blocks, size=n, replace=False).tolist()
        mgr.h2d(hids, back).Await()
        assert mir.transfer(False, hids, back, []) == 0
        mir.check(mgr, dev)
        want[path] += 2
        if path == "bounce_copies":
            want["staged_copies"] += 2  # a lane copy is a staged copy too
        stats = mgr.engine_stats()
        assert {k: stats[k] for k in want} == want, (n, scattered, stats)
    # A long load and a long save in flight together (disjoint host ranges).
    hids = rng.choice(hb, size=600, replace=False).tolist()
    ids = rng.choice(blocks, size=300, replace=False).tolist()
    mgr.d2h(ids, hids[:300]).Await()
    assert mir.transfer(True, ids, hids[:300], []) == 0
    back = rng.choice(blocks, size=300, replace=False).tolist()
    save_ids = [b for b in rng.permutation(blocks).tolist() if b not in set(back)][:300]
    f1 = mgr.h2d(hids[:300], back)
    f2 = mgr.d2h(save_ids, hids[300:])
    f1.Await()
    f2.Await()
    assert mir.transfer(True, save_ids, hids[300:], []) == 0
    assert mir.transfer(False, hids[:300], back, []) == 0
    mir.check(mgr, dev)
    mgr.close()


def test_auto_bounds_staged_chunks_in_flight(kvx, cuda):
    """Auto mode keeps at most 32 staged chunks of a direction in flight: five
    staged offloads of 8 chunks each, issued while the stream they depend on
    is held by a spin kernel, go staged four times and through the lanes the
    fifth time; all five land byte for byte. 8 storages x 1 MiB blocks, 4 MiB
    chunks: 4 contiguous blocks are 4 MiB runs (staged), 8 chunks."""
    rng = np.random.default_rng(43)
    layers, blocks, hb, bb = 8, 64, 24, 1 << 20
    host, dev = dev_pools(rng, cuda, layers, 1, blocks, bb)
    mgr = make_mgr(kvx, dev, hb, staging_chunk_bytes=4 << 20, staging_chunks=2,
                   direct_min_bytes=1 << 40, host_copy_threads=3)
    mir = Mirror(host, hb)
    hold = torch.cuda.Stream(cuda)
    torch.cuda.synchronize()
    with torch.cuda.stream(hold):
        torch.cuda._sleep(200_000_000)  # bounded spin, well past the issue below
    futs, copies = [], []
    for k in range(5):
        ids = rng.choice(blocks, size=4, replace=False).tolist()
        hids = list(range(4 * k, 4 * k + 4))
        futs.append(mgr.d2h(ids, hids, stream=hold))
        copies.append((ids, hids))
    for f in futs:
        f.Await()
    for ids, hids in copies:
        assert mir.transfer(True, ids, hids, []) == 0
    mir.check(mgr, dev)
    stats = mgr.engine_stats()
    assert stats["staged_copies"] == 5 and stats["bounce_copies"] == 1, stats
    assert stats["zero_copy_copies"] == 0 and stats["direct_copies"] == 0, stats
    mgr.close()


@pytest.mark.parametrize("mode", MODES)
def test_duplicate_destinations_last_wins(kvx, cuda, mode):
    rng = np.random.default_rng(3)
    host, dev = dev_pools(rng, cuda, 2, 1, 16, 256)
    mgr = make_mgr(kvx, dev, 8, direct_min_bytes=1 << 40, transfer_mode=mode)
    # Two device blocks to host block 5: the later entry wins, as when the
    # copies are issued in order.
    mgr.d2h([1, 9], [5, 5], [1, 1]).Await()
    for l in range(2):
        assert np.array_equal(mgr.host_view(l).reshape(8, 256)[5], host[l][0][9])
    # Two host blocks to device block 3.
    mgr.h2d([5, 0], [3, 3], [1, 1]).Await()
    for l in range(2):
        assert not dev_np(dev[l][0])[3].any()  # host block 0 is still zero
    mgr.close()


def test_reference_known_answers_dtypes(kvx, cuda, golden):
    """The reference's e2e cases (shift copy, partial chunks, auto-allocate,
    whole-layer copy) at their block shape (128, 8, 8, 128) for fp8, bf16,
    fp32 and int32 byte widths, on every copy path."""
    elems = 128 * 8 * 8 * 128
    for itemsize, dtype in [(1, "fp8"), (2, "bf16"), (4, "fp32"), (4, "int32")]:
        for path in ("direct", "staged", "zero_copy", "bounce", "big_blocks"):
            for case in golden["transfer_cases"]:
                L, P, H = case["layers"], case["blocks"], case["host_blocks"]
                rng = np.random.default_rng(101)
                host, dev = dev_pools(rng, cuda, L, 1, P, elems * itemsize)
                kw = {"staged": dict(direct_min_bytes=1 << 40, transfer_mode="staged"),
                      # pageable mirror: block copies and whole-layer copies
                      # through the bounce lanes
                      "bounce": dict(direct_min_bytes=1 << 40, host_alloc="malloc"),
                      # blocks larger than a staging chunk: one DMA per run
                      "big_blocks": dict(direct_min_bytes=1 << 40, staging_chunk_bytes=1 << 16,
                                         transfer_mode="staged")}.get(path, None)
                mgr = make_mgr(kvx, dev, H, **(kw if kw is not None else PATHS[path]))
                print(f"{dtype} {path} {case['source']}", flush=True)
                for op in case["ops"]:
                    if op["op"] == "d2h_auto_allocate":
                        ids, f = mgr.d2h_auto_allocate(op["src"], op["sizes"])
                        assert ids == op["expect_ids"]
                        f.Await()
                    elif op["op"] == "d2h":
                        mgr.d2h(op["src"], op["dst"], op["sizes"]).Await()
                    else:
                        mgr.h2d(op["src"], op["dst"], op["sizes"]).Await()
                for l in range(L):
                    got = dev_np(dev[l][0])
                    for e in case["expect_device"]:
                        assert np.array_equal(got[e["dst"]], host[l][0][e["orig"]]), \
                            (dtype, path, case["source"])
                mgr.close()


@pytest.mark.parametrize("bb", [2048, 12992])
@pytest.mark.parametrize("block_major", [False, True])
def test_device_gather_scatter_match_oracle(kvx, oracle, cuda, block_major, bb):
    """bb 2048: many blocks per workgroup; bb 12992 (812 vectors): one block
    per workgroup on the single-piece fast path, its 4/2/1-vector tail, and
    the scatter's storage-interleaved order."""
    rng = np.random.default_rng(8)
    L, P = 6, 96
    host, dev = dev_pools(rng, cuda, L, 1, P, bb)
    mgr = make_mgr(kvx, dev, 4)
    ids = rng.choice(P, size=40, replace=False)
    stg = torch.empty(L * len(ids) * bb, dtype=torch.uint8, device=cuda)
    mgr.gather(ids.tolist(), stg, block_major=block_major).Await()
    rc, want = oracle.extract([h[0].reshape(-1) for h in host], bb, ids,
                              order=1 if block_major else 0)
    assert rc == 0
    assert np.array_equal(dev_np(stg), want)
    # Scatter the staging into fresh pools at other ids.
    fresh = [[torch.zeros(P, bb, dtype=torch.uint8, device=cuda)] for _ in range(L)]
    mgr2 = make_mgr(kvx, fresh, 4)
    dst = rng.choice(P, size=40, replace=False)
    mgr2.scatter(dst.tolist(), stg, block_major=block_major).Await()
    ref = [np.zeros(P * bb, np.uint8) for _ in range(L)]
    assert oracle.insert(ref, bb, dst, want, order=1 if block_major else 0) == 0
    for l in range(L):
        assert np.array_equal(dev_np(fresh[l][0]).reshape(-1), ref[l])
    # One layer only.
    stg1 = torch.empty(len(ids) * bb, dtype=torch.uint8, device=cuda)
    mgr.gather(ids.tolist(), stg1, layer_idx=2).Await()
    assert np.array_equal(dev_np(stg1).reshape(len(ids), bb), host[2][0][ids])
    with pytest.raises(kvx.KvxError) as e:
        mgr2.scatter([1, 1], stg)
    assert e.value.code == 3
    with pytest.raises(kvx.KvxError) as e:
        mgr.gather([P], stg)
    assert e.value.code == 11
    with pytest.raises(kvx.KvxError) as e:
        mgr.gather(ids.tolist(), stg1)  # staging too small for all layers
    assert e.value.code == 3
    mgr.close()
    mgr2.close()


def test_raw_kernel_bad_id_flag(kvx, cuda):
    rng = np.random.default_rng(9)
    W, P, bb, n = 3, 20, 512, 6
    pools = [torch.from_numpy(rng.integers(0, 256, (P, bb), dtype=np.uint8)).to(cuda)
             for _ in range(W)]
    table = torch.tensor([p.data_ptr() for p in pools], dtype=torch.int64, device=cuda)
    ids = torch.tensor([3, 19, 20, 0, -1, 7], dtype=torch.int64, device=cuda)
    stg = torch.full((W, n, bb), 0xAB, dtype=torch.uint8, device=cuda)
    err = torch.zeros(1, dtype=torch.int32, device=cuda)
    lib = kvx._capi.load()
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.kvx_gather_blocks(table.data_ptr(), W, bb, P, ids.data_ptr(), n,
                               stg.data_ptr(), 0, err.data_ptr(), stream)
    assert rc == 0
    torch.cuda.synchronize()
    assert int(err.item()) == 1
    got = stg.cpu().numpy()
    for w in range(W):
        ref = pools[w].cpu().numpy()
        for i, b in enumerate([3, 19, 20, 0, -1, 7]):
            if 0 <= b < P:
                assert np.array_equal(got[w, i], ref[b])
            else:
                assert (got[w, i] == 0xAB).all()
    # Scatter back block-major into zeroed pools; bad ids write nothing.
    zero = [torch.zeros(P, bb, dtype=torch.uint8, device=cuda) for _ in range(W)]
    table2 = torch.tensor([p.data_ptr() for p in zero], dtype=torch.int64, device=cuda)
    stg_bm = stg.permute(1, 0, 2).contiguous()
    err.zero_()
    rc = lib.kvx_scatter_blocks(table2.data_ptr(), W, bb, P, ids.data_ptr(), n,
                                stg_bm.data_ptr(), 1, err.data_ptr(), stream)
    assert rc == 0
    torch.cuda.synchronize()
    assert int(err.item()) == 1
    for w in range(W):
        z = zero[w].cpu().numpy()
        for b in (3, 19, 0, 7):
            assert np.array_equal(z[b], pools[w].cpu().numpy()[b])
        assert z.sum(dtype=np.int64) == sum(int(pools[w].cpu().numpy()[b].sum(dtype=np.int64))
                                            for b in (3, 19, 0, 7))
    assert lib.kvx_gather_blocks(0, W, bb, P, ids.data_ptr(), n, stg.data_ptr(), 0, 0,
                                 stream) == 3


@pytest.mark.parametrize("bb", [32768, 16384])
@pytest.mark.parametrize("n", [1, 2, 3, 4, 5, 7, 8, 33, 510])
@pytest.mark.parametrize("W,order", [(2, 0), (4, 1), (6, 0)])
def test_sliced_gather_matches_oracle(kvx, oracle, cuda, n, W, order, bb):
    """32 KiB blocks at 16-byte vectors over an even number of whole
    storages take the sliced gather (a quarter of each of 4 consecutive ids
    per workgroup; 16 KiB blocks, the fast kernel, alongside): any n, so the
    last group holds 1-4 ids, duplicate ids, layer-major (0) and block-major
    (1) staging, byte for byte against the oracle's extract."""
    rng = np.random.default_rng(1000 + 10 * n + W + bb)
    P = 600
    host = [rng.integers(0, 256, (P, bb), dtype=np.uint8) for _ in range(W)]
    pools = [torch.from_numpy(h).to(cuda) for h in host]
    table = torch.tensor([p.data_ptr() for p in pools], dtype=torch.int64, device=cuda)
    id_list = rng.integers(0, P, size=n)
    ids = torch.tensor(id_list, dtype=torch.int64, device=cuda)
    stg = torch.full((W * n * bb,), 0x3D, dtype=torch.uint8, device=cuda)
    err = torch.zeros(1, dtype=torch.int32, device=cuda)
    lib = kvx._capi.load()
    stream = torch.cuda.current_stream().cuda_stream
    assert lib.kvx_gather_blocks(table.data_ptr(), W, bb, P, ids.data_ptr(), n,
                                 stg.data_ptr(), order, err.data_ptr(), stream) == 0
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    rc, want = oracle.extract([h.reshape(-1) for h in host], bb, id_list, order=order)
    assert rc == 0
    assert np.array_equal(stg.cpu().numpy(), want)


@pytest.mark.parametrize("bb", [32768, 16384])
def test_sliced_gather_bad_ids_in_a_group_and_in_the_last(kvx, cuda, bb):
    """The sliced gather (32 KiB blocks; 16 KiB blocks, the fast kernel,
    alongside) with bad ids: two in the first group of 4, one in the second,
    one in the last (short) group. Good blocks land, bad ones leave their
    staging untouched, and the error flag is set."""
    rng = np.random.default_rng(31)
    W, P = 2, 20
    id_list = [3, 20, 5, -1, 8, 9, 99, 0, 7, -2]
    n = len(id_list)
    pools = [torch.from_numpy(rng.integers(0, 256, (P, bb), dtype=np.uint8)).to(cuda)
             for _ in range(W)]
    table = torch.tensor([p.data_ptr() for p in pools], dtype=torch.int64, device=cuda)
    ids = torch.tensor(id_list, dtype=torch.int64, device=cuda)
    stg = torch.full((W, n, bb), 0xAB, dtype=torch.uint8, device=cuda)
    err = torch.zeros(1, dtype=torch.int32, device=cuda)
    lib = kvx._capi.load()
    stream = torch.cuda.current_stream().cuda_stream
    assert lib.kvx_gather_blocks(table.data_ptr(), W, bb, P, ids.data_ptr(), n,
                                 stg.data_ptr(), 0, err.data_ptr(), stream) == 0
    torch.cuda.synchronize()
    assert int(err.item()) == 1
    got = stg.cpu().numpy()
    for w in range(W):
        ref = pools[w].cpu().numpy()
        for i, b in enumerate(id_list):
            if 0 <= b < P:
                assert np.array_equal(got[w, i], ref[b]), (w, i)
            else:
                assert (got[w, i] == 0xAB).all(), (w, i)


@pytest.mark.parametrize("bb", [16, 48, 36, 3, 1024])
@pytest.mark.parametrize("id_list", [[-1, 25, 4, 99, 11], [-5, 30, 21]])
def test_raw_small_blocks_bad_first_or_all(kvx, cuda, bb, id_list):
    """Small-block path (many blocks per workgroup): a workgroup whose first
    blocks have bad ids, and one whose blocks all have bad ids, move exactly
    the good blocks and flag the bad ones."""
    rng = np.random.default_rng(bb + len(id_list))
    W, P = 4, 21
    n = len(id_list)
    pools = [torch.from_numpy(rng.integers(0, 256, (P, bb), dtype=np.uint8)).to(cuda)
             for _ in range(W)]
    table = torch.tensor([p.data_ptr() for p in pools], dtype=torch.int64, device=cuda)
    ids = torch.tensor(id_list, dtype=torch.int64, device=cuda)
    stg = torch.full((W, n, bb), 0x5C, dtype=torch.uint8, device=cuda)
    err = torch.zeros(1, dtype=torch.int32, device=cuda)
    lib = kvx._capi.load()
    stream = torch.cuda.current_stream().cuda_stream
    assert lib.kvx_gather_blocks(table.data_ptr(), W, bb, P, ids.data_ptr(), n,
                                 stg.data_ptr(), 0, err.data_ptr(), stream) == 0
    torch.cuda.synchronize()
    assert int(err.item()) == 1
    got = stg.cpu().numpy()
    for w in range(W):
        ref = pools[w].cpu().numpy()
        for i, b in enumerate(id_list):
            if 0 <= b < P:
                assert np.array_equal(got[w, i], ref[b])
            else:
                assert (got[w, i] == 0x5C).all()
    zero = [torch.zeros(P, bb, dtype=torch.uint8, device=cuda) for _ in range(W)]
    table2 = torch.tensor([p.data_ptr() for p in zero], dtype=torch.int64, device=cuda)
    err.zero_()
    assert lib.kvx_scatter_blocks(table2.data_ptr(), W, bb, P, ids.data_ptr(), n,
                                  stg.data_ptr(), 0, err.data_ptr(), stream) == 0
    torch.cuda.synchronize()
    assert int(err.item()) == 1
    good = [b for b in id_list if 0 <= b < P]
    for w in range(W):
        z = zero[w].cpu().numpy()
        want = np.zeros_like(z)
        want[good] = pools[w].cpu().numpy()[good]
        assert np.array_equal(z, want)


def bf16_normal(rng, shape):
    """float32 N(0,1) rounded to bf16 (nearest even) on the bit pattern."""
    x = rng.standard_normal(shape, dtype=np.float32).view(np.uint32)
    r = ((x >> 16) & 1) + 0x7FFF
    return ((x + r) >> 16).astype(np.uint16)


def test_cpu_only_config_round_trip(kvx, oracle, cuda):
    """2 layers x 64 blocks x 16 tokens x 8 heads x 128 dim, K and V
    separate, bf16 N(0,1); extract 16 unique ids into a contiguous buffer,
    insert into a fresh pool; byte-exact, checked against the oracle."""
    rng = np.random.default_rng(0)
    L, P, T, H, D = 2, 64, 16, 8, 128
    S = 2 * L
    bb = T * H * D * 2
    pools_np = [bf16_normal(rng, (P, T * H * D)).view(np.uint8).reshape(P, bb)
                for _ in range(S)]
    ids = rng.choice(P, size=16, replace=False)
    rc, want = oracle.extract([p.reshape(-1) for p in pools_np], bb, ids)
    assert rc == 0
    pools = [torch.from_numpy(p).to(cuda) for p in pools_np]
    mgr = kvx.KVCacheManager(pools, host_blocks_to_allocate=16)
    stg = torch.empty(S * 16 * bb, dtype=torch.uint8, device=cuda)
    mgr.gather(ids.tolist(), stg).Await()
    assert np.array_equal(dev_np(stg), want)
    fresh = [torch.zeros(P, bb, dtype=torch.uint8, device=cuda) for _ in range(S)]
    mgr2 = kvx.KVCacheManager(fresh, host_blocks_to_allocate=16)
    mgr2.scatter(ids.tolist(), stg).Await()
    for s in range(S):
        got = dev_np(fresh[s])
        assert np.array_equal(got[ids], pools_np[s][ids])
        mask = np.ones(P, bool)
        mask[ids] = False
        assert not got[mask].any()
    # Same through the host tier: offload to host 0..15, reload to a fresh pool.
    mgr.d2h(ids.tolist(), list(range(16))).Await()
    for s in range(S):
        assert np.array_equal(mgr.host_view(s)[:16 * bb], want[s * 16 * bb:(s + 1) * 16 * bb])
    mgr.close()
    mgr2.close()


def test_nan_denormal_bit_patterns_preserved(kvx, cuda):
    rng = np.random.default_rng(4)
    P, bb = 32, 16 * 8 * 128
    raw = rng.integers(0, 256, (P, bb), dtype=np.uint8)
    mask = rng.random((P, bb)) < 1e-3
    special = np.array([0x7F, 0xFF, 0x01, 0x07, 0x81, 0x87], np.uint8)
    raw[mask] = rng.choice(special, size=int(mask.sum()))
    bf = bf16_normal(rng, (P, bb // 2))
    nanmask = rng.random(bf.shape) < 1e-3
    bf[nanmask] = rng.choice(np.array([0x7FC1, 0xFF81, 0x0001, 0x8001, 0x7F80], np.uint16),
                             size=int(nanmask.sum()))
    pools_np = [raw, bf.view(np.uint8).reshape(P, bb)]
    pools = [torch.from_numpy(p).to(cuda) for p in pools_np]
    for path in ("staged", "zero_copy"):
        mgr = kvx.KVCacheManager(pools, host_blocks_to_allocate=P, transfer_mode=path)
        ids = rng.permutation(P).tolist()
        mgr.d2h(ids, list(range(P))).Await()
        back = rng.permutation(P).tolist()
        mgr.h2d(list(range(P)), back).Await()
        for s in range(2):
            got = dev_np(pools[s])
            assert np.array_equal(got[back], pools_np[s][ids])
        pools_np = [dev_np(p) for p in pools]
        mgr.close()


def test_slot_addressing(kvx, cuda):
    rng = np.random.default_rng(12)
    host, dev = dev_pools(rng, cuda, 2, 1, 16, 1024)
    mgr = kvx.KVCacheManager([d[0] for d in dev], max_blocks=4, num_slots=3)
    assert mgr.host_blocks == 12
    mgr.d2h([5, 9, 2], [0, 1, 2], slot_idx=2).Await()
    for l in range(2):
        hv = mgr.host_view(l).reshape(12, 1024)
        assert np.array_equal(hv[8:11], host[l][0][[5, 9, 2]])
        assert not hv[:8].any()
    mgr.h2d([0, 1, 2], [0, 1, 2], slot_idx=2).Await()
    for l in range(2):
        assert np.array_equal(dev_np(dev[l][0])[:3], host[l][0][[5, 9, 2]])
    with pytest.raises(kvx.KvxError) as e:
        mgr.d2h([0], [4], slot_idx=0)  # beyond the slot's 4 blocks
    assert e.value.code == 3
    with pytest.raises(kvx.KvxError) as e:
        mgr.d2h([0], [0], slot_idx=3)
    assert e.value.code == 11
    mgr.close()


def test_validation_before_issue(kvx, cuda):
    rng = np.random.default_rng(13)
    host, dev = dev_pools(rng, cuda, 2, 1, 8, 256)
    mgr = make_mgr(kvx, dev, 4)
    cases = [
        (mgr.d2h, ([0, 1], [0], [1, 1]), 3),
        (mgr.d2h, ([-1], [0], [1]), 3),
        (mgr.d2h, ([7], [0], [2]), 3),      # device range
        (mgr.d2h, ([0], [3], [2]), 3),      # host range
        (mgr.h2d, ([3], [0], [2]), 3),      # host source range
        (mgr.h2d, ([0], [7], [2]), 3),      # device destination range
        (mgr.d2h, ([0], [], []), 3),        # sources without destinations
        (mgr.d2h, ([], [], []), 11),        # whole layer exceeds the host mirror
        (mgr.h2d, ([], [], []), 3),
    ]
    for fn, args, code in cases:
        with pytest.raises(kvx.KvxError) as e:
            fn(*args)
        assert e.value.code == code, (args, str(e.value))
    with pytest.raises(kvx.KvxError) as e:
        mgr.d2h([0], [0], [1], layer_idx=2)
    assert e.value.code == 11
    # Nothing was copied by any failing call.
    for l in range(2):
        assert not mgr.host_view(l).any()
    mgr.close()


def test_futures_and_stream_order(kvx, cuda):
    rng = np.random.default_rng(14)
    host, dev = dev_pools(rng, cuda, 4, 1, 64, 65536)
    mgr = make_mgr(kvx, dev, 64)
    f = mgr.d2h(list(range(64)), list(range(64)))
    f.PollError()
    f.Await()
    assert f.IsReady()
    # A producer kernel on torch's stream, then an offload ordered after it.
    s = torch.cuda.current_stream()
    for l in range(4):
        dev[l][0].add_(1)
    f = mgr.d2h([10, 20], [0, 1], stream=s)
    f.Await()
    for l in range(4):
        want = (host[l][0][[10, 20]].astype(np.uint16) + 1).astype(np.uint8)
        assert np.array_equal(mgr.host_view(l).reshape(64, 65536)[:2], want)
    # A consumer on torch's stream waits for a reload without host blocking.
    f = mgr.h2d([0, 1], [30, 31])
    f.wait_on_stream(s)
    sums = [dev[l][0][30:32].to(torch.int64).sum() for l in range(4)]
    torch.cuda.synchronize()
    for l in range(4):
        want = (host[l][0][[10, 20]].astype(np.uint16) + 1).astype(np.uint8)
        assert int(sums[l].item()) == int(want.astype(np.int64).sum())
    mgr.wait_for_pending_work()
    mgr.close()


@pytest.mark.parametrize("host_alloc", ["pinned", "malloc"])
def test_concurrent_disjoint_blocks(kvx, cuda, host_alloc):
    """tpu_sync/frameworks/jax/kv_cache_manager_test.py:520-594: one thread
    loops H2D/D2H of blocks 0:4 while another moves 4:8 once; both ranges
    keep their values (malloc: both threads share the bounce lanes)."""
    shape = (8, 128 * 8 * 8 * 128 * 4 // 8)
    init = np.zeros(shape, np.float32)
    init[0:4] = 1.0
    init[4:8] = 2.0
    raw = init.view(np.uint8).reshape(8, -1)
    pools = [torch.from_numpy(raw.copy()).to(cuda) for _ in range(2)]
    mgr = kvx.KVCacheManager(pools, host_blocks_to_allocate=8, host_alloc=host_alloc)
    mgr.d2h().Await()
    stop = threading.Event()
    errors = []

    def loop():
        try:
            while not stop.is_set():
                mgr.h2d([0], [0], [4]).Await()
                mgr.d2h([0], [0], [4]).Await()
        except Exception as e:  # noqa: BLE001
            errors.append(e)

    t1 = threading.Thread(target=loop)
    t1.start()
    mgr.h2d([4], [4], [4]).Await()
    stop.set()
    t1.join()
    assert not errors
    for p in pools:
        got = dev_np(p).view(np.float32).reshape(8, -1)
        assert (got[0:4] == 1.0).all() and (got[4:8] == 2.0).all()
    mgr.close()


@pytest.mark.parametrize("mode", MODES)
def test_llama3_8b_pool_full_size_round_trip(kvx, cuda, mode):
    """32 layers x (K, V) x 16384 blocks x 16 tokens x 8 heads x 128 dim bf16
    (32 GiB pool): offload 512 random blocks to pinned host, reload into 512
    random free slots; bit-exact through size-independent checks (every
    reloaded block equals its source; every other block unchanged, through a
    weighted 64-bit word sum per (storage, block), which also catches two
    blocks swapped or errors that cancel in a plain sum)."""
    S, P, bb, n = 64, 16384, 32768, 512
    gen = torch.Generator(device=cuda).manual_seed(0)
    pools = [torch.randint(-2**31, 2**31 - 1, (P, bb // 4), dtype=torch.int32,
                           device=cuda, generator=gen).view(torch.uint8)
             for _ in range(S)]
    rng = np.random.default_rng(1)
    perm = rng.permutation(P)
    ids, free = perm[:n], perm[n:2 * n]
    ids_t = torch.from_numpy(ids).to(cuda)
    free_t = torch.from_numpy(free).to(cuda)
    orig = [p.index_select(0, ids_t).clone() for p in pools]
    keep = torch.ones(P, dtype=torch.bool, device=cuda)
    keep[free_t] = False
    # Fixed random odd weights per word position: a block's fingerprint is
    # the wrapping sum of its int64 words times their weights.
    weights = torch.randint(-(1 << 62), 1 << 62, (bb // 8,), dtype=torch.int64, device=cuda,
                            generator=gen) | 1

    def fingerprints(p):
        return (p.view(torch.int64) * weights).sum(dim=1)

    before = [fingerprints(p) for p in pools]
    mgr = kvx.KVCacheManager(pools, host_blocks_to_allocate=n, transfer_mode=mode)
    print(f"{mode}: offload 512 blocks x 64 storages", flush=True)
    mgr.d2h(ids.tolist(), list(range(n))).Await()
    print("reload into 512 free slots", flush=True)
    mgr.h2d(list(range(n)), free.tolist()).Await()
    for s in range(S):
        assert torch.equal(pools[s].index_select(0, free_t), orig[s]), s
        assert torch.equal(fingerprints(pools[s])[keep], before[s][keep]), s
    stats = mgr.engine_stats()
    key = "staged_copies" if mode == "staged" else "zero_copy_copies"
    assert stats[key] == 2 and stats["kernel_launches"] >= 2
    mgr.close()


@pytest.mark.parametrize("threads,alloc", [(1, "malloc"), (0, "shm")])
def test_bounce_lanes_overlap_and_drain(kvx, oracle, cuda, threads, alloc):
    """Pageable mirror (malloc, or a /dev/shm segment): 8 offloads and 8
    reloads of disjoint host ranges are issued without waiting (the two lanes
    run them concurrently, each in submission order); wait_for_pending_work
    drains both lanes, then device and host equal the oracle's. threads=1:
    the issuing thread alone copies."""
    rng = np.random.default_rng(41 + threads)
    layers, blocks, bb, hb = 4, 64, 16384, 64
    host, dev = dev_pools(rng, cuda, layers, 1, blocks, bb)
    tier = {}
    if alloc == "shm":
        tier = {"shm_key": f"kvx_test_bounce_{os.getpid()}"}
    mgr = make_mgr(kvx, dev, hb, host_alloc=alloc, staging_chunk_bytes=1 << 18,
                   staging_chunks=3, direct_min_bytes=1 << 40, host_copy_threads=threads,
                   **tier)
    mir = Mirror(host, hb)
    # Host blocks 32..63 hold data to reload; 0..31 receive offloads.
    for l in range(layers):
        fill = rng.integers(0, 256, 32 * bb, dtype=np.uint8)
        mgr.host_view(l)[32 * bb:] = fill
        mir.host[l][32 * bb:] = fill
    futs = []
    for i in range(8):
        src = [int(x) for x in rng.choice(32, 4, replace=False)]
        print(f"threads={threads} round {i} offload {src} -> {4 * i}..", flush=True)
        futs.append(mgr.d2h(src, [4 * i + k for k in range(4)], [1] * 4))
        assert mir.transfer(True, src, [4 * i + k for k in range(4)], [1] * 4) == 0
        hsrc = [32 + int(x) for x in rng.choice(32, 4, replace=False)]
        dst = [32 + 4 * i + k for k in range(4)]
        futs.append(mgr.h2d(hsrc, dst, [1] * 4))
        assert mir.transfer(False, hsrc, dst, [1] * 4) == 0
    mgr.wait_for_pending_work()
    for f in futs:
        assert f.is_ready()
        f.Await()
    mir.check(mgr, dev)
    assert mgr.engine_stats()["bounce_copies"] == 16
    mgr.close()
    if tier:
        for name in os.listdir("/dev/shm"):
            if name.startswith(tier["shm_key"]):
                os.unlink(os.path.join("/dev/shm", name))


def test_auto_duplex_short_runs_take_the_lanes(kvx, oracle, cuda):
    """Auto mode on a pinned mirror with single-block host runs: a lone copy
    goes zero-copy; a save issued while a load is in flight goes through the
    lanes, and so do both copies of the next load + save inside the duplex
    window; after an idle pause longer than the window a lone copy is
    zero-copy again. Every step's bytes against the oracle."""
    import time
    rng = np.random.default_rng(77)
    layers, blocks, hb, bb, n = 4, 512, 1024, 32768, 256
    host, dev = dev_pools(rng, cuda, layers, 1, blocks, bb)
    mgr = make_mgr(kvx, dev, hb, staging_chunk_bytes=1 << 20, staging_chunks=4,
                   host_copy_threads=3)
    mir = Mirror(host, hb)

    def pick():
        d = rng.permutation(blocks)
        h = rng.permutation(hb)
        return d[:n].tolist(), d[n:2 * n].tolist(), h[:n].tolist(), h[n:2 * n].tolist()

    def kinds():
        st = mgr.engine_stats()
        return st["zero_copy_copies"], st["bounce_copies"]

    ones = [1] * n
    d0, _, h0, _ = pick()
    print("lone offload", flush=True)
    mgr.d2h(d0, h0, ones).Await()
    assert mir.transfer(True, d0, h0, ones) == 0
    assert kinds() == (1, 0)
    # A load of 32 MiB keeps its kernel busy while the save is issued.
    for step in range(2):
        d_load, d_save, h_load, h_save = pick()
        h_load = h0 if step == 0 else h_load  # the first load reads real bytes
        print(f"load + save {step}", flush=True)
        f1 = mgr.h2d(h_load, d_load, ones)
        f2 = mgr.d2h(d_save, h_save, ones)
        f1.Await()
        f2.Await()
        assert mir.transfer(False, h_load, d_load, ones) == 0
        assert mir.transfer(True, d_save, h_save, ones) == 0
        mir.check(mgr, dev)
    zc, lanes = kinds()
    # The first load was lone (zero-copy); its save and the second pair rode the lanes.
    assert zc == 2 and lanes == 3, (zc, lanes)
    time.sleep(0.4)
    d1, _, h1, _ = pick()
    print("lone offload after a pause", flush=True)
    mgr.d2h(d1, h1, ones).Await()
    assert mir.transfer(True, d1, h1, ones) == 0
    mir.check(mgr, dev)
    assert kinds() == (3, 3)
    mgr.close()


def test_auto_mid_runs_alone_go_zero_copy(kvx, oracle, cuda):
    """Auto mode on a pinned mirror with runs long enough to move directly
    (at least 4 MiB) that average under 32 MiB: one zero-copy launch while
    the other direction is idle, one DMA per run while a copy of the other
    direction is in flight, and one DMA per run for runs of 32 MiB. Every
    step's bytes against the oracle."""
    import time
    rng = np.random.default_rng(78)
    layers, blocks, hb, bb = 4, 96, 96, 1 << 20
    host, dev = dev_pools(rng, cuda, layers, 1, blocks, bb)
    mgr = make_mgr(kvx, dev, hb)
    mir = Mirror(host, hb)

    def counts():
        st = mgr.engine_stats()
        return st["zero_copy_copies"], st["direct_copies"], st["memcpy_calls"]

    print("lone offload, 8 MiB runs", flush=True)
    mgr.d2h([0, 40], [0, 8], [8, 8]).Await()
    assert mir.transfer(True, [0, 40], [0, 8], [8, 8]) == 0
    mir.check(mgr, dev)
    assert counts() == (1, 0, 0)
    print("lone offload, one 32 MiB run", flush=True)
    mgr.d2h([48], [32], [32]).Await()
    assert mir.transfer(True, [48], [32], [32]) == 0
    mir.check(mgr, dev)
    assert counts() == (1, 1, layers)
    # A load of 128 MiB (16 MiB runs, zero-copy: it is alone) keeps its
    # kernel busy while an offload of 8 MiB runs is issued behind it; the
    # two touch disjoint device and host blocks.
    print("load of 16 MiB runs, then an offload of 8 MiB runs", flush=True)
    f1 = mgr.h2d([0, 16], [16, 64], [16, 16])
    f2 = mgr.d2h([0, 40], [64, 72], [8, 8])
    f1.Await()
    f2.Await()
    assert mir.transfer(False, [0, 16], [16, 64], [16, 16]) == 0
    assert mir.transfer(True, [0, 40], [64, 72], [8, 8]) == 0
    mir.check(mgr, dev)
    assert counts() == (2, 2, 3 * layers), counts()
    time.sleep(0.4)
    print("lone reload after a pause", flush=True)
    mgr.h2d([64], [88], [8]).Await()
    assert mir.transfer(False, [64], [88], [8]) == 0
    mir.check(mgr, dev)
    assert counts() == (3, 2, 3 * layers), counts()
    mgr.close()


def test_zero_copy_needs_pinned_host(kvx, cuda):
    t = torch.zeros(4, 256, dtype=torch.uint8, device=cuda)
    with pytest.raises(kvx.KvxError) as e:
        kvx.KVCacheManager([t], host_blocks_to_allocate=4, host_alloc="malloc",
                           transfer_mode="zero_copy")
    assert e.value.code == 3
    # A pageable mirror falls back to the staged path in auto mode.
    mgr = kvx.KVCacheManager([t], host_blocks_to_allocate=4, host_alloc="malloc")
    t[1].fill_(7)
    mgr.d2h([1], [2]).Await()
    assert (mgr.host_view(0).reshape(4, 256)[2] == 7).all()
    assert mgr.engine_stats()["staged_copies"] == 1
    mgr.close()


def test_auto_mode_picks_by_host_fragmentation(kvx, cuda):
    """Auto mode stages copies whose host runs average at least 4 MiB per
    storage and moves shorter ones with the zero-copy kernel; both are
    bit-exact."""
    rng = np.random.default_rng(31)
    bb = 65536
    host, dev = dev_pools(rng, cuda, 2, 1, 256, bb)
    mgr = make_mgr(kvx, dev, 256)
    ids = rng.choice(256, size=64, replace=False).tolist()
    mgr.d2h(ids, list(range(64))).Await()  # one 4 MiB run per storage
    assert mgr.engine_stats()["staged_copies"] == 1
    mgr.d2h(ids[:32], list(range(64, 96))).Await()  # one 2 MiB run
    assert mgr.engine_stats()["zero_copy_copies"] == 1
    hids = (96 + rng.choice(160, size=64, replace=False)).tolist()  # clear of 0..95
    mgr.d2h(ids, hids).Await()
    assert mgr.engine_stats()["zero_copy_copies"] == 2
    for l in range(2):
        hv = mgr.host_view(l).reshape(256, bb)
        assert np.array_equal(hv[64:96], host[l][0][ids[:32]])
        assert np.array_equal(hv[:64], host[l][0][ids])
        assert np.array_equal(hv[hids], host[l][0][ids])
    mgr.close()


@pytest.mark.parametrize("host_alloc", ["pinned", "malloc"])
def test_empty_and_zero_size_copies_move_nothing(kvx, cuda, host_alloc):
    """Zero-size runs, empty id lists and empty entry lists are no-ops that
    return completed futures, on every path (pinned and pageable mirrors)."""
    rng = np.random.default_rng(21)
    host, dev = dev_pools(rng, cuda, 2, 1, 16, 4096)
    mgr = make_mgr(kvx, dev, 16, host_alloc=host_alloc)
    before = [d[0].clone() for d in dev]
    for f in (mgr.d2h([3], [4], [0]), mgr.h2d([4], [3], [0]),
              mgr.d2h([1, 2], [5, 6], [0, 0])):
        f.Await()
        assert f.IsReady()
    stg = torch.empty(0, dtype=torch.uint8, device=cuda)
    mgr.gather([], stg).Await()
    mgr.scatter([], stg).Await()
    mgr.d2h_pool_blocks(0, []).Await()
    mgr.h2d_pool_blocks(1, []).Await()
    kvx.copy_strided([], device=0).Await()
    mgr.wait_for_pending_work()
    for l in range(2):
        assert not mgr.host_view(l).any()
        assert torch.equal(dev[l][0], before[l])
    mgr.close()


def test_on_ready_callbacks(kvx, cuda):
    """PjRtCopyFuture::OnReady (raw_transfer_core.h:491-530): each callback
    runs once, after its copy's bytes landed, with the final status code; on
    a done future before on_ready returns; a failed (queued, invalid) copy
    reports its code."""
    rng = np.random.default_rng(23)
    host, dev = dev_pools(rng, cuda, 4, 1, 64, 65536)
    mgr = make_mgr(kvx, dev, 64)
    got = {}
    done = threading.Event()

    def record(k):
        def cb(code):
            # The copy's bytes are in the host mirror when the callback runs.
            ok = np.array_equal(mgr.host_view(0).reshape(64, 65536)[k], host[0][0][k])
            got[k] = (code, ok)
            if len(got) == 16:
                done.set()
        return cb

    for k in range(16):
        mgr.d2h([k], [k], [1]).on_ready(record(k))
    assert done.wait(60)
    assert all(v == (0, True) for v in got.values()), got
    f = mgr.d2h([20], [20], [1])
    f.Await()
    sync_codes = []
    f.on_ready(sync_codes.append)  # already done: called before returning
    assert sync_codes == [0]
    mgr.close()
    qm = make_mgr(kvx, dev, 64, dispatch="queued")
    codes = []
    fired = threading.Event()
    bad = qm.d2h([70], [0], [1])  # device range error, reported through the future

    def on_bad(code):
        codes.append(code)
        fired.set()

    bad.on_ready(on_bad)
    assert fired.wait(60)
    assert codes == [3]
    qm.close()


@pytest.mark.parametrize("bb", [65536, 131072, 100000, 70004, 262144 + 2])
def test_blocks_split_over_workgroups_match_oracle(kvx, oracle, cuda, bb):
    """Blocks larger than one workgroup's pass (32 KiB at 16-byte vectors,
    8 KiB at 4-byte, 2 KiB at 1-byte) go to consecutive workgroups, a pass
    each, the last one short when the block is not a whole number of passes:
    device gather and scatter (storage pairs / all storages), staged offload
    and reload through small staging chunks, and zero-copy (whose capped grid
    keeps one workgroup per block), all against the oracle."""
    rng = np.random.default_rng(bb % 1000)
    layers, P, n = 2, 24, 9
    host, dev = dev_pools(rng, cuda, layers, 1, P, bb)
    for mode in ("staged", "zero_copy"):
        mgr = make_mgr(kvx, dev, 16, transfer_mode=mode, staging_chunk_bytes=3 * bb,
                       staging_chunks=2)
        ids = rng.choice(P, n, replace=False).tolist()
        if mode == "staged":
            stg = torch.zeros(layers * n * bb, dtype=torch.uint8, device=cuda)
            mgr.gather(ids, stg).Await()
            got = dev_np(stg).reshape(layers, n, bb)
            for l in range(layers):
                assert np.array_equal(got[l], dev_np(dev[l][0])[ids]), (l, mode)
            dst = [i for i in range(P) if i not in ids][:n]
            mgr.scatter(dst, stg).Await()
            for l in range(layers):
                assert np.array_equal(dev_np(dev[l][0])[dst], got[l]), (l, mode)
        cur = [dev_np(dev[l][0]).reshape(-1).copy() for l in range(layers)]
        hostm = [np.zeros(16 * bb, np.uint8) for _ in range(layers)]
        slot = rng.permutation(16)[:n].tolist()
        mgr.d2h(ids, slot).Await()
        assert oracle.transfer(True, cur, hostm, [bb] * layers, [c.nbytes for c in cur],
                               ids, slot, [1] * n) == 0
        for l in range(layers):
            assert np.array_equal(mgr.host_view(l), hostm[l]), (l, mode)
        back = rng.choice(P, n, replace=False).tolist()
        mgr.h2d(slot, back).Await()
        assert oracle.transfer(False, cur, hostm, [bb] * layers, [c.nbytes for c in cur],
                               slot, back, [1] * n) == 0
        for l in range(layers):
            assert np.array_equal(dev_np(dev[l][0]).reshape(-1), cur[l]), (l, mode)
        mgr.close()


@pytest.mark.parametrize("cap", [0, -1, 1, 8])
@pytest.mark.parametrize("layers", [3, 4])
def test_gather_scatter_every_block_of_the_pool(kvx, cuda, layers, cap):
    """Maximum size for a pool: all P block ids, permuted, gathered into one
    staging buffer (storage pairs when the storage count is even, storage-
    major when odd) and scattered back under the inverse permutation into a
    zeroed pool: the pool must come back byte for byte. `cap` is the gather's
    workgroups-per-CU limit (0: the default, -1: none)."""
    rng = np.random.default_rng(24 + layers)
    P, bb = 512, 16384
    host, dev = dev_pools(rng, cuda, layers, 1, P, bb)
    mgr = make_mgr(kvx, dev, 4, gather_workgroups_per_cu=cap)
    perm = rng.permutation(P)
    stg = torch.empty(layers * P * bb, dtype=torch.uint8, device=cuda)
    mgr.gather(perm.tolist(), stg).Await()
    got = dev_np(stg).reshape(layers, P, bb)
    for l in range(layers):
        assert np.array_equal(got[l], host[l][0][perm]), l
    fresh = [[torch.zeros(P, bb, dtype=torch.uint8, device=cuda)] for _ in range(layers)]
    mgr2 = make_mgr(kvx, fresh, 4)
    mgr2.scatter(perm.tolist(), stg).Await()
    for l in range(layers):
        assert np.array_equal(dev_np(fresh[l][0]), host[l][0]), l
    mgr.close()
    mgr2.close()
