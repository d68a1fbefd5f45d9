"""GPU: pool-block copies (D2hPoolBlocks / H2dPoolBlocks,
kv_cache_manager_base.cc:1801-1872) move exactly the live bytes named by the
oracle's copy extents (oracle/pool_layout.py) between HBM and the host
mirror, at the same byte offsets on both sides, and nothing else: padding
bytes keep a sentinel on the receiving side. Covers the strided-copy kernel
path (pinned mirror, short extents), the bounce lane (malloc mirror: live
bytes packed into staging chunks), the DMA path (extents of at least
direct_min_bytes, or a malloc mirror left to the runtime), shard selection,
the implicit opaque pools and host-mirror growth on registration."""
import numpy as np
import pytest

from oracle import pool_layout as O

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

SENTINEL = 0xAB


def u8(t):
    torch.cuda.synchronize()
    return t.detach().cpu().contiguous().view(torch.uint8).numpy().reshape(-1)


def spec(kvx, pool, storage_index=0):
    P = kvx.pool_layout
    return P.PoolSpec(pool["tag"], storage_index, pool["base"], pool["block_stride"],
                      pool["num_blocks"], tuple(P.RegionSpec(*r) for r in pool["regions"]),
                      "")


def covered(pool, ids, size):
    mask = np.zeros(size, bool)
    for off, n in O.copy_extents(pool, ids):
        mask[off:off + n] = True
    return mask


def device_storages(cuda, rng, num_shards, nbytes, major):
    shards = []
    for _ in range(num_shards):
        t = torch.from_numpy(rng.integers(0, 256, nbytes, dtype=np.uint8)).to(cuda)
        shards.append(t.view(major, nbytes // major))
    return shards


# FA-like pool: 4 head groups per block, each 64 tokens x (K 256 B, V 256 B)
# packed, groups 70 KiB apart inside a 320 KiB block stride; plus a sparse
# pool whose units leave 48 B holes.
FA = {"tag": "fa", "base": 4096, "block_stride": 327680, "num_blocks": 24,
      "regions": [("fa", g * 71680, 512, 256, 64, 2) for g in range(4)]}
SPARSE = {"tag": "sparse", "base": 0, "block_stride": 4096, "num_blocks": 96,
          "regions": [("k", 0, 80, 32, 40, 1), ("s", 3216, 16, 8, 4, 1)]}


@pytest.mark.parametrize("host_alloc", ["pinned", "malloc", "malloc_runtime", "pinned_lanes"])
@pytest.mark.parametrize("pool", [FA, SPARSE], ids=["fa", "sparse"])
def test_pool_copies_move_exactly_the_live_bytes(kvx, cuda, host_alloc, pool):
    """pinned: the strided kernel reads/writes the mapped mirror; malloc: the
    bounce lane (staging chunks of 48 KiB, so extents split across chunks);
    malloc_runtime: one pageable hipMemcpyAsync per (storage, extent);
    pinned_lanes: a pinned mirror in transfer_mode "lanes" (the bounce lane)."""
    rng = np.random.default_rng(11)
    nbytes = O.storage_extent_end(pool) + 1000
    nbytes += (-nbytes) % pool["block_stride"]
    major = nbytes // pool["block_stride"]
    shards = device_storages(cuda, rng, 2, nbytes, major)
    kw = {"host_alloc": host_alloc}
    if host_alloc == "malloc":
        kw.update(staging_chunk_bytes=48 << 10, staging_chunks=2)
    elif host_alloc == "pinned_lanes":
        kw.update(host_alloc="pinned", transfer_mode="lanes", staging_chunk_bytes=48 << 10,
                  staging_chunks=2)
    elif host_alloc == "malloc_runtime":
        kw.update(host_alloc="malloc", host_copy_threads=-1)
    mgr = kvx.KVCacheManager([shards], host_blocks_to_allocate=major, **kw)
    mgr.register_pools([spec(kvx, pool)])
    hv = [mgr.host_view(0, s) for s in range(2)]
    for h in hv:
        h[:] = SENTINEL
    ids = [int(x) for x in rng.choice(pool["num_blocks"], 9, replace=False)]
    before = mgr.engine_stats()
    mgr.d2h_pool_blocks(0, ids).Await()
    after = mgr.engine_stats()
    if host_alloc == "pinned":
        assert after["extent_kernel_copies"] == before["extent_kernel_copies"] + 1
    elif host_alloc in ("malloc", "pinned_lanes"):
        # Packed into staging chunks, one DMA per chunk through a bounce lane.
        assert after["bounce_copies"] == before["bounce_copies"] + 1
    else:
        assert after["memcpy_calls"] - before["memcpy_calls"] == \
            2 * len(O.copy_extents(pool, ids))
    mask = covered(pool, ids, nbytes)
    for s in range(2):
        dev = u8(shards[s])
        assert np.array_equal(hv[s][:nbytes][mask], dev[mask])
        assert np.all(hv[s][:nbytes][~mask] == SENTINEL)
    # Reload into shard 1 only: new host bytes, device padding untouched.
    dev_before = [u8(t).copy() for t in shards]
    for h in hv:
        h[:nbytes] = rng.integers(0, 256, nbytes, dtype=np.uint8)
    ids2 = ids[:5]
    mgr.h2d_pool_blocks(0, ids2, shard_idx=1).Await()
    mask2 = covered(pool, ids2, nbytes)
    got1 = u8(shards[1])
    assert np.array_equal(got1[mask2], hv[1][:nbytes][mask2])
    assert np.array_equal(got1[~mask2], dev_before[1][~mask2])
    assert np.array_equal(u8(shards[0]), dev_before[0])
    mgr.close()


def test_large_extents_use_dma(kvx, cuda):
    """Extents of at least direct_min_bytes go through hipMemcpyAsync even with
    a pinned mirror."""
    rng = np.random.default_rng(12)
    block = 1 << 20
    shards = device_storages(cuda, rng, 1, 16 * block, 16)
    mgr = kvx.KVCacheManager([shards], host_blocks_to_allocate=16, host_alloc="pinned",
                             direct_min_bytes=block)
    pool = {"tag": "dense", "base": 0, "block_stride": block, "num_blocks": 16,
            "regions": [("block", 0, block, block, 1, 1)]}
    mgr.register_pools([spec(kvx, pool)])
    before = mgr.engine_stats()
    mgr.d2h_pool_blocks(0, [3, 4, 9]).Await()
    after = mgr.engine_stats()
    assert after["extent_kernel_copies"] == before["extent_kernel_copies"]
    assert after["memcpy_calls"] - before["memcpy_calls"] == 2  # 3-4 coalesced, 9
    h = mgr.host_view(0)
    dev = u8(shards[0])
    for b in (3, 4, 9):
        assert np.array_equal(h[b * block:(b + 1) * block], dev[b * block:(b + 1) * block])
    mgr.close()


def test_implicit_opaque_pools_copy_whole_blocks(kvx, cuda):
    rng = np.random.default_rng(13)
    layers = [device_storages(cuda, rng, 1, 64 * 2048, 64) for _ in range(3)]
    mgr = kvx.KVCacheManager(layers, host_blocks_to_allocate=16)
    assert mgr.num_pools() == 3 and not mgr.has_explicit_pools()
    assert mgr.pool_ids_with_tag("opaque") == [0, 1, 2]
    assert mgr.pool_spec(2)["num_blocks"] == 16
    mgr.d2h_pool_blocks(1, [0, 5, 6, 15]).Await()
    h = mgr.host_view(1)
    dev = u8(layers[1][0])
    for b in (0, 5, 6, 15):
        assert np.array_equal(h[b * 2048:(b + 1) * 2048], dev[b * 2048:(b + 1) * 2048])
    assert not h[2048:5 * 2048].any()
    with pytest.raises(kvx.KvxError, match="out of range"):
        mgr.d2h_pool_blocks(1, [16])
    with pytest.raises(kvx.KvxError, match="pool index 3 out of range"):
        mgr.d2h_pool_blocks(3, [0])
    mgr.close()


def test_register_pools_grows_host_mirror(kvx, cuda):
    """kv_cache_manager_test.cc:198-225 on a device-backed manager: the mirror
    (1 block of 64 B) grows to the pool's 4 blocks and keeps its bytes."""
    rng = np.random.default_rng(14)
    shards = device_storages(cuda, rng, 1, 256, 4)
    mgr = kvx.KVCacheManager([shards], host_blocks_to_allocate=1)
    h = mgr.host_view(0)
    assert h.size == 64
    h[:] = np.arange(64, dtype=np.uint8)
    pool = {"tag": "kind_a", "base": 0, "block_stride": 64, "num_blocks": 4,
            "regions": [("block", 0, 64, 64, 1, 1)]}
    mgr.register_pools([spec(kvx, pool)])
    h = mgr.host_view(0)
    assert h.size >= 256
    assert np.array_equal(h[:64], np.arange(64, dtype=np.uint8))
    assert mgr.get_block_ref(0, 3)["ptr"] == \
        kvx._capi.load().kvx_manager_host_ptr(mgr._h, 0, 0) + 3 * 64
    mgr.d2h_pool_blocks(0, [3]).Await()
    assert np.array_equal(mgr.host_view(0)[192:256], u8(shards[0])[192:256])
    # A pool past the device storage is refused (the device size bounds it).
    bad = dict(pool, num_blocks=5)
    with pytest.raises(kvx.KvxError, match="exceeds storage bytes"):
        mgr.register_pools([spec(kvx, bad)])
    mgr.close()
