"""Block-pool geometry and the manager's pool table on the CPU.

The oracle (oracle/pool_layout.py) is pinned by the reference's known answers
(tests/golden/pool_cases.json) and by brute force over a byte mask of live
bytes; the product (the library's restatement, through the C-ABI) must then
agree with the oracle on the goldens and on random pools, including errors.
Manager cases follow kv_cache_manager_test.cc:120-325 and
kv_cache_manager_host_test.py:25-135 on host-only managers."""
import json
import os

import numpy as np
import pytest

from oracle import pool_layout as O

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "pool_cases.json")))


# -- helpers -----------------------------------------------------------------
def to_spec(kvx, pool, storage_index=0):
    P = kvx.pool_layout
    regions = tuple(P.RegionSpec(*r) for r in pool["regions"])
    return P.PoolSpec(pool.get("tag", "p"), storage_index, pool["base"], pool["block_stride"],
                      pool["num_blocks"], regions, pool.get("dtype_tag", ""))


def mgr_pool(kvx, kind, tag, storage, base, stride, nblocks):
    """DensePool / StridedPool of kv_cache_manager_test.cc:74-116."""
    P = kvx.pool_layout
    if kind == "dense":
        reg = P.RegionSpec("block", 0, stride, stride, 1, 1)
    else:
        reg = P.RegionSpec("payload", 0, 64, 32, 2, 1)
    return P.PoolSpec(tag, storage, base, stride, nblocks, (reg,), "dtype_a")


def live_mask(pool, block_ids, size):
    """Brute force: every live byte of every block id, marked in a mask."""
    m = np.zeros(size, np.int32)
    for b in block_ids:
        base = pool["base"] + b * pool["block_stride"]
        for _, off, stride, unit, num, ups in pool["regions"]:
            for u in range(num):
                s = base + off + u * stride
                m[s:s + unit * ups] += 1
    return m


def runs(mask):
    out, i, n = [], 0, len(mask)
    while i < n:
        if mask[i]:
            j = i
            while j < n and mask[j]:
                j += 1
            out.append((i, j - i))
            i = j
        else:
            i += 1
    return out


def random_pool(rng, allow_overlap=False):
    stride_b = int(rng.integers(64, 600))
    regions = []
    for k in range(int(rng.integers(1, 4))):
        unit = int(rng.integers(1, 24))
        ups = int(rng.integers(1, 3))
        num = int(rng.integers(0, 6))
        stride = unit * ups + int(rng.integers(0, 3)) * int(rng.integers(0, 20))
        off = int(rng.integers(0, stride_b // 2))
        if num > 1 and stride == 0:
            stride = unit * ups
        end = off + max(num - 1, 0) * stride + unit * ups
        if num > 0 and end > stride_b:
            continue
        regions.append((f"r{k}", off, stride, unit, num, ups))
    if not regions:
        regions = [("r", 0, stride_b, stride_b, 1, 1)]
    return {"tag": "t", "base": int(rng.integers(0, 100)), "block_stride": stride_b,
            "num_blocks": int(rng.integers(1, 8)), "regions": regions}


# -- oracle pinned by the reference's known answers ---------------------------
def test_oracle_known_answers():
    g = GOLD["region_live_bytes"]
    r = g["region"]
    assert r[3] * r[4] * r[5] == g["live_bytes"]
    assert O.region_extent_end(r) == g["extent_end"]
    assert O.storage_extent_end(GOLD["pool_storage"]["pool"]) == GOLD["pool_storage"]["extent_end"]
    assert O.storage_extent_end(GOLD["gdn_ssm"]["pool"]) == GOLD["gdn_ssm"]["extent_end"]
    c = GOLD["cover_range"]
    assert O.regions_cover_range(c["regions"], *c["true"])
    assert not O.regions_cover_range(c["regions"], *c["false"])
    for k in ("extents_basic", "extents_padding", "extents_fa"):
        g = GOLD[k]
        assert O.copy_extents(g["pool"], g["ids"]) == [tuple(e) for e in g["extents"]], k
    assert O.live_segments(GOLD["segments_strided"]["pool"]) == [
        tuple(s) for s in GOLD["segments_strided"]["segments"]]
    g = GOLD["segments_abutting"]
    assert O.live_segments(g["pool"]) == [tuple(s) for s in g["segments"]]
    bad = dict(g["pool"], regions=[g["pool"]["regions"][0],
                                   ["b", g["overlap_b_offset"]] + g["pool"]["regions"][1][2:]])
    with pytest.raises(O.PoolError, match=g["fail_substr"]):
        O.live_segments(bad)
    g = GOLD["physical_to_logical"]
    segs = O.live_segments(g["pool"])
    assert O.physical_to_logical(segs, g["ok"][0], g["ok"][1]) == (g["ok"][2], g["ok"][3])
    with pytest.raises(O.PoolError, match=g["fail_substr"]):
        O.physical_to_logical(segs, *g["fail"])


def test_oracle_matches_brute_force():
    """Extents = runs of the live-byte mask; segments = runs of one block's
    mask with compact offsets; overlap iff some byte is live twice; a
    compact-live copy splits exactly where either side's physical bytes stop
    being consecutive."""
    rng = np.random.default_rng(0)
    checked = 0
    for _ in range(400):
        pool = random_pool(rng)
        size = O.storage_extent_end(pool) + pool["block_stride"]
        one = dict(pool, base=0, num_blocks=1)
        mask1 = live_mask(one, [0], pool["block_stride"])
        if mask1.max() > 1:
            with pytest.raises(O.PoolError):
                O.live_segments(pool)
            continue
        ids = sorted(set(int(x) for x in rng.integers(0, pool["num_blocks"], 5)))
        m = live_mask(pool, ids, size)
        assert O.copy_extents(pool, ids) == runs(m > 0)
        segs = O.live_segments(pool)
        want, logical = [], 0
        for s, n in runs(mask1 > 0):
            want.append((logical, s, n))
            logical += n
        assert segs == want
        # Compact-live translation between this pool and another one.
        other = random_pool(rng)
        try:
            osegs = O.live_segments(other)
        except O.PoolError:
            continue
        ls, ld = sum(s[2] for s in segs), sum(s[2] for s in osegs)
        if min(ls, ld) < 2:
            continue
        so, do = int(rng.integers(0, ls - 1)), int(rng.integers(0, ld - 1))
        size_c = int(rng.integers(1, min(ls - so, ld - do) + 1))
        sp = [p for lo, po, sz in segs for p in range(po, po + sz)][so:so + size_c]
        dp = [p for lo, po, sz in osegs for p in range(po, po + sz)][do:do + size_c]
        chunks, i = [], 0
        while i < size_c:
            j = i + 1
            while j < size_c and sp[j] == sp[j - 1] + 1 and dp[j] == dp[j - 1] + 1:
                j += 1
            chunks.append((sp[i], dp[i], j - i))
            i = j
        assert O.translate_live_copy(segs, osegs, so, do, size_c) == chunks
        checked += 1
    assert checked > 100


def test_oracle_cover_range_brute_force():
    rng = np.random.default_rng(1)
    for _ in range(300):
        pool = random_pool(rng)
        n = pool["block_stride"]
        m = live_mask(dict(pool, base=0, num_blocks=1), [0], n) > 0
        a = int(rng.integers(0, n))
        b = int(rng.integers(a, n + 1))
        assert O.regions_cover_range(pool["regions"], a, b) == bool(m[a:b].all())


# -- product against the oracle -------------------------------------------------
def test_product_known_answers(kvx):
    P = kvx.pool_layout
    g = GOLD["region_live_bytes"]
    r = P.RegionSpec(*g["region"])
    assert r.live_bytes == g["live_bytes"] and r.extent_end_bytes == g["extent_end"]
    r.validate(g["validate_ok_slot"])
    with pytest.raises(ValueError, match=g["fail_substr"]):
        r.validate(g["validate_fail_slot"])
    g = GOLD["pool_storage"]
    pool = to_spec(kvx, g["pool"])
    P.validate_native(pool, g["ok_storage"])
    P.validate_native(pool, g["ok_exact"])
    assert P.storage_extent_end_native(pool) == g["extent_end"]
    with pytest.raises(kvx.KvxError, match=g["fail_substr"]) as e:
        P.validate_native(pool, g["fail_storage"])
    assert e.value.code == 3
    neg = P.PoolSpec("pool0", 0, 0, 1000, 10, (P.RegionSpec("key", -1, 100, 10, 5, 2),))
    with pytest.raises(kvx.KvxError, match="offset_bytes must be >= 0"):
        P.validate_native(neg, 10000)
    g = GOLD["gdn_ssm"]
    pool = to_spec(kvx, g["pool"])
    assert P.storage_extent_end_native(pool) == g["extent_end"]
    P.validate_native(pool, g["ok_storage"])
    c = GOLD["cover_range"]
    regs = [P.RegionSpec(*r) for r in c["regions"]]
    assert P.regions_cover_range(regs, *c["true"])
    assert not P.regions_cover_range(regs, *c["false"])
    for k in ("extents_basic", "extents_padding", "extents_fa"):
        g = GOLD[k]
        pool = to_spec(kvx, g["pool"])
        if "ok_storage" in g:
            P.validate_native(pool, g["ok_storage"])
        assert P.compute_pool_block_copy_extents(pool, g["ids"]) == \
            [tuple(e) for e in g["extents"]], k
    g = GOLD["segments_strided"]
    assert P.expand_pool_live_segments(to_spec(kvx, g["pool"])) == \
        [tuple(s) for s in g["segments"]]
    g = GOLD["segments_abutting"]
    assert P.expand_pool_live_segments(to_spec(kvx, g["pool"])) == \
        [tuple(s) for s in g["segments"]]
    bad = dict(g["pool"], regions=[g["pool"]["regions"][0],
                                   ["b", g["overlap_b_offset"]] + g["pool"]["regions"][1][2:]])
    with pytest.raises(kvx.KvxError, match=g["fail_substr"]):
        P.expand_pool_live_segments(to_spec(kvx, bad))
    g = GOLD["physical_to_logical"]
    pool = to_spec(kvx, g["pool"])
    assert P.physical_live_range_to_logical(pool, g["ok"][0], g["ok"][1]) == \
        (g["ok"][2], g["ok"][3])
    with pytest.raises(kvx.KvxError, match=g["fail_substr"]):
        P.physical_live_range_to_logical(pool, *g["fail"])
    with pytest.raises(kvx.KvxError, match="out of range") as e:
        P.compute_pool_block_copy_extents(to_spec(kvx, GOLD["extents_basic"]["pool"]), [10])
    assert e.value.code == 11


def test_product_matches_oracle_random(kvx):
    P = kvx.pool_layout
    rng = np.random.default_rng(2)
    for _ in range(300):
        pool = random_pool(rng)
        spec = to_spec(kvx, pool)
        assert P.storage_extent_end_native(spec) == O.storage_extent_end(pool)
        ids = [int(x) for x in rng.integers(0, pool["num_blocks"], int(rng.integers(0, 7)))]
        assert P.compute_pool_block_copy_extents(spec, ids) == O.copy_extents(pool, ids)
        try:
            want = O.live_segments(pool)
        except O.PoolError:
            with pytest.raises(kvx.KvxError):
                P.expand_pool_live_segments(spec)
            continue
        assert P.expand_pool_live_segments(spec) == want
        n = pool["block_stride"]
        a = int(rng.integers(0, n))
        b = int(rng.integers(a, n + 1))
        assert P.regions_cover_range(spec.regions, a, b) == \
            O.regions_cover_range(pool["regions"], a, b)
        size = int(rng.integers(1, 30))
        off = int(rng.integers(0, n))
        try:
            w = O.physical_to_logical(want, off, size)
        except O.PoolError:
            with pytest.raises(kvx.KvxError):
                P.physical_live_range_to_logical(spec, off, size)
        else:
            assert P.physical_live_range_to_logical(spec, off, size) == w
        other = random_pool(rng)
        try:
            osegs = O.live_segments(other)
        except O.PoolError:
            continue
        ls, ld = sum(s[2] for s in want), sum(s[2] for s in osegs)
        so, do = int(rng.integers(0, ls + 2)), int(rng.integers(0, ld + 2))
        size_c = int(rng.integers(1, 60))
        try:
            w = O.translate_live_copy(want, osegs, so, do, size_c)
        except O.PoolError:
            with pytest.raises(kvx.KvxError):
                P.translate_live_copy(spec, to_spec(kvx, other), so, do, size_c)
        else:
            assert P.translate_live_copy(spec, to_spec(kvx, other), so, do, size_c) == w


def test_product_large_extent_lists(kvx):
    """More extents than the first output buffer holds (the binding grows it)."""
    P = kvx.pool_layout
    pool = {"tag": "big", "base": 0, "block_stride": 4096, "num_blocks": 64,
            "regions": [("u", 0, 64, 16, 64, 1)]}
    ids = list(range(0, 64, 2))
    got = P.compute_pool_block_copy_extents(to_spec(kvx, pool), ids)
    assert got == O.copy_extents(pool, ids) and len(got) == 32 * 64


# -- manager pool table (host-only managers) ------------------------------------
def host_mgr(kvx, num_layers, slice_bytes, host_blocks):
    return kvx.KVCacheManager.create_host_only_for_testing(
        num_layers=num_layers, num_shards=1, slice_byte_size=slice_bytes,
        host_blocks=host_blocks)


def test_register_pools_validates_against_storage(kvx):
    g = GOLD["manager_register"]
    m = host_mgr(kvx, g["num_layers"], g["slice"], g["host_blocks"])
    assert not m.has_explicit_pools()
    assert m.num_pools() == 2  # implicit "opaque" pools, one per storage
    assert m.pool_spec(1)["tag"] == "opaque"
    assert m.pool_spec(1)["num_blocks"] == g["host_blocks"]
    m.register_pools([mgr_pool(kvx, *p) for p in g["ok_pools"]])
    assert m.has_explicit_pools() and m.num_pools() == 3
    with pytest.raises(ValueError, match="storage_index"):
        m.register_pools([mgr_pool(kvx, *g["bad_storage_index"])])
    with pytest.raises(kvx.KvxError, match="exceeds storage bytes") as e:
        m.register_pools([mgr_pool(kvx, *g["bad_exceeds"])])
    assert e.value.code == 3
    # The native check alone (bypassing the Python pre-checks).
    P = kvx.pool_layout
    arr, keep = P.native_pools([mgr_pool(kvx, *g["bad_storage_index"])])
    with pytest.raises(kvx.KvxError, match="storage_index 5 out of range"):
        kvx._capi.check(kvx._capi.load().kvx_manager_register_pools(m._h, arr, 1))
    with pytest.raises(ValueError, match="non-empty"):
        m.register_pools([])
    assert m.num_pools() == 3  # failed registrations leave the table alone


def test_pool_block_ref_pointer_math(kvx):
    g = GOLD["manager_block_ref"]
    m = host_mgr(kvx, g["num_layers"], g["slice"], g["host_blocks"])
    m.register_pools([mgr_pool(kvx, *p) for p in g["pools"]])
    base = kvx._capi.load().kvx_manager_host_ptr(m._h, 0, 0)
    for pool_idx, block_id, off in g["refs"]:
        ref = m.get_block_ref(pool_idx, block_id)
        assert ref["ptr"] == base + off
        assert ref["pool_idx"] == pool_idx and ref["block_id"] == block_id
    assert m.get_block_ref(0, 1)["block_stride_bytes"] == 128
    assert m.get_block_ref(0, 1)["tag"] == "kind_a"
    for pool_idx, shard, block_id in g["out_of_range"]:
        with pytest.raises(kvx.KvxError) as e:
            m.get_block_ref(pool_idx, block_id, shard_idx=shard)
        assert e.value.code == 11


def test_pool_indices_with_tag_and_base_stride(kvx):
    g = GOLD["manager_tags"]
    m = host_mgr(kvx, g["num_layers"], g["slice"], g["host_blocks"])
    pools = [mgr_pool(kvx, *p) for p in g["pools"]]
    import dataclasses
    pools[1] = dataclasses.replace(pools[1], dtype_tag="dtype_b")
    m.register_pools(pools)
    assert m.pool_ids_with_tag("kind_a") == g["kind_a"]
    assert m.pool_ids_with_tag("kind_b") == g["kind_b"]
    assert m.pool_ids_with_tag("missing") == []
    assert m.pool_spec(1)["dtype_tag"] == "dtype_b"
    assert m.pool_spec(2)["regions"][0] == {"name": "payload", "offset_bytes": 0,
                                            "stride_bytes": 64, "unit_bytes": 32,
                                            "num_units": 2, "units_per_stride": 1}
    g = GOLD["manager_base_stride"]
    m = host_mgr(kvx, g["num_layers"], g["slice"], g["host_blocks"])
    m.register_pools([mgr_pool(kvx, *p) for p in g["pools"]])
    base1 = kvx._capi.load().kvx_manager_host_ptr(m._h, 1, 0)
    pool_idx, block_id, off = g["ref"]
    assert m.get_block_ref(pool_idx, block_id)["ptr"] == base1 + off


def test_python_admission_surface(kvx):
    P = kvx.pool_layout
    g = GOLD["python_aliased"]
    m = host_mgr(kvx, 1, g["slice"], g["host_blocks"])
    pool = to_spec(kvx, g["pool"])
    assert pool.storage_extent_end_bytes == g["extent_end"]
    pool.validate(storage_bytes=g["extent_end"])
    assert m.register_pools((pool,))["admitted"]
    assert m.get_block_ref(0, 1)["ptr"] == m.get_block_ref(0, 0)["ptr"] + 128
    g = GOLD["python_summary"]
    m = host_mgr(kvx, 1, g["slice"], g["host_blocks"])
    assert m.admission_summary() == {"admitted": False}
    pools = [to_spec(kvx, p) for p in g["pools"]]
    summary = m.register_pools([p.to_dict() for p in pools])  # mappings coerce too
    assert summary == g["summary"] and m.admission_summary() == summary
    first, last = m.get_block_ref(0, 0), m.get_block_ref(0, 3)
    second = m.get_block_ref(1, 2)
    assert last["ptr"] == first["ptr"] + 3 * 128
    assert second["ptr"] == first["ptr"] + (640 - 32) + 2 * 64
    assert second["dtype_tag"] == "dtype_b" and second["block_stride_bytes"] == 64
    assert m.pool_spec(1)["base_offset_bytes"] == 640
    with pytest.raises(RuntimeError, match="host-only manager"):
        m.d2h_pool_blocks(pool_idx=0, block_ids=[0])
    with pytest.raises(RuntimeError, match="host-only manager"):
        m.h2d_pool_blocks(pool_idx=0, block_ids=[0])
    with pytest.raises(ValueError, match="invalid pool 0"):
        m.register_pools([P.PoolSpec("x", 0, 0, 0, 1, (P.RegionSpec("r", 0, 1, 1, 1),))])


def test_delegate_addressing_follows_pools(kvx):
    """Block arrays become pools once registered (kv_cache_manager_base.cc:
    1470-1523, 2321-2395, 2530-2548), with the reference tests' answers."""
    lib = kvx._capi.load()
    g = GOLD["delegate_base_stride"]
    m = host_mgr(kvx, g["num_layers"], g["slice"], g["host_blocks"])
    assert m.num_block_arrays() == 2 and m.block_bytes(1) == 128
    legacy = m.get_block_chunks(1, 0, [1, 3], 200)
    s1 = m.get_host_pointer(1)
    assert legacy == [(s1 + 128, 128), (s1 + 3 * 128, 72)]
    m.register_pools([mgr_pool(kvx, *p) for p in g["pools"]])
    assert m.num_block_arrays() == 1 and m.block_bytes(0) == 64
    pool_idx, block_id, off = g["block_ptr"]
    assert lib.kvx_manager_block_array_block_ptr(m._h, pool_idx, 0, block_id) == s1 + off
    assert lib.kvx_manager_block_array_block_ptr(m._h, 0, 0, 4) == 0  # past the pool
    assert m.get_block_array_host_pointer(0) == s1 + 128
    assert m.get_block_chunks(0, 0, g["chunks_ids"], g["chunks_total"]) == \
        [(s1 + o, n) for o, n in g["chunks"]]
    assert m.get_block_chunks(0, 0, [4], 64) == []  # out of the pool: no chunks
    assert m.get_block_chunks(3, 0, [0], 64) == []
    g = GOLD["delegate_aliased"]
    m = host_mgr(kvx, g["num_layers"], g["slice"], g["host_blocks"])
    m.register_pools([mgr_pool(kvx, *p) for p in g["pools"]])
    s0 = m.get_host_pointer(0)
    assert m.get_block_array_host_size(0) == g["block_array_size"]
    assert m.get_block_ref(0, 1)["ptr"] == s0 + g["ref_block1"]
    assert m.get_block_chunks(0, 0, g["chunks_ids"], g["chunks_total"]) == \
        [(s0 + o, n) for o, n in g["chunks"]]
    g = GOLD["delegate_two_pools"]
    m = host_mgr(kvx, g["num_layers"], g["slice"], g["host_blocks"])
    m.register_pools([mgr_pool(kvx, *p) for p in g["pools"]])
    assert m.num_block_arrays() == g["num_block_arrays"]
