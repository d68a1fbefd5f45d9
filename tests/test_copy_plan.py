"""Copy specs, the load plan and the staging-slot pool on the CPU.

The product's OffsetsImpl / BuildCoalescedCopySpec / BuildLoadCopyPlan
(through the C-ABI) against the oracle; the oracle's load plan against
invariants fixed independently of its loop; the slot pool
(kv_cache_manager_with_transfer.cc:1807-1916) on host-only managers."""
import numpy as np
import pytest


def expand(spec):
    out = []
    for s, d, z in zip(spec["src_offsets"], spec["dst_offsets"], spec["sizes"]):
        out += [(s + k, d + k) for k in range(z)]
    return out


def as_spec(t):
    return {"src_offsets": t[0], "dst_offsets": t[1], "sizes": t[2]}


def test_product_specs_match_oracle(kvx, oracle, golden):
    cp = kvx.copy_plan
    for c in golden["offsets_impl_cases"]:
        assert cp.offsets_impl(c["ids"], c["source_is_compact"]) == as_spec(c["expect"])
    rng = np.random.default_rng(5)
    for _ in range(300):
        n = int(rng.integers(0, 40))
        ids = rng.choice(100, n, replace=False).tolist()
        if rng.random() < 0.5:
            ids.sort()
        for compact in (True, False):
            assert cp.offsets_impl(ids, compact) == as_spec(oracle.offsets_impl(ids, compact))
        other = rng.choice(100, n, replace=False).tolist()
        if rng.random() < 0.5:
            other.sort()
        assert cp.build_coalesced_copy_spec(ids, other) == \
            as_spec(oracle.build_coalesced_copy_spec(ids, other))
    with pytest.raises(kvx.KvxError):
        cp.build_coalesced_copy_spec([1, 2], [3])


def random_load(rng, dup_conflict=False):
    n = int(rng.integers(0, 30))
    remote = rng.integers(0, 20, n).tolist()  # repeats allowed
    local = rng.integers(0, 25, n).tolist()
    mapping = {}
    host = []
    for l in local:
        if l not in mapping:
            mapping[l] = int(rng.integers(0, 200))
        host.append(mapping[l])
    if dup_conflict and n > 1:
        seen = {}
        for i, l in enumerate(local):
            if l in seen:
                host[i] = host[seen[l]] + 1
                break
            seen[l] = i
    return remote, local, host


def test_oracle_load_plan_invariants(oracle):
    """Transport order = stable sort of (remote, host) by remote; expanding
    the H2D runs gives one copy per distinct local id from its host id; a
    local id repeated with another host id is rejected."""
    rng = np.random.default_rng(6)
    for _ in range(300):
        remote, local, host = random_load(rng)
        p = oracle.build_load_copy_plan(remote, local, host)
        pairs = sorted(zip(remote, range(len(remote)), host))
        assert p["producer_remote_block_ids"] == [r for r, _, _ in pairs]
        assert p["transport_host_block_ids"] == [h for _, _, h in pairs]
        want = sorted({(h, l) for l, h in zip(local, host)}, key=lambda t: t[1])
        assert expand(p["h2d_copy"]) == want
        assert p["h2d_local_block_ids"] == sorted(set(local))
    conflicts = 0
    for _ in range(200):
        remote, local, host = random_load(rng, dup_conflict=True)
        if len(set(zip(local, host))) != len(set(local)):
            conflicts += 1
            with pytest.raises(ValueError, match="Duplicate local block IDs"):
                oracle.build_load_copy_plan(remote, local, host)
    assert conflicts > 50


def test_product_load_plan_matches_oracle(kvx, oracle):
    rng = np.random.default_rng(7)
    for _ in range(300):
        remote, local, host = random_load(rng, dup_conflict=rng.random() < 0.3)
        try:
            want = oracle.build_load_copy_plan(remote, local, host)
        except ValueError:
            with pytest.raises(kvx.KvxError, match="Duplicate local block IDs") as e:
                kvx.copy_plan.build_load_copy_plan(remote, local, host)
            assert e.value.code == 3
            continue
        got = kvx.copy_plan.build_load_copy_plan(remote, local, host)
        for k, v in want.items():
            assert got[k] == v, k
        assert got["num_blocks"] == len(remote)
    with pytest.raises(kvx.KvxError, match="same length"):
        kvx.copy_plan.build_load_copy_plan([1], [2], [])


def slot_mgr(kvx, num_layers=2, num_shards=1, slice_bytes=64, host_blocks=12):
    return kvx.KVCacheManager.create_host_only_for_testing(
        num_layers=num_layers, num_shards=num_shards, slice_byte_size=slice_bytes,
        host_blocks=host_blocks)


def test_slot_pool_allocation_and_fifo(kvx):
    m = slot_mgr(kvx)
    with pytest.raises(kvx.KvxError, match="not configured") as e:
        m.initialize_slot_pool(2)
    assert e.value.code == 9
    m.configure_host_staging_slots(4, 4)
    with pytest.raises(kvx.KvxError, match="Required: 16, Available: 12") as e:
        m.initialize_slot_pool(4)
    assert e.value.code == 9
    m.initialize_slot_pool(3)
    # Ascending free ids from the host block manager, locked.
    assert [m.slot_block_ids(i) for i in range(3)] == [[0, 1, 2, 3], [4, 5, 6, 7],
                                                      [8, 9, 10, 11]]
    lbm = m.host_block_manager()
    assert lbm.num_free_blocks == 0 and lbm.num_locked_blocks == 12
    assert [m.acquire_slot() for _ in range(3)] == [0, 1, 2]
    with pytest.raises(kvx.KvxError, match="slot pool exhausted") as e:
        m.acquire_slot()
    assert e.value.code == 8
    m.release_slot(1)
    m.release_slot(0)
    m.release_slot(7)  # out of range: ignored
    assert m.num_free_slots() == 2
    assert [m.acquire_slot(), m.acquire_slot()] == [1, 0]
    with pytest.raises(kvx.KvxError) as e:
        m.slot_block_ids(3)
    assert e.value.code == 11


def test_layer_spans_follow_slot_runs(kvx):
    m = slot_mgr(kvx, num_layers=2, num_shards=2, slice_bytes=32, host_blocks=10)
    # Fragment the free list so slot 0's ids are not contiguous.
    lbm = m.host_block_manager()
    lbm.allocate_target([1, 4])
    m.configure_host_staging_slots(2, 4)
    m.initialize_slot_pool(2)
    ids = m.slot_block_ids(0)
    assert ids == [0, 2, 3, 5]
    spans = m.layer_spans(0, 4)
    lib = kvx._capi.load()
    runs = [(0, 1), (2, 2), (5, 1)]
    assert len(spans) == 2 * 2 * len(runs)
    k = 0
    for layer in range(2):
        for shard in range(2):
            base = lib.kvx_manager_block_array_host_ptr(m._h, layer, shard)
            for start, n in runs:
                s = spans[k]
                assert (s["layer_idx"], s["shard_idx"], s["base_major"], s["num_major"]) == \
                    (layer, shard, start, n)
                assert s["ptr"] == base + start * 32 and s["nbytes"] == n * 32
                assert s["slot_idx"] == 0
                k += 1
    assert m.layer_spans(0, 2)[0]["num_major"] == 1 and len(m.layer_spans(0, 0)) == 0
    with pytest.raises(kvx.KvxError) as e:
        m.layer_spans(0, 5)
    assert e.value.code == 11


def test_prepare_load_assigns_slot_ids_per_distinct_local(kvx, oracle):
    m = slot_mgr(kvx)
    m.configure_host_staging_slots(3, 4)
    m.initialize_slot_pool(3)
    r = m.prepare_load([5, 6, 7, 1], [3, 3, 8, 0])
    assert r["slot_idx"] == 0
    assert r["host_block_ids"] == [0, 0, 1, 2]
    want = oracle.build_load_copy_plan([5, 6, 7, 1], [3, 3, 8, 0], [0, 0, 1, 2])
    for k, v in want.items():
        assert r["plan"][k] == v
    # Caller-supplied host ids: no slot taken.
    free = m.num_free_slots()
    r = m.prepare_load([1, 2], [4, 5], [9, 10])
    assert r["slot_idx"] == -1 and r["host_block_ids"] == [9, 10]
    assert m.num_free_slots() == free
    with pytest.raises(kvx.KvxError, match="exceeds the slot size") as e:
        m.prepare_load(list(range(5)), list(range(5)))
    assert e.value.code == 8
    # A conflicting caller mapping fails and takes no slot.
    with pytest.raises(kvx.KvxError, match="Duplicate local block IDs"):
        m.prepare_load([1, 2], [4, 4], [9, 10])
    assert m.num_free_slots() == free


def test_slot_copies_need_a_device_backed_manager(kvx):
    m = slot_mgr(kvx)
    m.configure_host_staging_slots(3, 4)
    m.initialize_slot_pool(3)
    with pytest.raises(kvx.KvxError, match="device-backed") as e:
        m.issue_h2d(0, 2, [5, 6])
    assert e.value.code == 9
    with pytest.raises(kvx.KvxError, match="num_blocks must match"):
        m.issue_h2d(0, 2, [5])
    with pytest.raises(kvx.KvxError, match="num_blocks out of range"):
        m.issue_h2d(0, 5, [1, 2, 3, 4, 5])
    free = m.num_free_slots()
    with pytest.raises(kvx.KvxError, match="device-backed"):
        m.stage_for_push([1, 2])
    assert m.num_free_slots() == free  # the slot went back
    with pytest.raises(kvx.KvxError, match="exceeds the slot size"):
        m.stage_for_push(list(range(5)))
