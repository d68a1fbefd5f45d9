"""Host-side logic through the C-ABI, on the CPU: block allocator, CPU-only
manager accessors, staging slots and error codes."""
import random

import numpy as np
import pytest


def run_lbm_case(make, case):
    m = make(case["n"])
    for op in case["ops"]:
        kind = op[0]
        if kind == "allocate":
            _, k, lock, expect = op
            code, ids = m.allocate(k, lock)
            if isinstance(expect, list):
                assert code == 0 and ids == expect, (case["source"], op)
            elif isinstance(expect, dict):
                assert code == 0 and len(ids) == expect["len"], (case["source"], op)
            else:
                assert code == expect, (case["source"], op)
        elif kind == "allocate_target":
            assert m.allocate_target(op[1]) == op[2], (case["source"], op)
        elif kind == "unlock":
            assert m.unlock(op[1]) == op[2], (case["source"], op)
        elif kind == "deallocate":
            assert m.deallocate(op[1]) == op[2], (case["source"], op)
        elif kind == "access":
            assert m.access(op[1]) == op[2], (case["source"], op)
    counts = m.counts()
    for k, v in case["expect"].items():
        assert counts[k] == v, (case["source"], k)


class ProductLbm:
    """Adapts the C-ABI allocator to the oracle's (code, value) convention."""

    def __init__(self, kvx, n):
        self.b = kvx.LogicalBlockManager(n)
        self.kvx = kvx

    def _code(self, fn, *a):
        try:
            r = fn(*a)
            return 0, r
        except self.kvx.KvxError as e:
            return e.code, None

    def allocate(self, k, lock=False):
        return self._code(self.b.allocate, k, lock)

    def allocate_target(self, ids):
        return self._code(self.b.allocate_target, ids)[0]

    def unlock(self, ids):
        return self._code(self.b.unlock, ids)[0]

    def deallocate(self, ids):
        return self._code(self.b.deallocate, ids)[0]

    def access(self, i):
        return self._code(self.b.access_block, i)[0]

    def counts(self):
        return {"total": self.b.total_blocks, "free": self.b.num_free_blocks,
                "allocated": self.b.num_allocated_blocks, "locked": self.b.num_locked_blocks}


def test_lbm_reference_cases_oracle(golden):
    from oracle import host_tier
    for case in golden["lbm_cases"]:
        run_lbm_case(host_tier.LogicalBlockManager, case)


def test_lbm_reference_cases_product(kvx, golden):
    for case in golden["lbm_cases"]:
        run_lbm_case(lambda n: ProductLbm(kvx, n), case)


def test_lbm_differential_random(kvx):
    from oracle import host_tier
    rnd = random.Random(11)
    for trial in range(20):
        n = rnd.randint(1, 40)
        a, b = host_tier.LogicalBlockManager(n), ProductLbm(kvx, n)
        for _ in range(300):
            kind = rnd.choice(["allocate", "allocate", "target", "unlock", "dealloc", "access"])
            if kind == "allocate":
                k, lock = rnd.randint(-1, n + 1), rnd.random() < 0.4
                assert a.allocate(k, lock) == b.allocate(k, lock)
            else:
                ids = [rnd.randint(-1, n) for _ in range(rnd.randint(0, 4))]
                if kind == "target":
                    assert a.allocate_target(ids) == b.allocate_target(ids)
                elif kind == "unlock":
                    assert a.unlock(ids) == b.unlock(ids)
                elif kind == "dealloc":
                    assert a.deallocate(ids) == b.deallocate(ids)
                else:
                    i = rnd.randint(-1, n)
                    assert a.access(i) == b.access(i)
            assert a.counts() == b.counts()
            for i in range(n):
                assert a.alloc[i] == b.b.is_allocated(i)
                assert a.locked[i] == b.b.is_locked(i)


@pytest.fixture
def cpu_mgr(kvx):
    m = kvx.KVCacheManager.create_host_only_for_testing(
        num_layers=3, num_shards=2, slice_byte_size=96, host_blocks=6)
    yield m
    m.close()


def test_cpu_manager_geometry(cpu_mgr):
    m = cpu_mgr
    assert m.num_layers == 3 and m.num_shards == 2 and m.host_blocks == 6
    assert m.bytes_per_block() == 96
    assert m.num_block_arrays() == 3
    assert m.block_bytes(1) == 96 and m.layer_block_byte_size(2) == 96
    assert m.layer_block_byte_size(3) == -1
    assert m.get_allocated_host_dram_bytes() == 3 * 2 * 6 * 96


def test_cpu_manager_block_bytes_round_trip(cpu_mgr, oracle):
    m = cpu_mgr
    rng = np.random.default_rng(0)
    payloads = {}
    for layer in range(3):
        for shard in range(2):
            for blk in range(6):
                p = rng.integers(0, 256, 96, dtype=np.uint8).tobytes()
                m.write_block_bytes(layer, blk, p, shard)
                payloads[layer, shard, blk] = p
    for (layer, shard, blk), p in payloads.items():
        assert m.read_block_bytes(layer, blk, shard) == p
        # The host mirror layout is [host_blocks][block bytes] per (layer, shard).
        view = m.host_view(layer, shard)
        rc, out = oracle.read_block(view, 96, blk)
        assert rc == 0 and out.tobytes() == p
    # Shard ids wrap modulo the local shard count.
    assert m.read_block_bytes(1, 2, 3) == payloads[1, 1, 2]
    ptr = m.get_block_host_pointer(2, 0, 4)
    assert ptr == m.get_block_host_pointer(2, 0, 0) + 4 * 96


def test_cpu_manager_errors(cpu_mgr, kvx):
    m = cpu_mgr
    with pytest.raises(kvx.KvxError) as e:
        m.read_block_bytes(0, 6)
    assert e.value.code == 11
    with pytest.raises(kvx.KvxError) as e:
        m.read_block_bytes(0, -1)
    assert e.value.code == 3
    with pytest.raises(kvx.KvxError) as e:
        m.write_block_bytes(0, 0, b"x" * 95)
    assert e.value.code == 3
    with pytest.raises(kvx.KvxError) as e:
        m.read_block_bytes(5, 0)
    assert e.value.code == 11
    for fn in (m.d2h, m.h2d):
        with pytest.raises(kvx.KvxError) as e:
            fn([0], [0], [1])
        assert e.value.code == 9 and "device-backed" in str(e.value)


def test_cpu_manager_staging_slots(cpu_mgr, kvx):
    m = cpu_mgr
    with pytest.raises(kvx.KvxError) as e:
        m.host_span(0, 0, 0, 1)
    assert e.value.code == 9
    with pytest.raises(kvx.KvxError):
        m.configure_host_staging_slots(0, 2)
    m.configure_host_staging_slots(3, 2)
    ptr, nbytes, base = m.host_span(1, 1, 2, 2)
    assert base == 4 and nbytes == 2 * 96
    assert ptr == m.get_block_host_pointer(1, 1, 4)
    for args, code in [((0, 0, 3, 1), 11), ((0, 0, 0, 3), 11), ((3, 0, 0, 1), 11),
                       ((0, 0, -1, 1), 11)]:
        with pytest.raises(kvx.KvxError) as e:
            m.host_span(*args)
        assert e.value.code == code


def test_cpu_manager_auto_allocate_needs_device(kvx):
    m = kvx.KVCacheManager.create_host_only_for_testing(num_layers=1, slice_byte_size=64,
                                                        host_blocks=4)
    lbm = m.host_block_manager()
    assert lbm.total_blocks == 4
    with pytest.raises(kvx.KvxError) as e:
        m.d2h_auto_allocate([0], [1])
    assert e.value.code == 9
    # Auto-allocate takes its ids before the copy fails, as the reference does.
    assert lbm.num_locked_blocks == 1
    m.close()


def test_node_id_kept(kvx):
    m = kvx.KVCacheManager.create_host_only_for_testing(num_layers=1, slice_byte_size=64,
                                                        host_blocks=4, node_id=5)
    assert m.node_id == 5
    m.close()
