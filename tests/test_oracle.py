"""Pins the oracle (CPU restatement of the reference's host path).

Each check is independent of the oracle's own code: brute-force expansion
of runs, numpy fancy indexing as the library routine for block moves, the
reference tests' known answers (tests/golden/reference_cases.json), and
error codes the reference returns for invalid input.
"""
import numpy as np
import pytest


def expand(src, dst, sizes):
    pairs = []
    for s, d, z in zip(src, dst, sizes):
        pairs += [(s + k, d + k) for k in range(z)]
    return pairs


def random_runs(rng, n, hi, max_run=4):
    src, dst, sizes = [], [], []
    for _ in range(n):
        z = int(rng.integers(1, max_run + 1))
        # Bias toward continuing runs so that coalescing has work to do.
        if src and rng.random() < 0.5:
            src.append(src[-1] + sizes[-1])
            dst.append(dst[-1] + sizes[-1] if rng.random() < 0.8 else int(rng.integers(0, hi)))
        else:
            src.append(int(rng.integers(0, hi)))
            dst.append(int(rng.integers(0, hi)))
        sizes.append(z)
    return src, dst, sizes


def test_coalesce_bruteforce(oracle):
    rng = np.random.default_rng(1)
    for _ in range(300):
        src, dst, sizes = random_runs(rng, int(rng.integers(0, 20)), 50)
        cs, cd, cz = oracle.coalesce(src, dst, sizes)
        # Same copies, same order.
        assert expand(cs, cd, cz) == expand(src, dst, sizes)
        # Maximal: no run continues its predecessor in both src and dst.
        for j in range(1, len(cs)):
            assert not (cs[j] == cs[j - 1] + cz[j - 1] and cd[j] == cd[j - 1] + cz[j - 1])
        assert len(cs) <= len(src)


def test_coalesce_and_offsets_known_cases(oracle, golden):
    for c in golden["coalesce_cases"]:
        assert oracle.coalesce(c["src"], c["dst"], c["sizes"]) == c["expect"], c["source"]
    for c in golden["offsets_impl_cases"]:
        assert oracle.offsets_impl(c["ids"], c["source_is_compact"]) == c["expect"], c["source"]


def test_offsets_impl_bruteforce(oracle):
    rng = np.random.default_rng(2)
    for _ in range(200):
        n = int(rng.integers(0, 30))
        ids = rng.choice(60, size=n, replace=False).tolist()
        if rng.random() < 0.5:
            ids.sort()
        for compact_src in (True, False):
            s, d, z = oracle.offsets_impl(ids, compact_src)
            pairs = expand(s, d, z)
            want = [(i, b) for i, b in enumerate(ids)] if compact_src else \
                   [(b, i) for i, b in enumerate(ids)]
            assert pairs == want


def test_build_coalesced_copy_spec_bruteforce(oracle):
    rng = np.random.default_rng(3)
    for _ in range(200):
        n = int(rng.integers(0, 30))
        a = rng.choice(80, size=n, replace=False)
        b = rng.choice(80, size=n, replace=False)
        if rng.random() < 0.5:
            a.sort()
            b.sort()
        s, d, z = oracle.build_coalesced_copy_spec(a.tolist(), b.tolist())
        assert expand(s, d, z) == list(zip(a.tolist(), b.tolist()))
    with pytest.raises(ValueError):
        oracle.build_coalesced_copy_spec([1, 2], [3])


def test_validate_codes(oracle):
    assert oracle.validate([0, 1], [0, 1], [1, 1]) == 0
    assert oracle.validate([0, 1], [0], [1, 1]) == 3   # length mismatch
    assert oracle.validate([0, 1], [0, 1], [1]) == 3
    assert oracle.validate([0], [], []) == 0           # empty dst/sizes allowed
    assert oracle.validate([-1], [0], [1]) == 3        # negative offset
    assert oracle.validate([0], [-2], [1]) == 3
    assert oracle.validate([0], [0], [-1]) == 3


def make_pools(rng, layers, blocks, bb):
    return [rng.integers(0, 256, size=blocks * bb, dtype=np.uint8) for _ in range(layers)]


def test_transfer_matches_numpy_indexing(oracle):
    rng = np.random.default_rng(4)
    for trial in range(60):
        layers, blocks, hb, bb = 3, 24, 20, int(rng.choice([16, 48, 256]))
        dev = make_pools(rng, layers, blocks, bb)
        host = [np.zeros(hb * bb, np.uint8) for _ in range(layers)]
        n = int(rng.integers(1, 10))
        src = rng.choice(blocks, size=n, replace=False).tolist()
        dst = rng.choice(hb, size=n, replace=False).tolist()
        rc = oracle.transfer(True, dev, host, [bb] * layers, [blocks * bb] * layers, src, dst, [])
        assert rc == 0
        for l in range(layers):
            want = np.zeros((hb, bb), np.uint8)
            want[np.array(dst)] = dev[l].reshape(blocks, bb)[np.array(src)]
            assert np.array_equal(host[l].reshape(hb, bb), want)
        # H2d back into other device blocks leaves every other block alone.
        before = [d.copy() for d in dev]
        dst2 = rng.choice(blocks, size=n, replace=False).tolist()
        rc = oracle.transfer(False, dev, host, [bb] * layers, [blocks * bb] * layers, dst, dst2, [])
        assert rc == 0
        for l in range(layers):
            want = before[l].reshape(blocks, bb).copy()
            want[np.array(dst2)] = before[l].reshape(blocks, bb)[np.array(src)]
            assert np.array_equal(dev[l].reshape(blocks, bb), want)


def test_transfer_reference_known_answers(oracle, golden):
    rng = np.random.default_rng(5)
    bb = 64
    for case in golden["transfer_cases"]:
        L, P, H = case["layers"], case["blocks"], case["host_blocks"]
        dev = make_pools(rng, L, P, bb)
        orig = [d.copy() for d in dev]
        host = [np.zeros(H * bb, np.uint8) for _ in range(L)]
        next_free = 0
        for op in case["ops"]:
            if op["op"] == "d2h_auto_allocate":
                total = sum(op["sizes"])
                ids = list(range(next_free, next_free + total))  # fresh manager: ascending
                assert ids == op["expect_ids"]
                srcs = [s + k for s, z in zip(op["src"], op["sizes"]) for k in range(z)]
                rc = oracle.transfer(True, dev, host, [bb] * L, [P * bb] * L, srcs, ids, [1] * total)
            else:
                rc = oracle.transfer(op["op"] == "d2h", dev, host, [bb] * L, [P * bb] * L,
                                     op["src"], op["dst"], op["sizes"])
            assert rc == 0, case["source"]
        for l in range(L):
            d = dev[l].reshape(P, bb)
            o = orig[l].reshape(P, bb)
            for e in case["expect_device"]:
                assert np.array_equal(d[e["dst"]], o[e["orig"]]), case["source"]


def test_transfer_error_codes(oracle):
    rng = np.random.default_rng(6)
    bb, P, H = 32, 8, 4
    dev = make_pools(rng, 2, P, bb)
    host = [np.zeros(H * bb, np.uint8) for _ in range(2)]
    args = ([bb] * 2, [P * bb] * 2)
    assert oracle.transfer(True, dev, host, *args, [7], [0], [2]) == 3   # device range
    assert oracle.transfer(True, dev, host, *args, [0], [3], [2]) == 3   # host range
    assert oracle.transfer(False, dev, host, *args, [3], [0], [2]) == 3  # host src range
    assert oracle.transfer(False, dev, host, *args, [0], [7], [2]) == 3  # device dst range
    assert oracle.transfer(True, dev, host, *args, [-1], [0], [1]) == 3
    assert oracle.transfer(True, dev, host, *args, [0], [], []) == 3     # no destinations
    # Whole-layer copy into a host mirror smaller than the layer.
    assert oracle.transfer(True, dev, host, *args, [], [], []) == 11
    assert oracle.transfer(False, dev, host, *args, [], [], []) == 3
    # A failing call moves nothing.
    assert not host[0].any()


@pytest.mark.parametrize("order", [0, 1])
@pytest.mark.parametrize("nthreads", [1, 3])
def test_extract_insert_match_numpy(oracle, order, nthreads):
    rng = np.random.default_rng(7 + order)
    L, P, bb = 4, 64, 256
    pools = make_pools(rng, L, P, bb)
    ids = rng.choice(P, size=16, replace=False)
    rc, stg = oracle.extract(pools, bb, ids, order=order, nthreads=nthreads)
    assert rc == 0
    want = np.stack([p.reshape(P, bb)[ids] for p in pools])  # [L][n][bb]
    if order == 1:
        want = want.transpose(1, 0, 2)
    assert np.array_equal(stg.reshape(want.shape), want)
    fresh = [np.zeros_like(p) for p in pools]
    assert oracle.insert(fresh, bb, ids, stg, order=order, nthreads=nthreads) == 0
    for l in range(L):
        got = fresh[l].reshape(P, bb)
        assert np.array_equal(got[ids], pools[l].reshape(P, bb)[ids])
        mask = np.ones(P, bool)
        mask[ids] = False
        assert not got[mask].any()


def test_read_write_block_codes(oracle):
    host = np.zeros(4 * 16, np.uint8)
    assert oracle.write_block(host, 16, 3, np.arange(16, dtype=np.uint8)) == 0
    rc, out = oracle.read_block(host, 16, 3)
    assert rc == 0 and out.tolist() == list(range(16))
    assert oracle.read_block(host, 16, 4)[0] == 11
    assert oracle.read_block(host, 16, -1)[0] == 3
    assert oracle.write_block(host, 16, 0, np.zeros(15, np.uint8)) == 3
