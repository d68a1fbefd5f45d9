"""Weight-sync host logic on the CPU: the oracle's strided-entry expansion and
shard-slice math against known answers, and the product's entry builders
(column split, shard slices) against the oracle and numpy slicing."""
import numpy as np
import pytest

from fake_device import FakeDeviceTensor
from oracle import weight_sync as W


def test_expand_entries_known_answers():
    # weight_synchronizer_base.cc:634-666: contiguous entries collapse to one
    # task, strided ones expand per row, count <= 0 means one row.
    assert W.expand_entries([(8, 100, 16, 4, 16, 16)]) == [(8, 100, 64)]
    assert W.expand_entries([(0, 0, 4, 3, 10, 4)]) == [(0, 0, 4), (10, 4, 4), (20, 8, 4)]
    assert W.expand_entries([(5, 7, 3, 0, 99, 99)]) == [(5, 7, 3)]
    assert W.expand_entries([(5, 7, 3, -2, 99, 99)]) == [(5, 7, 3)]
    assert W.expand_entries([(0, 1, 2, 2, 2, 5)]) == [(0, 1, 2), (2, 6, 2)]


def test_nd_shard_slices_known_answers():
    # nd_slice_math.py:55-68: the last shard takes the remainder.
    assert W.nd_shard_slices((10,), (3,)) == [[(0, 3)], [(3, 6)], [(6, 10)]]
    assert W.nd_shard_slices((4, 10), (2, 2)) == [
        [(0, 2), (0, 5)], [(0, 2), (5, 10)], [(2, 4), (0, 5)], [(2, 4), (5, 10)]]
    assert W.nd_shard_slices((7, 7), (1, 8))[-1] == [(0, 7), (0, 7)]  # tile 0
    with pytest.raises(ValueError):
        W.nd_shard_slices((4,), (1, 1))


def test_nd_shard_slices_reference_goldens(kvx):
    """The reference's own goldens (nd_slice_math_test.py:70-100), for the
    oracle and the product."""
    import json
    import os
    path = os.path.join(os.path.dirname(__file__), "golden", "nd_slice_cases.json")
    with open(path) as f:
        cases = json.load(f)["cases"]
    assert len(cases) == 2
    for c in cases:
        want = [[tuple(d) for d in shard] for shard in c["bounds"]]
        shape, mesh = tuple(c["global_shape"]), tuple(c["mesh_shape"])
        assert [[tuple(d) for d in s] for s in W.nd_shard_slices(shape, mesh)] == want
        assert [[tuple(d) for d in s] for s in kvx.compute_nd_shard_slices(shape, mesh)] == want


def test_product_shard_slices_match_oracle(kvx):
    rng = np.random.default_rng(0)
    for _ in range(200):
        rank = int(rng.integers(1, 4))
        shape = tuple(int(x) for x in rng.integers(1, 50, rank))
        mesh = tuple(int(x) for x in rng.integers(1, 6, rank))
        assert kvx.compute_nd_shard_slices(shape, mesh) == W.nd_shard_slices(shape, mesh)
    with pytest.raises(ValueError):
        kvx.compute_nd_shard_slices((4, 4), (0, 1))


def test_column_split_entries_equal_numpy_slicing(kvx):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(1)
    for rows, cols, k in [(5, 16, 8), (7, 13, 3), (4, 4096, 8), (3, 9, 8), (2, 5, 8)]:
        w = torch.from_numpy(rng.integers(-30000, 30000, (rows, cols), dtype=np.int16))
        bounds = W.nd_shard_slices((rows, cols), (1, k))
        outs = [torch.zeros(rows, b[1][1] - b[1][0], dtype=torch.int16) for b in bounds]
        entries = {e.dst: e for e in kvx.column_split_entries(
            FakeDeviceTensor(w), [FakeDeviceTensor(o) for o in outs])}
        # Execute the entries with the oracle on the host bytes: every output
        # must equal the numpy column slice (empty chunks have no entry).
        src = w.numpy().view(np.uint8).reshape(-1)
        base = w.data_ptr()
        for o, b in zip(outs, bounds):
            if o.numel() == 0:
                assert o.data_ptr() not in entries or o.data_ptr() == 0
                continue
            e = entries[o.data_ptr()]
            dst = o.numpy().view(np.uint8).reshape(-1)
            W.apply_entries(src, dst, [(e.src - base, 0, e.size, e.count, e.src_stride,
                                        e.dst_stride)])
            assert np.array_equal(o.numpy(), w.numpy()[:, b[1][0]:b[1][1]])


def test_strided_plan_holds_the_entries(kvx):
    """A StridedPlan is the C-ABI entry array of its entries, field by field
    (offsets folded into the addresses)."""
    rng = np.random.default_rng(3)
    entries = [kvx.StridedEntry(int(rng.integers(1, 1 << 47)), int(rng.integers(1, 1 << 47)),
                                int(rng.integers(1, 1 << 20)), int(rng.integers(1, 5000)),
                                int(rng.integers(0, 1 << 30)), int(rng.integers(0, 1 << 30)))
               for _ in range(300)]
    plan = kvx.StridedPlan(entries)
    assert plan.n == 300
    for e, a in zip(entries, plan._arr):
        assert (a.src, a.dst, a.size_bytes, a.count, a.src_stride_bytes,
                a.dst_stride_bytes) == e.as_tuple()
        assert a.src_offset_bytes == 0 and a.dst_offset_bytes == 0
    assert kvx.StridedPlan([]).n == 0


def test_offset_table_definition():
    offs, total = W.offset_table([10, 256, 1, 0, 300])
    assert offs == [0, 256, 512, 768, 768] and total == 1280
    img, offs = W.pack([np.full(3, 7, np.uint8), np.arange(5, dtype=np.uint8)])
    assert offs == [0, 256] and img.size == 512
    assert list(img[:4]) == [7, 7, 7, 0] and list(img[256:261]) == [0, 1, 2, 3, 4]
