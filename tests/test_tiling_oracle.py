"""Tiled layouts on the CPU: the oracle (XLA nested tiling element by element)
against the reference tiling tests' known answers, an independent numpy
formulation of 2-D tiling and row packing, and brute-force bijection /
padding checks; the product's host-side layout logic (element counts,
validation) against the oracle; the kernel's multiply-high division against
'/'. No GPU."""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DTYPES = {"f32": np.float32, "bf16": np.uint16, "s8": np.int8}


def _cases():
    with open(os.path.join(ROOT, "tests", "golden", "tiling_cases.json")) as f:
        return json.load(f)["cases"]


def _values(case):
    n = int(np.prod(case["dims"]))
    a, b, m = case["values"]
    i = np.arange(n, dtype=np.float64 if isinstance(a, float) else np.int64)
    v = i * a + b
    if m is not None:
        v = v % m
    return v.astype(DTYPES[case["dtype"]])


def _layout(case):
    return {"itemsize": np.dtype(DTYPES[case["dtype"]]).itemsize, "dims": case["dims"],
            "minor_to_major": case["minor_to_major"], "tiles": case["tiles"]}


def numpy_tile_2d(x, tH, tW, P=1):
    """Independent formulation of a row-major [..., H, W] array in a (tH, tW)
    tiled layout (optionally followed by a (P, 1) row packing): pad with
    zeros to whole tiles, split rows and columns into (tile, in-tile) axes,
    bring the tile axes before the in-tile axes, and for P > 1 move the P rows
    of each row group next to each other within a column."""
    *batch, H, W = x.shape
    nT0, nT1 = -(-H // tH), -(-W // tW)
    pad = np.zeros(tuple(batch) + (nT0 * tH, nT1 * tW), x.dtype)
    pad[..., :H, :W] = x
    t = pad.reshape(tuple(batch) + (nT0, tH, nT1, tW))
    t = np.moveaxis(t, -3, -2)  # [..., nT0, nT1, tH, tW]
    if P > 1:
        t = t.reshape(t.shape[:-2] + (tH // P, P, tW))
        t = np.swapaxes(t, -1, -2)  # [..., tH / P, tW, P]
    return np.ascontiguousarray(t).reshape(-1)


@pytest.mark.parametrize("case", _cases(), ids=lambda c: c["name"])
def test_oracle_reference_known_answers(oracle, case):
    lay = _layout(case)
    x = _values(case)
    if "tiled_elements" in case:
        assert oracle.tiled_elements(lay) == case["tiled_elements"]
    tiled = oracle.tile(lay, x).view(x.dtype)
    for pos, val in case.get("expect", []):
        assert tiled[pos] == val, (case["name"], pos)
    back = oracle.detile(lay, tiled).view(x.dtype)
    assert np.array_equal(back, x)


@pytest.mark.parametrize("case", _cases(), ids=lambda c: c["name"])
def test_oracle_matches_numpy_formulation(oracle, case):
    """Every reference case with row-major order or permuted outer
    dimensions, one 2-D tile and an optional (P, 1) packing, against the
    numpy formulation (the permutation applied with np.transpose first)."""
    tiles, mtm, dims = case["tiles"], case["minor_to_major"], case["dims"]
    if not tiles or len(tiles[0]) != 2 or len(tiles) > 2:
        pytest.skip("not a 2-D tiling")
    P = 1
    if len(tiles) == 2:
        if tiles[1][1] != 1:
            pytest.skip("second tile is not a row packing")
        P = tiles[1][0]
    x = _values(case).reshape(dims)
    if len(dims) == 1:
        x = x.reshape(1, -1)
    else:
        x = np.transpose(x, list(reversed(mtm)))  # physical (major-to-minor) order
    want = numpy_tile_2d(x, tiles[0][0], tiles[0][1], P)
    got = oracle.tile(_layout(case), _values(case)).view(want.dtype)
    assert np.array_equal(got, want), case["name"]


def _random_layout(rng):
    rank = int(rng.integers(1, 5))
    dims = [int(rng.integers(1, 9)) for _ in range(rank)]
    mtm = [int(v) for v in rng.permutation(rank)]
    tiles = []
    for _ in range(int(rng.integers(1, 4))):
        k = int(rng.integers(1, 4))
        tiles.append([int(rng.integers(1, 5)) for _ in range(k)])
    return {"itemsize": 4, "dims": dims, "minor_to_major": mtm, "tiles": tiles}


def test_oracle_bijection_and_padding_random_layouts(oracle):
    """Random nested layouts (ranks 1-4, any permutation, 1-3 tiles of rank
    1-3): tiling values 1..n puts each exactly once, zero everywhere else,
    and detiling gives them back."""
    rng = np.random.default_rng(7)
    for _ in range(300):
        lay = _random_layout(rng)
        n = int(np.prod(lay["dims"]))
        x = np.arange(1, n + 1, dtype=np.uint32)
        t = oracle.tile(lay, x).view(np.uint32)
        assert t.size == oracle.tiled_elements(lay)
        nz = t[t != 0]
        assert np.array_equal(np.sort(nz), x), lay
        assert np.array_equal(oracle.detile(lay, t).view(np.uint32), x), lay


def test_oracle_rank1_and_untiled(oracle):
    # A rank-1 tensor is tiled as (1, W): row 0 of each (8, 128) tile.
    lay = {"itemsize": 2, "dims": [300], "minor_to_major": [0], "tiles": [[8, 128]]}
    x = np.arange(300, dtype=np.uint16) + 1
    t = oracle.tile(lay, x).view(np.uint16).reshape(3, 8, 128)
    assert np.array_equal(t[:, 0, :].reshape(-1)[:300], x)
    assert not t[:, 1:, :].any() and not t[2, 0, 44:].any()
    # No tiles: the bytes as they are, whatever the dimension order.
    lay = {"itemsize": 4, "dims": [3, 5], "minor_to_major": [0, 1], "tiles": []}
    x = np.arange(15, dtype=np.uint32)
    assert np.array_equal(oracle.tile(lay, x).view(np.uint32), x)


def _c_layout(kvx, lay):
    from tpu_sync_amd.tiling import TiledLayout
    return TiledLayout(lay["itemsize"], lay["dims"], lay["tiles"], lay["minor_to_major"])


def test_product_elements_match_oracle(kvx, oracle):
    from tpu_sync_amd.tiling import tiled_buffer_elements
    for case in _cases():
        lay = _layout(case)
        if case["tiles"]:
            assert tiled_buffer_elements(_c_layout(kvx, lay)) == oracle.tiled_elements(lay)
    rng = np.random.default_rng(11)
    for _ in range(300):
        lay = _random_layout(rng)
        assert tiled_buffer_elements(_c_layout(kvx, lay)) == oracle.tiled_elements(lay), lay


@pytest.mark.parametrize("bad, msg", [
    ({"itemsize": 3, "dims": [4, 4], "minor_to_major": [1, 0], "tiles": [[2, 2]]}, "itemsize"),
    ({"itemsize": 2, "dims": [4, 4], "minor_to_major": [1, 1], "tiles": [[2, 2]]}, "permutation"),
    ({"itemsize": 2, "dims": [4, 4], "minor_to_major": [1, 0], "tiles": [[0, 2]]}, ">= 1"),
    ({"itemsize": 2, "dims": [4, 4], "minor_to_major": [1, 0], "tiles": [[-1, 2]]}, ">= 1"),
    ({"itemsize": 2, "dims": [4, -4], "minor_to_major": [1, 0], "tiles": [[2, 2]]}, "negative"),
])
def test_product_rejects_bad_layouts(kvx, bad, msg):
    from tpu_sync_amd.tiling import tiled_buffer_elements
    with pytest.raises(kvx.KvxError, match=msg):
        tiled_buffer_elements(_c_layout(kvx, bad))


def test_tile_entry_points_reject_bad_layouts_before_any_device_call(kvx):
    """kvx_tile_buffer / kvx_detile_buffer validate the layout first (no HIP
    call is made, so this runs without a GPU)."""
    import ctypes
    from tpu_sync_amd import _capi
    from tpu_sync_amd.tiling import TiledLayout
    lib = _capi.load()
    bad = TiledLayout(2, (4, 4), [(0, 2)]).to_c()
    out = ctypes.c_void_p()
    for fn in (lib.kvx_tile_buffer, lib.kvx_detile_buffer):
        rc = fn(0, ctypes.byref(bad), 4096, 8192, None, ctypes.byref(out))
        assert rc == 3 and out.value is None
    c = TiledLayout(2, (4, 4), [(2, 2)]).to_c()
    c.rank = 9
    assert lib.kvx_tiled_buffer_elements(ctypes.byref(c), ctypes.byref(ctypes.c_int64())) == 3


def test_fast_division_matches_integer_division(tmp_path):
    cxx = shutil.which("g++") or shutil.which("c++")
    if cxx is None:
        pytest.skip("no C++ compiler")
    exe = tmp_path / "fast_div_check"
    env = {k: v for k, v in os.environ.items() if k != "LD_PRELOAD"}
    subprocess.run([cxx, "-O2", "-std=c++17", "-Wall", "-Werror", "-D__HIP_PLATFORM_AMD__",
                    "-I/opt/rocm/include",
                    "-I", os.path.join(ROOT, "tpu-sync_amd", "csrc", "kernels"),
                    os.path.join(ROOT, "tests", "fast_div_check.cc"), "-o", str(exe)],
                   check=True, capture_output=True, text=True, env=env)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120, env=env)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "fast div ok" in r.stdout


def test_tiled_job_builder_alignment_and_limits(tmp_path):
    """The job builder of libkvx on the CPU (tests/tiled_jobs_check.cc):
    buffers below the element size's alignment are refused for every form,
    and the 32-bit unit limits are re-checked at the vector width the
    buffers allow (an 8 GiB int8 tensor at 1- or 2-byte alignment is refused
    instead of wrapping its unit indices)."""
    cxx = shutil.which("g++") or shutil.which("c++")
    libdir = os.path.join(ROOT, "tpu-sync_amd")
    if cxx is None or not os.path.exists(os.path.join(libdir, "libkvx.so")):
        pytest.skip("no C++ compiler or libkvx.so not built")
    exe = tmp_path / "tiled_jobs_check"
    env = {k: v for k, v in os.environ.items() if k != "LD_PRELOAD"}
    r = subprocess.run([cxx, "-O1", "-std=c++17", "-Wall", "-Werror", "-D__HIP_PLATFORM_AMD__",
                        "-I/opt/rocm/include",
                        "-I", os.path.join(ROOT, "tpu-sync_amd", "csrc", "host"),
                        os.path.join(ROOT, "tests", "tiled_jobs_check.cc"), "-o", str(exe),
                        "-L", libdir, "-lkvx", f"-Wl,-rpath,{libdir}"],
                       capture_output=True, text=True, env=env)
    assert r.returncode == 0, r.stdout + r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120, env=env)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all checks passed" in r.stdout


def _standard(lay):
    dims, tiles, mtm = lay["dims"], lay["tiles"], lay["minor_to_major"]
    r = len(dims)
    if any(mtm[i] != r - 1 - i for i in range(r)) or not tiles or len(tiles[0]) != 2:
        return None
    P = 1
    if len(tiles) == 2:
        if len(tiles[1]) != 2 or tiles[1][1] != 1 or tiles[1][0] not in (2, 4):
            return None
        P = tiles[1][0]
        if P * lay["itemsize"] != 4 or tiles[0][0] % P:
            return None
    elif len(tiles) > 2:
        return None
    W = dims[-1]
    H = 1 if r == 1 else dims[-2]
    B = int(np.prod(dims)) // (W * H)
    return B, H, W, tiles[0][0], tiles[0][1], P


def test_threaded_standard_detile_matches_oracle(oracle):
    """The timed CPU baseline (the reference's standard-form host detile,
    tile rows over threads) against the element-by-element oracle."""
    rng = np.random.default_rng(13)
    lays = [_layout(c) for c in _cases()]
    for _ in range(60):
        s = int(rng.choice([1, 2, 4, 8]))
        packed = s in (1, 2) and rng.random() < 0.5
        P = 4 // s if packed else 1
        tH = int(rng.choice([1, 2, 4, 8])) * P
        tW = int(rng.choice([1, 3, 16, 128]))
        dims = [int(rng.integers(1, 4)) for _ in range(int(rng.integers(0, 3)))]
        dims += [int(rng.integers(1, 30)), int(rng.integers(1, 300))]
        tiles = [[tH, tW]] + ([[P, 1]] if packed else [])
        lays.append({"itemsize": s, "dims": dims,
                     "minor_to_major": list(range(len(dims) - 1, -1, -1)), "tiles": tiles})
    checked = 0
    for lay in lays:
        std = _standard(lay)
        if std is None:
            continue
        y = rng.integers(0, 256, oracle.tiled_elements(lay) * lay["itemsize"], dtype=np.uint8)
        want = oracle.detile(lay, y)
        for nthreads in (1, 3, 8):
            got = oracle.detile_std(lay["itemsize"], *std, y, nthreads=nthreads)
            assert np.array_equal(got, want), (lay, nthreads)
        checked += 1
    assert checked >= 60
