"""GPU: tiled layouts (tile / detile in HBM) bit-exact against the oracle
(XLA nested tiling element by element, oracle/kvx_oracle.c), on every
reference tiling test case, on random standard layouts over every vector
width, packing and padding, on random general layouts, with misaligned
buffers, at a full Llama-3-8B MLP weight's size, and through the weight
synchronizer (chunked D2h / H2d with chunk boundaries inside tiled tensors,
per-layer copies, device pack / unpack)."""
import json
import os

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NP = {1: np.uint8, 2: np.uint16, 4: np.uint32, 8: np.uint64}


def golden_layouts():
    with open(os.path.join(ROOT, "tests", "golden", "tiling_cases.json")) as f:
        cases = json.load(f)["cases"]
    size = {"f32": 4, "bf16": 2, "s8": 1}
    return [(c["name"], dict(itemsize=size[c["dtype"]], dims=c["dims"],
                             minor_to_major=c["minor_to_major"], tiles=c["tiles"]))
            for c in cases]


def random_standard_layouts(seed=3, n=40):
    """Row-major layouts with one (tH, tW) tile, optionally a (P, 1) packing
    (P = 2 for 2-byte, 4 for 1-byte elements): widths chosen so the row and
    tile widths allow 16, 8, 4, 2 and 1-byte vectors, heights and widths with
    and without padding, 1 to 3 batch dimensions."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        itemsize = int(rng.choice([1, 2, 4, 8]))
        packed = itemsize in (1, 2) and rng.random() < 0.5
        P = 4 // itemsize if packed else 1
        tH = int(rng.choice([1, 2, 4, 8, 16])) * P if packed else int(rng.choice([1, 2, 3, 4, 8]))
        tW = int(rng.choice([1, 3, 8, 16, 64, 128]))
        W = int(rng.integers(1, 5)) * tW + int(rng.choice([0, 0, 1, 3, int(rng.integers(1, 200))]))
        H = int(rng.integers(1, 40))
        batch = [int(rng.integers(1, 4)) for _ in range(int(rng.integers(0, 3)))]
        dims = batch + [H, W]
        tiles = [[tH, tW]] + ([[P, 1]] if packed else [])
        out.append((f"std{i}", dict(itemsize=itemsize, dims=dims,
                                    minor_to_major=list(range(len(dims) - 1, -1, -1)),
                                    tiles=tiles)))
    # 1-D tensors, as norms are stored.
    out.append(("norm1d", dict(itemsize=2, dims=[4096], minor_to_major=[0],
                               tiles=[[8, 128], [2, 1]])))
    out.append(("norm1d_pad", dict(itemsize=4, dims=[1000], minor_to_major=[0],
                                   tiles=[[8, 128]])))
    return out


def random_general_layouts(seed=5, n=40):
    """Any permutation, 1-3 tiles of rank 1-3 (including packings that do not
    match the element size), ranks 1-4."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        rank = int(rng.integers(1, 5))
        dims = [int(rng.integers(1, 24)) for _ in range(rank)]
        mtm = [int(v) for v in rng.permutation(rank)]
        tiles = [[int(rng.integers(1, 9)) for _ in range(int(rng.integers(1, 4)))]
                 for _ in range(int(rng.integers(1, 4)))]
        out.append((f"gen{i}", dict(itemsize=int(rng.choice([1, 2, 4, 8])), dims=dims,
                                    minor_to_major=mtm, tiles=tiles)))
    out.append(("bf16_pack4", dict(itemsize=2, dims=[16, 256], minor_to_major=[1, 0],
                                   tiles=[[8, 128], [4, 1]])))
    out.append(("f32_pack2", dict(itemsize=4, dims=[10, 100], minor_to_major=[1, 0],
                                  tiles=[[8, 128], [2, 1]])))
    return out


def as_layout(kvx, lay):
    return kvx.tiling.TiledLayout(lay["itemsize"], lay["dims"], lay["tiles"],
                                  lay["minor_to_major"])


def u8(t):
    torch.cuda.synchronize()
    return t.detach().cpu().contiguous().view(torch.uint8).numpy().reshape(-1)


def check_layout(kvx, oracle, cuda, lay, rng, lin_off=0, tiled_off=0):
    """tile_buffer and detile_buffer against the oracle; the tiled buffer
    starts filled with 0xA5 so padding must be written; buffers may start
    lin_off / tiled_off bytes into their allocations."""
    L = as_layout(kvx, lay)
    nlin, ntil = L.logical_bytes, L.tiled_bytes
    x = rng.integers(0, 256, nlin, dtype=np.uint8)
    lin_all = torch.zeros(nlin + lin_off + 64, dtype=torch.uint8, device=cuda)
    lin_all[lin_off:lin_off + nlin] = torch.from_numpy(x).to(cuda)
    lin = lin_all[lin_off:lin_off + nlin]
    til_all = torch.full((ntil + tiled_off + 64,), 0xA5, dtype=torch.uint8, device=cuda)
    til = til_all[tiled_off:tiled_off + ntil]
    kvx.tiling.tile_buffer(L, lin, til).Await()
    want = oracle.tile(lay, x)
    assert np.array_equal(u8(til), want), lay
    # Bytes around the buffers are untouched.
    assert not u8(lin_all[:lin_off]).any() and not u8(lin_all[lin_off + nlin:]).any()
    assert (u8(til_all[:tiled_off]) == 0xA5).all() and (u8(til_all[tiled_off + ntil:]) == 0xA5).all()
    # Detile a tiled buffer whose padding holds garbage: it must not leak.
    y = rng.integers(0, 256, ntil, dtype=np.uint8)
    til.copy_(torch.from_numpy(y).to(cuda))
    out_all = torch.full((nlin + lin_off + 64,), 0x5A, dtype=torch.uint8, device=cuda)
    out = out_all[lin_off:lin_off + nlin]
    kvx.tiling.detile_buffer(L, til, out).Await()
    assert np.array_equal(u8(out), oracle.detile(lay, y)), lay
    assert (u8(out_all[:lin_off]) == 0x5A).all() and (u8(out_all[lin_off + nlin:]) == 0x5A).all()


@pytest.mark.parametrize("name,lay", golden_layouts(), ids=[n for n, _ in golden_layouts()])
def test_reference_cases_match_oracle(kvx, oracle, cuda, name, lay):
    print("tiling case", name, flush=True)
    check_layout(kvx, oracle, cuda, lay, np.random.default_rng(1))


def test_random_standard_layouts_match_oracle(kvx, oracle, cuda):
    rng = np.random.default_rng(2)
    for name, lay in random_standard_layouts():
        print("tiling case", name, lay, flush=True)
        check_layout(kvx, oracle, cuda, lay, rng)


def test_random_general_layouts_match_oracle(kvx, oracle, cuda):
    rng = np.random.default_rng(4)
    for name, lay in random_general_layouts():
        print("tiling case", name, lay, flush=True)
        check_layout(kvx, oracle, cuda, lay, rng)


def test_misaligned_buffers_match_oracle(kvx, oracle, cuda):
    """Buffers 1-8 bytes past a 256-byte boundary narrow the vectors (a packed
    layout below 4-byte vectors goes element by element); buffers that are not
    aligned to the element size are refused."""
    rng = np.random.default_rng(6)
    lays = [dict(itemsize=2, dims=[40, 384], minor_to_major=[1, 0], tiles=[[8, 128], [2, 1]]),
            dict(itemsize=1, dims=[40, 384], minor_to_major=[1, 0], tiles=[[8, 128], [4, 1]]),
            dict(itemsize=4, dims=[3, 20, 200], minor_to_major=[2, 1, 0], tiles=[[8, 128]])]
    for lay in lays:
        for lo, to in [(2, 0), (0, 2), (4, 8), (8, 4), (1, 0), (0, 1)]:
            print("tiling case misaligned", lay, lo, to, flush=True)
            if lo % lay["itemsize"] or to % lay["itemsize"]:
                # Below the element size: refused on the host before any launch.
                check_misaligned_refused(kvx, cuda, lay, lo, to)
                continue
            check_layout(kvx, oracle, cuda, lay, rng, lin_off=lo, tiled_off=to)


def check_misaligned_refused(kvx, cuda, lay, lin_off, tiled_off):
    """tile_buffer / detile_buffer with a buffer that is not aligned to the
    element size return INVALID_ARGUMENT and leave both buffers untouched."""
    L = as_layout(kvx, lay)
    lin_all = torch.full((L.logical_bytes + lin_off,), 0x11, dtype=torch.uint8, device=cuda)
    til_all = torch.full((L.tiled_bytes + tiled_off,), 0x22, dtype=torch.uint8, device=cuda)
    lin = lin_all[lin_off:]
    til = til_all[tiled_off:]
    for fn, args in ((kvx.tiling.tile_buffer, (L, lin, til)),
                     (kvx.tiling.detile_buffer, (L, til, lin))):
        with pytest.raises(kvx.KvxError) as e:
            fn(*args).Await()
        assert e.value.code == 3, e.value
    assert (u8(lin_all) == 0x11).all() and (u8(til_all) == 0x22).all()


def numpy_tile_2d(x, tH, tW, P=1):
    *batch, H, W = x.shape
    nT0, nT1 = -(-H // tH), -(-W // tW)
    pad = np.zeros(tuple(batch) + (nT0 * tH, nT1 * tW), x.dtype)
    pad[..., :H, :W] = x
    t = np.moveaxis(pad.reshape(tuple(batch) + (nT0, tH, nT1, tW)), -3, -2)
    if P > 1:
        t = np.swapaxes(t.reshape(t.shape[:-2] + (tH // P, P, tW)), -1, -2)
    return np.ascontiguousarray(t).reshape(-1)


def test_full_size_mlp_weight(kvx, cuda):
    """A Llama-3-8B gate projection ([14336, 4096] bf16) in T(8,128)(2,1):
    tile on the device, compare with the numpy formulation, detile back."""
    gen = torch.Generator(device=cuda).manual_seed(0)
    w = torch.randint(-32768, 32767, (14336, 4096), dtype=torch.int16, device=cuda,
                      generator=gen)
    L = kvx.tiling.TiledLayout(2, (14336, 4096), [(8, 128), (2, 1)])
    til = torch.empty(L.tiled_bytes // 2, dtype=torch.int16, device=cuda)
    kvx.tiling.tile_buffer(L, w, til).Await()
    want = numpy_tile_2d(w.cpu().numpy().view(np.uint16), 8, 128, 2)
    assert np.array_equal(til.cpu().numpy().view(np.uint16), want)
    back = torch.empty_like(w)
    kvx.tiling.detile_buffer(L, til, back).Await()
    assert torch.equal(back, w)


@pytest.mark.parametrize("itemsize,P,H,W", [(2, 2, 2050, 2048), (1, 4, 1030, 4096),
                                           (2, 2, 2103, 2048), (1, 4, 1061, 4096)])
def test_detile_sliced_slot_groups(kvx, cuda, itemsize, P, H, W):
    """Detiling packed layouts at 16-byte rows takes its slots sliced over
    groups of 8 workgroups: shapes with whole groups and a last group of 1-7
    workgroups (and rows past the matrix in the last tile row). The tiled
    bytes come from the numpy formulation of the tiling; the detiled matrix
    must equal the original, and tiling it back the numpy bytes."""
    rng = np.random.default_rng(H + W + P)
    dt = np.uint16 if itemsize == 2 else np.uint8
    x = rng.integers(0, 1 << (8 * itemsize), (H, W), dtype=dt)
    L = kvx.tiling.TiledLayout(itemsize, (H, W), [(8, 128), (P, 1)])
    tiled_np = numpy_tile_2d(x, 8, 128, P)
    assert tiled_np.nbytes == L.tiled_bytes
    til = torch.from_numpy(tiled_np.view(np.uint8).copy()).to(cuda)
    out = torch.zeros(H * W * itemsize, dtype=torch.uint8, device=cuda)
    kvx.tiling.detile_buffer(L, til, out).Await()
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(dt).reshape(H, W), x)
    back = torch.full((L.tiled_bytes,), 0x5A, dtype=torch.uint8, device=cuda)
    kvx.tiling.tile_buffer(L, out, back).Await()
    torch.cuda.synchronize()
    assert np.array_equal(back.cpu().numpy(), tiled_np.view(np.uint8))


def _sync_set(kvx, cuda, rng):
    """Mixed weights: tiled (packed bf16, packed int8, f32, general permuted,
    1-D) and row-major; device tensors hold the tiled bytes."""
    lays = [dict(itemsize=2, dims=[300, 1000], minor_to_major=[1, 0], tiles=[[8, 128], [2, 1]]),
            None,
            dict(itemsize=1, dims=[257, 640], minor_to_major=[1, 0], tiles=[[8, 128], [4, 1]]),
            dict(itemsize=4, dims=[3, 100, 130], minor_to_major=[2, 1, 0], tiles=[[8, 128]]),
            dict(itemsize=2, dims=[6, 40, 96], minor_to_major=[2, 0, 1], tiles=[[8, 128], [2, 1]]),
            dict(itemsize=2, dims=[4096], minor_to_major=[0], tiles=[[8, 128], [2, 1]]),
            None]
    tensors, layouts = [], []
    for lay in lays:
        if lay is None:
            n = int(rng.integers(1000, 300000))
            tensors.append(torch.from_numpy(rng.integers(0, 256, n, dtype=np.uint8)).to(cuda))
            layouts.append(None)
        else:
            L = as_layout(kvx, lay)
            tensors.append(torch.from_numpy(
                rng.integers(0, 256, L.tiled_bytes, dtype=np.uint8)).to(cuda))
            layouts.append(L)
    return lays, tensors, layouts


@pytest.mark.parametrize("chunk", [64 << 10, 200 << 10, 0])
def test_weight_sync_tiled_tensors(kvx, oracle, cuda, chunk):
    """D2h detiles every tiled weight into its host copy and H2d tiles it back
    (padding zero) through staging chunks of 64 KiB, 200 KiB and the default,
    so tiled weights straddle chunk boundaries; row-major weights move as
    before; per-layer copies and the device pack / unpack agree."""
    rng = np.random.default_rng(chunk + 1)
    lays, tensors, layouts = _sync_set(kvx, cuda, rng)
    ws = kvx.WeightSynchronizer([[t] for t in tensors], layouts=[[l] for l in layouts],
                                chunk_bytes=chunk)
    dev0 = [u8(t) for t in tensors]
    ws.d2h().Await()

    def want_host(k, dev):
        return oracle.detile(lays[k], dev) if lays[k] is not None else dev

    for k in range(len(tensors)):
        ptr, n, off = ws.host_buffer_info(k, 0)
        got = ws.host_image()[off:off + n]
        assert np.array_equal(got, want_host(k, dev0[k])), k
    # New host bytes -> H2d -> device tiled bytes with zero padding.
    img = ws.host_image()
    new = {}
    for k in range(len(tensors)):
        _, n, off = ws.host_buffer_info(k, 0)
        new[k] = rng.integers(0, 256, n, dtype=np.uint8)
        img[off:off + n] = new[k]
        tensors[k].fill_(0xA5)
    ws.h2d().Await()
    for k in range(len(tensors)):
        want = oracle.tile(lays[k], new[k]) if lays[k] is not None else new[k]
        assert np.array_equal(u8(tensors[k]), want), k
    # Per-layer copies of each tiled weight.
    for k in (0, 3, 4):
        img[ws.host_buffer_info(k, 0)[2]:][:ws.host_buffer_info(k, 0)[1]] = 0
        ws.d2h_layer(k).Await()
        _, n, off = ws.host_buffer_info(k, 0)
        assert np.array_equal(img[off:off + n], new[k]), k
        tensors[k].fill_(0x11)
        ws.h2d_layer(k).Await()
        assert np.array_equal(u8(tensors[k]), oracle.tile(lays[k], new[k])), k
    # Device pack / unpack against the same host image.
    staging = torch.zeros(ws.total_bytes, dtype=torch.uint8, device=cuda)
    ws.pack(staging).Await()
    for k in range(len(tensors)):
        _, n, off = ws.host_buffer_info(k, 0)
        assert np.array_equal(u8(staging)[off:off + n], new[k]), k
    for t in tensors:
        t.fill_(0x77)
    ws.unpack(staging).Await()
    for k in range(len(tensors)):
        want = oracle.tile(lays[k], new[k]) if lays[k] is not None else new[k]
        assert np.array_equal(u8(tensors[k]), want), k
    # The host view of a tiled weight has its logical shape.
    assert tuple(ws.get_host_buffer(0, 0).shape) == (300, 1000)
    ws.close()


def test_weight_sync_odd_tile_row_cuts_keep_alignment(kvx, oracle, cuda):
    """4 KiB staging chunks over an int8 weight whose tile rows are 301 bytes:
    the chunk cuts fall on odd byte offsets (3913, 7826, 11739), and the
    chunk starting at 11739 holds a whole f32 tiled weight (host offset
    12288) and the head of a packed bf16 one. Each chunk sits in its staging
    buffer at its start's offset modulo 256, so those weights stay 256-byte
    aligned in staging; both directions match the oracle."""
    rng = np.random.default_rng(11)
    lays = [dict(itemsize=1, dims=[40, 301], minor_to_major=[1, 0], tiles=[[1, 128]]),
            dict(itemsize=4, dims=[8, 64], minor_to_major=[1, 0], tiles=[[2, 64]]),
            dict(itemsize=2, dims=[16, 128], minor_to_major=[1, 0], tiles=[[2, 128], [2, 1]]),
            None]
    tensors, layouts = [], []
    for lay in lays:
        L = as_layout(kvx, lay) if lay is not None else None
        n = L.tiled_bytes if L is not None else 1000
        tensors.append(torch.from_numpy(rng.integers(0, 256, n, dtype=np.uint8)).to(cuda))
        layouts.append(L)
    ws = kvx.WeightSynchronizer([[t] for t in tensors], layouts=[[l] for l in layouts],
                                chunk_bytes=4096)
    assert [ws.host_buffer_info(k, 0)[2] for k in range(4)] == [0, 12288, 14336, 18432]
    dev0 = [u8(t) for t in tensors]
    ws.d2h().Await()
    img = ws.host_image()
    for k in range(4):
        _, n, off = ws.host_buffer_info(k, 0)
        want = oracle.detile(lays[k], dev0[k]) if lays[k] is not None else dev0[k]
        assert np.array_equal(img[off:off + n], want), k
    new = {}
    for k in range(4):
        _, n, off = ws.host_buffer_info(k, 0)
        new[k] = rng.integers(0, 256, n, dtype=np.uint8)
        img[off:off + n] = new[k]
        tensors[k].fill_(0xA5)
    ws.h2d().Await()
    for k in range(4):
        want = oracle.tile(lays[k], new[k]) if lays[k] is not None else new[k]
        assert np.array_equal(u8(tensors[k]), want), k
    ws.close()


def test_weight_sync_rejects_small_tiled_buffers_and_chunks(kvx, cuda):
    L = kvx.tiling.TiledLayout(2, (300, 1000), [(8, 128), (2, 1)])
    small = torch.zeros(L.tiled_bytes - 2, dtype=torch.uint8, device=cuda)
    with pytest.raises(kvx.KvxError, match="smaller than its tiled layout"):
        kvx.WeightSynchronizer([[small]], layouts=[[L]])
    ok = torch.zeros(L.tiled_bytes, dtype=torch.uint8, device=cuda)
    with pytest.raises(kvx.KvxError, match="tile row"):
        kvx.WeightSynchronizer([[ok]], layouts=[[L]], chunk_bytes=2000)
