"""GPU: weight-sync pack / D2H / H2D / unpack and strided (column-split)
copies, bit-exact against the numpy oracle (oracle/weight_sync.py), plus the
full Llama-3-8B parameter set (291 bf16 tensors, 16.06 GB) round trip and
8-way column split checked against torch slicing on the device."""
import numpy as np
import pytest

from oracle import weight_sync as W

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


def u8(t):
    torch.cuda.synchronize()
    return t.detach().cpu().contiguous().view(torch.uint8).numpy().reshape(-1)


def test_strided_copy_random_entries_match_oracle(kvx, cuda):
    """Random entries over every vector width (sizes/strides/offsets that are
    multiples of 16, 8, 4, 2 and 1 bytes), rows longer than one tile and many
    entries in one launch, against the oracle's expansion."""
    rng = np.random.default_rng(7)
    src_np = rng.integers(0, 256, 1 << 22, dtype=np.uint8)
    src = torch.from_numpy(src_np).to(cuda)
    for align in (16, 8, 4, 2, 1):
        dst = torch.zeros(1 << 22, dtype=torch.uint8, device=cuda)
        want = np.zeros(1 << 22, np.uint8)
        entries, ora = [], []
        dpos = 0
        for _ in range(int(rng.integers(1, 40))):
            size = int(rng.integers(1, 400)) * align
            count = int(rng.integers(1, 12))
            s_stride = size + int(rng.integers(0, 5)) * align
            d_stride = size + int(rng.integers(0, 3)) * align
            s_off = int(rng.integers(0, 1000)) * align
            if s_off + (count - 1) * s_stride + size > src_np.size:
                continue
            if dpos + (count - 1) * d_stride + size > want.size:
                break
            entries.append(kvx.StridedEntry(src.data_ptr() + s_off, dst.data_ptr() + dpos,
                                            size, count, s_stride, d_stride))
            ora.append((s_off, dpos, size, count, s_stride, d_stride))
            dpos += (count - 1) * d_stride + size
            dpos = (dpos + align - 1) // align * align
        # One long row spanning many 32 KiB tiles.
        long_n = 300_000 // align * align
        if dpos + long_n <= want.size:
            entries.append(kvx.StridedEntry(src.data_ptr() + 3 * align, dst.data_ptr() + dpos,
                                            long_n, 1, 0, 0))
            ora.append((3 * align, dpos, long_n, 1, 0, 0))
        kvx.copy_strided(entries, device=0).Await()
        W.apply_entries(src_np, want, ora)
        assert np.array_equal(u8(dst), want), align


def test_strided_copy_sliced_tile_groups_match_oracle(kvx, cuda):
    """At 16-byte vectors tiles move in groups of 32 (a workgroup takes 1 KiB
    of each tile of its group): long rows whose 32nd tile is partial, long
    rows with a group and leftover tiles in several strided rows, two
    groups; short-row entries whose 32nd tile holds fewer rows, one group
    and leftover tiles, rows that are not a multiple of 1 KiB. Long and
    short entries interleaved in one launch (long-row tiles are numbered
    first), through a per-call launch and a plan, against the oracle."""
    rng = np.random.default_rng(17)
    n = 64 << 20
    src_np = rng.integers(0, 256, n, dtype=np.uint8)
    src = torch.from_numpy(src_np).to(cuda)
    T = 32768
    shapes = [  # (size, count, extra source stride, extra destination stride)
        (3584, 284, 25088, 0),          # short: 9 rows a tile, 32 tiles, the last 5 rows
        (1024, 1030, 7168, 0),          # short: 32 rows a tile, 33 tiles
        (2000, 700, 48, 16),            # short: 16 rows a tile, 44 tiles
        (32 * T - 1600, 1, 0, 0),       # long: 32 tiles, the last partial
        (41 * T + 48, 3, 4096, 16),     # long: 42 tiles a row, three rows
        (64 * T, 1, 0, 0),              # long: two groups
        (T, 40, 16, 0),                 # one tile per row: short entry of 40 tiles
    ]
    order = rng.permutation(len(shapes))
    entries, ora = [], []
    s_pos = d_pos = 0
    for k in order:
        size, count, s_extra, d_extra = shapes[k]
        s_stride, d_stride = size + s_extra, size + d_extra
        ora.append((s_pos, d_pos, size, count, s_stride, d_stride))
        s_pos += ((count - 1) * s_stride + size + 4095) // 4096 * 4096
        d_pos += ((count - 1) * d_stride + size + 4095) // 4096 * 4096
    assert s_pos <= n and d_pos <= n
    want = np.zeros(n, np.uint8)
    W.apply_entries(src_np, want, ora)
    for use_plan in (False, True):
        dst = torch.zeros(n, dtype=torch.uint8, device=cuda)
        entries = [kvx.StridedEntry(src.data_ptr() + a, dst.data_ptr() + b, sz, c, ss, ds)
                   for a, b, sz, c, ss, ds in ora]
        if use_plan:
            plan = kvx.StridedPlan(entries)
            kvx.copy_strided(plan, device=0).Await()
            plan.close()
        else:
            kvx.copy_strided(entries, device=0).Await()
        assert np.array_equal(u8(dst), want), use_plan


def test_strided_plan_matches_oracle_on_every_run(kvx, cuda):
    """A StridedPlan's device table (uploaded once) gives the oracle's bytes on
    every run: random entries of each vector width, three runs into cleared
    outputs, runs on two streams at once (disjoint outputs), an empty plan,
    and a plan closed while its last run may still be in flight."""
    rng = np.random.default_rng(11)
    src_np = rng.integers(0, 256, 1 << 21, dtype=np.uint8)
    src = torch.from_numpy(src_np).to(cuda)
    streams = [torch.cuda.Stream(cuda), torch.cuda.Stream(cuda)]
    for align in (16, 8, 4, 2, 1):
        dsts = [torch.zeros(1 << 21, dtype=torch.uint8, device=cuda) for _ in range(2)]
        wants = [np.zeros(1 << 21, np.uint8) for _ in range(2)]
        plans = []
        for dst, want in zip(dsts, wants):
            entries, ora, dpos = [], [], 0
            for _ in range(int(rng.integers(2, 30))):
                size = int(rng.integers(1, 300)) * align
                count = int(rng.integers(1, 10))
                s_stride = size + int(rng.integers(0, 5)) * align
                d_stride = size + int(rng.integers(0, 3)) * align
                s_off = int(rng.integers(0, 1000)) * align
                if s_off + (count - 1) * s_stride + size > src_np.size:
                    continue
                if dpos + (count - 1) * d_stride + size > want.size:
                    break
                entries.append(kvx.StridedEntry(src.data_ptr() + s_off, dst.data_ptr() + dpos,
                                                size, count, s_stride, d_stride))
                ora.append((s_off, dpos, size, count, s_stride, d_stride))
                dpos += (count - 1) * d_stride + size
                dpos = (dpos + align - 1) // align * align
            W.apply_entries(src_np, want, ora)
            plans.append(kvx.StridedPlan(entries))
        for run in range(3):
            for dst in dsts:
                dst.zero_()
            torch.cuda.synchronize()
            futs = [kvx.copy_strided(p, stream=s, device=0) for p, s in zip(plans, streams)]
            for f in futs:
                f.Await()
            for dst, want in zip(dsts, wants):
                assert np.array_equal(u8(dst), want), (align, run)
        # Closing right after a run: the plan waits for it before freeing.
        dsts[0].zero_()
        torch.cuda.synchronize()
        kvx.copy_strided(plans[0], stream=streams[0], device=0)
        plans[0].close()
        assert np.array_equal(u8(dsts[0]), wants[0]), align
        plans[1].close()
    empty = kvx.StridedPlan([])
    kvx.copy_strided(empty, device=0).Await()  # no launch; completes at once
    empty.close()


def test_strided_plan_kernel_times(kvx, cuda):
    """A plan made with profile_kernels times each run's launch: launches,
    a positive duration and 2 x the bytes its entries move per run, counted
    while the copies stay byte-exact; reset drops the samples."""
    src = torch.randint(0, 256, (3 << 20,), dtype=torch.uint8, device=cuda)
    dst = torch.zeros_like(src)
    entries = [kvx.StridedEntry(src.data_ptr(), dst.data_ptr(), 1 << 20),
               kvx.StridedEntry(src.data_ptr() + (1 << 20), dst.data_ptr() + (1 << 20),
                                4096, 256, 4096, 4096)]
    per_run = (1 << 20) + 4096 * 256
    plan = kvx.StridedPlan(entries, profile_kernels=True)
    assert plan.kernel_times() == {"launches": 0, "total_ms": 0.0, "bytes": 0}
    s = torch.cuda.Stream(cuda)
    for _ in range(3):
        kvx.copy_strided(plan, stream=s, device=0).Await()
    kt = plan.kernel_times()
    assert kt["launches"] == 3 and kt["bytes"] == 3 * 2 * per_run and kt["total_ms"] > 0, kt
    assert plan.kernel_times(reset=True)["launches"] == 3
    assert plan.kernel_times()["launches"] == 0
    torch.cuda.synchronize()
    assert torch.equal(dst[:per_run], src[:per_run])
    assert not dst[per_run:].any()
    plain = kvx.StridedPlan(entries)
    kvx.copy_strided(plain, stream=s, device=0).Await()
    assert plain.kernel_times()["launches"] == 0
    plan.close()
    plain.close()


def _tensors(rng, cuda, sizes, dtype=torch.bfloat16):
    out = []
    for n in sizes:
        t = torch.from_numpy(rng.integers(0, 256, n, dtype=np.uint8)).to(cuda)
        out.append(t)
    return out


@pytest.mark.parametrize("chunk,host_alloc", [(0, "pinned"), (4096, "pinned"),
                                              (70_000, "pinned"), (70_000, "malloc")])
def test_weight_sync_round_trip_matches_oracle(kvx, cuda, chunk, host_alloc):
    """Tensors of awkward sizes (odd, sub-16-byte, multi-chunk); the host
    image must equal the oracle's pack at every tensor's offset, and h2d
    restores the device tensors after they are overwritten (pinned or
    pageable host image)."""
    rng = np.random.default_rng(8)
    sizes = [1, 7, 16, 250, 4096, 12345, 65536, 100_003, 3, 2048]
    ts = _tensors(rng, cuda, sizes)
    originals = [u8(t).copy() for t in ts]
    ws = kvx.WeightSynchronizer([[t] for t in ts], chunk_bytes=chunk, staging_chunks=2,
                                host_alloc=host_alloc)
    want, offs = W.pack(originals)
    assert ws.total_bytes == want.size
    ws.d2h().Await()
    img = ws.host_image()
    for o, t in zip(offs, originals):
        assert np.array_equal(img[o:o + t.size], t)
        assert ws.host_buffer_info(offs.index(o))[2] == o
    for i, t in enumerate(originals):
        assert np.array_equal(ws.get_host_buffer(i).numpy().view(np.uint8).reshape(-1), t)
    for t in ts:
        t.zero_()
    ws.h2d().Await()
    for t, want_t in zip(ts, originals):
        assert np.array_equal(u8(t), want_t)
    # Per-layer copies.
    ts[5].fill_(9)
    ws.d2h_layer(5).Await()
    assert np.all(ws.get_host_buffer(5).numpy().view(np.uint8) == 9)
    ws.host_image()[offs[6]:offs[6] + sizes[6]] = 42
    ws.h2d_layer(6).Await()
    assert np.all(u8(ts[6]) == 42)
    ws.close()


def test_weight_sync_device_pack_unpack(kvx, cuda):
    rng = np.random.default_rng(9)
    sizes = [8192, 8190, 1 << 20, 5, 300_000]
    ts = _tensors(rng, cuda, sizes)
    originals = [u8(t).copy() for t in ts]
    ws = kvx.WeightSynchronizer([[t] for t in ts])
    staging = torch.zeros(ws.total_bytes, dtype=torch.uint8, device=cuda)
    ws.pack(staging).Await()
    want, offs = W.pack(originals)
    got = u8(staging)
    for o, t in zip(offs, originals):
        assert np.array_equal(got[o:o + t.size], t)
    for t in ts:
        t.zero_()
    ws.unpack(staging).Await()
    for t, want_t in zip(ts, originals):
        assert np.array_equal(u8(t), want_t)
    with pytest.raises(kvx.KvxError):
        ws.pack(staging[:-1])
    ws.close()


def llama3_8b_shapes():
    h, kv, ffn, vocab, layers = 4096, 1024, 14336, 128256, 32
    shapes = [("embed_tokens", (vocab, h))]
    for i in range(layers):
        shapes += [(f"l{i}.input_layernorm", (h,)), (f"l{i}.q_proj", (h, h)),
                   (f"l{i}.k_proj", (kv, h)), (f"l{i}.v_proj", (kv, h)),
                   (f"l{i}.o_proj", (h, h)), (f"l{i}.post_attention_layernorm", (h,)),
                   (f"l{i}.gate_proj", (ffn, h)), (f"l{i}.up_proj", (ffn, h)),
                   (f"l{i}.down_proj", (h, ffn))]
    shapes += [("norm", (h,)), ("lm_head", (vocab, h))]
    return shapes


def test_llama3_8b_parameter_set_round_trip_and_column_split(kvx, cuda):
    shapes = llama3_8b_shapes()
    assert len(shapes) == 291
    assert sum(int(np.prod(s)) for _, s in shapes) == 8_030_261_248
    gen = torch.Generator(device=cuda).manual_seed(0)
    params = [torch.randn(s, generator=gen, device=cuda, dtype=torch.float32)
              .mul_(0.02).to(torch.bfloat16) for _, s in shapes]
    saved = [t.clone() for t in params]
    ws = kvx.WeightSynchronizer([[t] for t in params])
    assert ws.total_bytes >= 16_060_522_496
    ws.d2h().Await()
    # Spot-check the host copies of the largest and smallest tensors.
    for i in (0, 1, 290):
        h = ws.get_host_buffer(i)
        assert torch.equal(h.view(torch.int16), params[i].cpu().view(torch.int16))
    for t in params:
        t.zero_()
    ws.h2d().Await()
    torch.cuda.synchronize()
    for t, s in zip(params, saved):
        assert torch.equal(t.view(torch.int16), s.view(torch.int16))
    del saved
    # Column split of every 2-D weight into 8 chunks, one launch.
    mats = [t for t in params if t.dim() == 2]
    assert len(mats) == 226
    entries, outs = [], []
    for m in mats:
        bounds = kvx.compute_nd_shard_slices(tuple(m.shape), (1, 8))
        chunk = [torch.empty(m.shape[0], b[1][1] - b[1][0], dtype=m.dtype, device=cuda)
                 for b in bounds]
        entries += kvx.column_split_entries(m, chunk)
        outs.append((m, bounds, chunk))
    kvx.copy_strided(entries, device=0).Await()
    torch.cuda.synchronize()
    for m, bounds, chunk in outs:
        for b, c in zip(bounds, chunk):
            assert torch.equal(c.view(torch.int16), m[:, b[1][0]:b[1][1]].view(torch.int16))
    # The same split again through a prepared plan, twice, into cleared outputs.
    plan = kvx.StridedPlan(entries)
    for _ in range(2):
        for _, _, chunk in outs:
            for c in chunk:
                c.zero_()
        kvx.copy_strided(plan, device=0).Await()
        torch.cuda.synchronize()
        for m, bounds, chunk in outs:
            for b, c in zip(bounds, chunk):
                assert torch.equal(c.view(torch.int16), m[:, b[1][0]:b[1][1]].view(torch.int16))
    ws.close()
