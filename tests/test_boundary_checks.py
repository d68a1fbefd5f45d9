"""The Python boundary checks every tensor it hands to a kernel before any
library call: a tensor off the HIP device, on another device than the
manager, non-contiguous or expanded, or spanning more bytes than its storage
is rejected with ValueError; a column split also needs a contiguous 2-D
weight and outputs of the weight's dtype. Tensors that claim to be on a
device are CPU tensors behind a wrapper: the checks run on the host only."""
import ctypes

import pytest

torch = pytest.importorskip("torch")

from fake_device import FakeDeviceTensor  # noqa: E402



class ShortStorage(FakeDeviceTensor):
    def untyped_storage(self):
        class S:
            def nbytes(self):
                return 8
        return S()


def test_device_buffer_accepts_a_contiguous_device_tensor(kvx):
    t = torch.empty(16, dtype=torch.float32)[4:]
    ptr, nbytes = kvx._capi.device_buffer(FakeDeviceTensor(t), "x", 0)
    assert ptr == t.data_ptr() and nbytes == 48


@pytest.mark.parametrize("make,msg", [
    (lambda: torch.empty(4), "HIP device"),
    (lambda: FakeDeviceTensor(torch.empty(4), index=1), "device 1"),
    (lambda: FakeDeviceTensor(torch.empty(1).expand(4096)), "contiguous"),
    (lambda: FakeDeviceTensor(torch.empty(8, 8).t()), "contiguous"),
    (lambda: ShortStorage(torch.empty(64, dtype=torch.uint8)), "storage holds 8"),
])
def test_device_buffer_rejects(kvx, make, msg):
    with pytest.raises(ValueError, match=msg):
        kvx._capi.device_buffer(make(), "x", 0)


def test_manager_rejects_host_and_mixed_device_pools(kvx):
    with pytest.raises(ValueError, match="HIP device"):
        kvx.KVCacheManager([torch.zeros(8, 64)], host_blocks_to_allocate=2)
    pools = [FakeDeviceTensor(torch.zeros(8, 64)), FakeDeviceTensor(torch.zeros(8, 64), 1)]
    with pytest.raises(ValueError, match="device 1"):
        kvx.KVCacheManager(pools, host_blocks_to_allocate=2)


def test_gather_and_scatter_reject_host_staging(kvx):
    mgr = kvx.KVCacheManager.create_host_only_for_testing(
        num_layers=2, slice_byte_size=64, host_blocks=4)
    for fn in (mgr.gather, mgr.scatter):
        with pytest.raises(ValueError, match="HIP device"):
            fn([0, 1], torch.empty(256, dtype=torch.uint8), stream=0)
        with pytest.raises(ValueError, match="contiguous"):
            fn([0], FakeDeviceTensor(torch.empty(1, dtype=torch.uint8).expand(256)), stream=0)
    mgr.close()


def test_column_split_entries_checks_weight_and_outputs(kvx):
    ws = kvx.weight_synchronizer
    w = torch.zeros(4, 8, dtype=torch.bfloat16)
    outs = [FakeDeviceTensor(torch.zeros(4, 4, dtype=torch.bfloat16)) for _ in range(2)]
    with pytest.raises(ValueError, match="HIP device"):
        ws.column_split_entries(w, outs)
    with pytest.raises(ValueError, match="contiguous"):
        ws.column_split_entries(FakeDeviceTensor(torch.zeros(8, 4, dtype=torch.bfloat16).t()),
                                outs)
    with pytest.raises(ValueError, match="dtype"):
        ws.column_split_entries(FakeDeviceTensor(w),
                                [FakeDeviceTensor(torch.zeros(4, 4, dtype=torch.float32))] * 2)
    with pytest.raises(ValueError, match="device 1"):
        ws.column_split_entries(FakeDeviceTensor(w),
                                [outs[0], FakeDeviceTensor(torch.zeros(4, 4, dtype=torch.bfloat16), 1)])
    with pytest.raises(ValueError, match="2-D"):
        ws.column_split_entries(FakeDeviceTensor(torch.zeros(8, dtype=torch.bfloat16)), outs)
    entries = ws.column_split_entries(FakeDeviceTensor(w), outs)
    assert [e.as_tuple() for e in entries] == [
        (w.data_ptr(), outs[0].data_ptr(), 8, 4, 16, 8),
        (w.data_ptr() + 8, outs[1].data_ptr(), 8, 4, 16, 8)]


def test_weight_synchronizer_rejects_host_tensors_and_staging(kvx):
    with pytest.raises(ValueError, match="HIP device"):
        kvx.WeightSynchronizer([[torch.zeros(16)]])
    ws = kvx.WeightSynchronizer.__new__(kvx.WeightSynchronizer)
    ws._device = 0
    for fn in (ws.pack, ws.unpack):
        with pytest.raises(ValueError, match="HIP device"):
            fn(torch.empty(64, dtype=torch.uint8), stream=0)
        with pytest.raises(ValueError, match="device 1"):
            fn(FakeDeviceTensor(torch.empty(64, dtype=torch.uint8), 1), stream=0)


@pytest.mark.parametrize("mode,threads,ok", [(3, 0, True), (3, 4, True), (3, -1, False),
                                             (4, 0, False), (-1, 0, False)])
def test_transfer_mode_validated_at_create(kvx, mode, threads, ok):
    """KVX_MODE_LANES needs the lanes' host threads; modes outside 0..3 are
    rejected before anything is allocated."""
    lib = kvx._capi.load()
    cfg = kvx._capi.ManagerConfig()
    cfg.num_layers, cfg.num_shards = 1, 1
    cfg.slice_byte_size, cfg.host_blocks = 64, 4
    cfg.host_alloc = kvx._capi.HOST_MALLOC
    cfg.transfer_mode = mode
    cfg.host_copy_threads = threads
    m = ctypes.c_void_p()
    rc = lib.kvx_manager_create(ctypes.byref(cfg), ctypes.byref(m))
    if ok:
        assert rc == 0, lib.kvx_last_error()
        lib.kvx_manager_destroy(m)
    else:
        assert rc == 3 and not m.value


@pytest.mark.parametrize("cap,ok", [(-1, True), (0, True), (1, True), (32, True), (-2, False),
                                    (33, False)])
def test_gather_workgroups_per_cu_validated_at_create(kvx, cap, ok):
    lib = kvx._capi.load()
    cfg = kvx._capi.ManagerConfig()
    cfg.num_layers, cfg.num_shards = 1, 1
    cfg.slice_byte_size, cfg.host_blocks = 64, 4
    cfg.host_alloc = kvx._capi.HOST_MALLOC
    cfg.gather_workgroups_per_cu = cap
    m = ctypes.c_void_p()
    rc = lib.kvx_manager_create(ctypes.byref(cfg), ctypes.byref(m))
    if ok:
        assert rc == 0, lib.kvx_last_error()
        lib.kvx_manager_destroy(m)
    else:
        assert rc == 3 and not m.value


def test_strided_plan_validates_entries_before_the_device(kvx):
    """kvx_strided_plan_create rejects what kvx_copy_strided rejects (empty
    rows, negative strides, overlapping destination rows, a null array) with
    INVALID_ARGUMENT before it touches a device; an empty plan needs none."""
    lib = kvx._capi.load()

    def create(entries, n=None):
        arr = (kvx._capi.StridedEntryC * max(len(entries), 1))()
        for a, e in zip(arr, entries):
            a.src, a.dst, a.size_bytes, a.count, a.src_stride_bytes, a.dst_stride_bytes = e
        p = ctypes.c_void_p()
        rc = lib.kvx_strided_plan_create(0, arr, len(entries) if n is None else n,
                                         ctypes.byref(p))
        return rc, p

    for bad in [(1, 2, 0, 1, 0, 0), (1, 2, 64, 1, -1, 0), (1, 2, 64, 3, 64, 32)]:
        rc, p = create([bad])
        assert rc == 3 and not p.value, bad
        assert lib.kvx_last_error()
    rc, p = create([], n=-1)
    assert rc == 3 and not p.value
    rc, p = create([])
    assert rc == 0 and p.value
    lib.kvx_strided_plan_destroy(p)
    assert lib.kvx_strided_plan_create(0, None, 0, None) == 3


def test_tile_entry_points_reject_bad_tensors(kvx):
    """tile_buffer / detile_buffer check both tensors (device, contiguity)
    and their sizes against the layout before any library call."""
    L = kvx.tiling.TiledLayout(2, (16, 256), [(8, 128), (2, 1)])
    lin = FakeDeviceTensor(torch.empty(16 * 256, dtype=torch.int16))
    til = FakeDeviceTensor(torch.empty(L.tiled_bytes // 2, dtype=torch.int16))
    for fn in (kvx.tiling.tile_buffer, kvx.tiling.detile_buffer):
        with pytest.raises(ValueError, match="HIP device"):
            fn(L, torch.empty(16 * 256, dtype=torch.int16), til) if fn is kvx.tiling.tile_buffer \
                else fn(L, til, torch.empty(16 * 256, dtype=torch.int16))
        short = FakeDeviceTensor(torch.empty(16 * 256 - 1, dtype=torch.int16))
        with pytest.raises(ValueError, match="linear buffer holds"):
            fn(L, short, til) if fn is kvx.tiling.tile_buffer else fn(L, til, short)
        with pytest.raises(ValueError, match="tiled buffer holds"):
            fn(L, lin, short) if fn is kvx.tiling.tile_buffer else fn(L, short, lin)
        with pytest.raises(ValueError, match="contiguous"):
            bad = FakeDeviceTensor(torch.empty(256, 32, dtype=torch.int16).t())
            fn(L, bad, til) if fn is kvx.tiling.tile_buffer else fn(L, til, bad)


def test_weight_sync_layouts_must_match_the_tensors(kvx):
    L = kvx.tiling.TiledLayout(2, (16, 256), [(8, 128), (2, 1)])
    t = FakeDeviceTensor(torch.empty(L.tiled_bytes, dtype=torch.uint8))
    with pytest.raises(RuntimeError, match="layouts must match"):
        kvx.WeightSynchronizer([[t], [t]], layouts=[[L]])
    with pytest.raises(RuntimeError, match="layouts must match"):
        kvx.WeightSynchronizer([[t, t]], layouts=[[L]])


def test_link_peaks_validate_arguments_before_the_device(kvx):
    """kvx_measure_link_peaks rejects a null output, zero or more than 16 GiB
    of bytes and reps outside 1..1000 with INVALID_ARGUMENT before it touches
    a device."""
    lib = kvx._capi.load()
    out = (ctypes.c_double * 3)()
    for nbytes, reps in [(0, 5), ((16 << 30) + 1, 5), (1 << 20, 0), (1 << 20, 1001),
                         (1 << 20, -1)]:
        assert lib.kvx_measure_link_peaks(nbytes, reps, out, None) == 3, (nbytes, reps)
        assert lib.kvx_last_error()
    assert lib.kvx_measure_link_peaks(1 << 20, 5, None, None) == 3
    with pytest.raises(kvx.KvxError):
        kvx.measure_link_peaks(0, 5)
