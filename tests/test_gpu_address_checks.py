"""GPU: entry points that take a raw device buffer refuse host memory with
INVALID_ARGUMENT before anything is issued (the reference validates every
argument before issuing, tpu_sync/kv_cache/kv_cache_manager_base.cc:72-102).

The calls go straight to the C-ABI (the Python layer refuses CPU tensors
itself). The host buffers are pinned, so the GPU could reach them: a refusal
that was missed would show as changed host bytes, never as a fault. The
entry points callable without a device object are covered on the CPU with
made-up addresses (tests/device_address_check.cc)."""
import ctypes

import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


def _ids(n):
    return (ctypes.c_int64 * n)(*range(n))


def test_manager_device_copies_refuse_host_staging(kvx, cuda):
    pools = [torch.randint(0, 256, (64, 4096), dtype=torch.uint8, device=cuda) for _ in range(4)]
    mgr = kvx.KVCacheManager(pools, host_blocks_to_allocate=8)
    lib = kvx._capi.load()
    host = torch.full((4 * 8 * 4096,), 0x5A, dtype=torch.uint8).pin_memory()
    out = ctypes.c_void_p()
    for name in ("kvx_manager_gather", "kvx_manager_scatter"):
        rc = getattr(lib, name)(mgr._h, _ids(8), 8, host.data_ptr(), host.numel(), 0, -1, -1,
                                None, ctypes.byref(out))
        assert rc == 3, name
        assert b"staging: host memory" in lib.kvx_last_error(), name
    rc = lib.kvx_manager_gather_no_alloc(mgr._h, _ids(8), 8, host.data_ptr(), host.numel(), 0,
                                         -1, -1, None)
    assert rc == 3 and b"staging: host memory" in lib.kvx_last_error()
    torch.cuda.synchronize()
    assert bool((host == 0x5A).all())
    # A device buffer of the same size still works, and so does a range that
    # fits the allocation exactly.
    dev = torch.empty(4 * 8 * 4096, dtype=torch.uint8, device=cuda)
    mgr.gather(list(range(8)), dev).Await()
    assert torch.equal(dev.view(4, 8, 4096), torch.stack([p[:8] for p in pools]))
    # One byte short of the staging the gather writes: refused before issue.
    short = dev[:-1]
    with pytest.raises(kvx.KvxError):
        mgr.gather(list(range(8)), short).Await()
    mgr.close()


def test_weight_sync_pack_refuses_host_staging(kvx, cuda):
    ts = [torch.randint(0, 256, (1 << 16,), dtype=torch.uint8, device=cuda) for _ in range(3)]
    ws = kvx.WeightSynchronizer([[t] for t in ts])
    lib = kvx._capi.load()
    host = torch.full((ws.total_bytes,), 0x33, dtype=torch.uint8).pin_memory()
    out = ctypes.c_void_p()
    for name in ("kvx_weight_sync_pack", "kvx_weight_sync_unpack"):
        rc = getattr(lib, name)(ws._h, host.data_ptr(), host.numel(), None, ctypes.byref(out))
        assert rc == 3 and b"staging: host memory" in lib.kvx_last_error(), name
    torch.cuda.synchronize()
    assert bool((host == 0x33).all())
    ws.close()


def test_raw_kernels_and_tiling_refuse_host_buffers(kvx, cuda):
    lib = kvx._capi.load()
    W, n, bb = 2, 4, 4096
    pool = [torch.zeros(16, bb, dtype=torch.uint8, device=cuda) for _ in range(W)]
    table = torch.tensor([p.data_ptr() for p in pool], dtype=torch.int64, device=cuda)
    ids = torch.arange(n, dtype=torch.int64, device=cuda)
    host = torch.full((W * n * bb,), 0x77, dtype=torch.uint8).pin_memory()
    rc = lib.kvx_gather_blocks(table.data_ptr(), W, bb, 16, ids.data_ptr(), n, host.data_ptr(),
                               0, 0, None)
    assert rc == 3 and b"staging: host memory" in lib.kvx_last_error()
    L = kvx.tiling.TiledLayout(2, (16, 128), [(8, 128)])
    c = L.to_c()
    out = ctypes.c_void_p()
    dev = torch.zeros(L.tiled_bytes, dtype=torch.uint8, device=cuda)
    rc = lib.kvx_tile_buffer(0, ctypes.byref(c), host.data_ptr(), dev.data_ptr(), None,
                             ctypes.byref(out))
    assert rc == 3 and b"src_linear: host memory" in lib.kvx_last_error()
    torch.cuda.synchronize()
    assert bool((host == 0x77).all()) and not dev.any()
