"""GPU: kvx_manager_gather_no_alloc (tables in a fixed per-GPU device array,
no allocation) against kvx_manager_gather (tables in the library's argument
ring) through the C-ABI: identical staging bytes for the same ids, two calls
in a row on one stream (the second smaller, so it reuses the array the first
one filled), calls back to back on two streams and from two host threads
(ordered on the GPU through the per-device event), every staging order and
restriction, two block sizes in one launch (fp8 payload + scales), the size
limits and the id checks.
"""
import ctypes
import threading

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

MAX_IDS = 16384
MAX_STORAGES = 4096


def _pools(rng, cuda, layers, shards, blocks, bb):
    return [[torch.from_numpy(rng.integers(0, 256, (blocks, bb), dtype=np.uint8)).to(cuda)
             for _ in range(shards)] for _ in range(layers)]


def _stream_ptr(stream):
    return ctypes.c_void_p(stream.cuda_stream)


def _existing(kvx, mgr, ids, staging, order, layer, shard, stream):
    lib = kvx._capi.load()
    arr, n = kvx._capi.i64_array(ids)
    fut = ctypes.c_void_p()
    rc = lib.kvx_manager_gather(mgr._h, arr, n, staging.data_ptr(), staging.numel(), order,
                                layer, shard, _stream_ptr(stream), ctypes.byref(fut))
    assert rc == 0, kvx._capi.last_error()
    assert lib.kvx_future_await(fut) == 0
    lib.kvx_future_release(fut)


def _no_alloc(kvx, mgr, ids, staging, order, layer, shard, stream):
    lib = kvx._capi.load()
    arr, n = kvx._capi.i64_array(ids)
    return lib.kvx_manager_gather_no_alloc(mgr._h, arr, n, staging.data_ptr(), staging.numel(),
                                           order, layer, shard, _stream_ptr(stream))


def _bytes(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.parametrize("order,layer,shard", [(0, -1, -1), (1, -1, -1), (0, 2, -1),
                                               (0, -1, 1), (1, 1, 0)])
def test_no_alloc_matches_gather_two_calls(kvx, cuda, order, layer, shard):
    rng = np.random.default_rng(70 + 10 * order + layer + 3 * shard)
    layers, shards, blocks, bb = 4, 2, 200, 4096
    pools = _pools(rng, cuda, layers, shards, blocks, bb)
    mgr = kvx.KVCacheManager(pools, host_blocks_to_allocate=8)
    w = (1 if layer >= 0 else layers) * (1 if shard >= 0 else shards)
    stream = torch.cuda.Stream(cuda)
    ids1 = rng.choice(blocks, 150, replace=False)
    ids2 = rng.choice(blocks, 37, replace=False)
    want1 = torch.zeros(w * len(ids1) * bb, dtype=torch.uint8, device=cuda)
    want2 = torch.zeros(w * len(ids2) * bb, dtype=torch.uint8, device=cuda)
    _existing(kvx, mgr, ids1, want1, order, layer, shard, stream)
    _existing(kvx, mgr, ids2, want2, order, layer, shard, stream)
    got1 = torch.full_like(want1, 0x5A)
    got2 = torch.full((want1.numel() + 4096,), 0x5A, dtype=torch.uint8, device=cuda)
    # Back to back on one stream, no host wait: the second call refills the
    # array only after the first call's gather has read it.
    assert _no_alloc(kvx, mgr, ids1, got1, order, layer, shard, stream) == 0
    assert _no_alloc(kvx, mgr, ids2, got2, order, layer, shard, stream) == 0
    stream.synchronize()
    assert np.array_equal(_bytes(got1), _bytes(want1))
    g2 = _bytes(got2)
    assert np.array_equal(g2[:want2.numel()], _bytes(want2))
    assert (g2[want2.numel():] == 0x5A).all()
    mgr.close()


def test_no_alloc_two_streams_and_threads_are_ordered(kvx, cuda):
    """Calls alternating between two streams with no host wait, then two host
    threads issuing on their own streams at once: each gather moves 2 GiB, so
    a later call's fills would overwrite the shared array while an earlier
    gather still reads it unless the calls are ordered. Every output must
    equal kvx_manager_gather's for its ids."""
    gen = torch.Generator(device=cuda).manual_seed(90)
    W, blocks, bb, n = 16, 8192, 32768, 4096
    pools = [torch.randint(0, 256, (blocks, bb), dtype=torch.uint8, device=cuda, generator=gen)
             for _ in range(W)]
    mgr = kvx.KVCacheManager(pools, host_blocks_to_allocate=4)
    streams = [torch.cuda.Stream(cuda) for _ in range(2)]
    rng = np.random.default_rng(91)
    id_sets = [rng.choice(blocks, n, replace=False) for _ in range(4)]
    want = []
    for ids in id_sets:
        w = torch.zeros(W * n * bb, dtype=torch.uint8, device=cuda)
        _existing(kvx, mgr, ids, w, 0, -1, -1, streams[0])
        want.append(w)
    got = [torch.full((W * n * bb,), 0x5A, dtype=torch.uint8, device=cuda) for _ in range(4)]
    torch.cuda.synchronize()
    print("no-alloc: 4 calls alternating between 2 streams", flush=True)
    for k in range(4):
        assert _no_alloc(kvx, mgr, id_sets[k], got[k], 0, -1, -1, streams[k % 2]) == 0
    torch.cuda.synchronize()
    for k in range(4):
        assert torch.equal(got[k], want[k]), k
    print("no-alloc: 2 host threads, 2 calls each", flush=True)
    for g in got:
        g.fill_(0x5A)
    torch.cuda.synchronize()
    rcs = []

    def issue(t):
        for k in (t, t + 2):
            rcs.append(_no_alloc(kvx, mgr, id_sets[k], got[k], 0, -1, -1, streams[t]))

    threads = [threading.Thread(target=issue, args=(t,)) for t in range(2)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    torch.cuda.synchronize()
    assert rcs == [0, 0, 0, 0]
    for k in range(4):
        assert torch.equal(got[k], want[k]), k
    mgr.close()


def test_no_alloc_fp8_payload_and_scales(kvx, cuda):
    """Two block sizes (16 KiB payload, 32 B scales): two pieces of one launch."""
    rng = np.random.default_rng(81)
    layers, blocks, heads = 3, 300, 8
    kv = [torch.from_numpy(rng.integers(0, 256, (blocks, 16 * heads * 128),
                                        dtype=np.uint8)).to(cuda) for _ in range(2 * layers)]
    sc = [torch.from_numpy(rng.standard_normal((blocks, heads), dtype=np.float32)).to(cuda)
          for _ in range(layers)]
    mgr = kvx.KVCacheManager(kv, host_blocks_to_allocate=8, scale_tables=sc)
    stream = torch.cuda.Stream(cuda)
    for n in (257, 19):
        ids = rng.choice(blocks, n, replace=False)
        need = n * (2 * layers * 16 * heads * 128 + layers * heads * 4)
        want = torch.zeros(need, dtype=torch.uint8, device=cuda)
        got = torch.full((need,), 0xA5, dtype=torch.uint8, device=cuda)
        _existing(kvx, mgr, ids, want, 0, -1, -1, stream)
        assert _no_alloc(kvx, mgr, ids, got, 0, -1, -1, stream) == 0
        stream.synchronize()
        assert np.array_equal(_bytes(got), _bytes(want))
    mgr.close()


def test_no_alloc_at_its_limits(kvx, cuda):
    """16384 ids (64 fill launches) over 300 storages, then a 3-id call."""
    rng = np.random.default_rng(82)
    layers, shards, blocks, bb = 150, 2, MAX_IDS + 100, 64
    pools = _pools(rng, cuda, layers, shards, blocks, bb)
    mgr = kvx.KVCacheManager(pools, host_blocks_to_allocate=4)
    stream = torch.cuda.Stream(cuda)
    w = layers * shards
    for n in (MAX_IDS, 3):
        ids = rng.choice(blocks, n, replace=False)
        want = torch.zeros(w * n * bb, dtype=torch.uint8, device=cuda)
        got = torch.full_like(want, 0x11)
        _existing(kvx, mgr, ids, want, 0, -1, -1, stream)
        assert _no_alloc(kvx, mgr, ids, got, 0, -1, -1, stream) == 0
        stream.synchronize()
        assert np.array_equal(_bytes(got), _bytes(want))
    big = torch.empty(w * (MAX_IDS + 1) * bb, dtype=torch.uint8, device=cuda)
    rc = _no_alloc(kvx, mgr, np.arange(MAX_IDS + 1), big, 0, -1, -1, stream)
    assert rc == 3 and "scratch" in kvx._capi.last_error()
    mgr.close()


def test_no_alloc_rejects_before_launching(kvx, cuda):
    rng = np.random.default_rng(83)
    pools = _pools(rng, cuda, 2, 1, 64, 1024)
    mgr = kvx.KVCacheManager(pools, host_blocks_to_allocate=4)
    stream = torch.cuda.Stream(cuda)
    st = torch.full((2 * 8 * 1024,), 7, dtype=torch.uint8, device=cuda)
    assert _no_alloc(kvx, mgr, [1, -2], st, 0, -1, -1, stream) == 3
    assert "non-negative" in kvx._capi.last_error()
    assert _no_alloc(kvx, mgr, [1, 64], st, 0, -1, -1, stream) == 11
    assert _no_alloc(kvx, mgr, [1, 2], st, 0, 5, -1, stream) == 11
    assert _no_alloc(kvx, mgr, [1, 2], st, 7, -1, -1, stream) == 3
    small = torch.empty(3 * 1024, dtype=torch.uint8, device=cuda)
    assert _no_alloc(kvx, mgr, [1, 2], small, 0, -1, -1, stream) == 3
    assert "too small" in kvx._capi.last_error()
    assert _no_alloc(kvx, mgr, [], st, 0, -1, -1, stream) == 0
    stream.synchronize()
    assert (_bytes(st) == 7).all()
    mgr.close()
