"""GPU: queued D2h/H2d dispatch moves the same bytes as inline dispatch
(against numpy indexing of the pools), honours the caller's stream as of the
submission (a copy submitted behind a fill on a torch stream sees the fill),
reports validation errors through the future, and a reload's future can make
a torch stream wait before its copy has even been issued."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


def u8(t):
    torch.cuda.synchronize()
    return t.detach().cpu().view(torch.uint8).numpy().reshape(t.shape[0], -1).copy()


def test_queued_round_trip_matches_inline(kvx, cuda):
    rng = np.random.default_rng(41)
    host = [rng.integers(0, 256, (64, 8192), dtype=np.uint8) for _ in range(4)]
    dev = [torch.from_numpy(h).to(cuda) for h in host]
    mgr = kvx.KVCacheManager(dev, host_blocks_to_allocate=32, dispatch="queued")
    assert mgr.queued_dispatch
    src = [int(x) for x in rng.choice(64, 20, replace=False)]
    futs = [mgr.d2h(src[:10], list(range(10))), mgr.d2h(src[10:], list(range(10, 20)))]
    for f in futs:
        f.Await()
    for l in range(4):
        assert np.array_equal(mgr.host_view(l).reshape(32, 8192)[:20], host[l][src])
    dst = [int(x) for x in rng.choice(64, 20, replace=False)]
    before = [u8(t) for t in dev]
    mgr.h2d(list(range(20)), dst).Await()
    for l in range(4):
        want = before[l].copy()
        want[dst] = host[l][src]
        assert np.array_equal(u8(dev[l]), want)
    assert mgr.dispatch_log() == "DDH"
    with pytest.raises(kvx.KvxError) as e:
        mgr.d2h([0, 1], [0], [1]).Await()
    assert e.value.code == 3
    mgr.close()


def test_queued_copy_follows_submission_stream(kvx, cuda):
    dev = [torch.zeros(16, 1 << 20, dtype=torch.uint8, device=cuda)]
    mgr = kvx.KVCacheManager(dev, host_blocks_to_allocate=16, dispatch="queued")
    s = torch.cuda.Stream(cuda)
    with torch.cuda.stream(s):
        big = torch.empty(1 << 28, dtype=torch.float32, device=cuda)
        for _ in range(8):
            big.normal_()  # keep the stream busy before the fill
        dev[0][3].fill_(7)
    f = mgr.d2h([3], [5], stream=s)
    f.Await()
    assert np.all(mgr.host_view(0).reshape(16, -1)[5] == 7)
    # A reload's future orders a consumer stream (possibly before it is issued).
    mgr.host_view(0).reshape(16, -1)[6] = 9
    f2 = mgr.h2d([6], [8])
    c = torch.cuda.Stream(cuda)
    f2.wait_on_stream(c)
    with torch.cuda.stream(c):
        got = dev[0][8].clone()
    c.synchronize()
    assert torch.all(got == 9)
    mgr.close()
