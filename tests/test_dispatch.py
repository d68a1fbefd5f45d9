"""Queued D2h/H2d dispatch on the CPU (kv_cache_manager_base.cc:452-512 and
the reference tests BackgroundWorkerThreadExecutesInFifoOrder /
BackgroundWorkerThreadDisabledByDefault, kv_cache_manager_test.cc:1212-1249):
copies are dispatched in submission order on the background thread, the call
returns a future at once and errors arrive through it; the environment switch
and shutdown cancellation."""
import os

import pytest


def host_mgr(kvx, **kw):
    return kvx.KVCacheManager.create_host_only_for_testing(
        num_layers=1, num_shards=1, slice_byte_size=128, host_blocks=2, **kw)


def queued_host_mgr(kvx):
    # create_host_only_for_testing follows the environment switch.
    os.environ["RAIDEN_ENABLE_ASYNC_DISPATCH"] = "1"
    try:
        return host_mgr(kvx)
    finally:
        del os.environ["RAIDEN_ENABLE_ASYNC_DISPATCH"]


def test_fifo_order_and_errors_through_futures(kvx):
    m = queued_host_mgr(kvx)
    assert m.queued_dispatch
    f1 = m.h2d([0], [0], [1])
    f2 = m.d2h([0], [0], [1])
    f3 = m.h2d([0], [0], [1])
    for f in (f1, f2, f3):
        with pytest.raises(kvx.KvxError, match="device-backed") as e:
            f.Await()
        assert e.value.code == 9
    assert m.dispatch_log() == "HDH"
    m.close()


def test_disabled_by_default(kvx):
    os.environ.pop("RAIDEN_ENABLE_ASYNC_DISPATCH", None)
    m = host_mgr(kvx)
    assert not m.queued_dispatch
    with pytest.raises(kvx.KvxError, match="device-backed"):
        m.h2d([0], [0], [1])
    assert m.dispatch_log() == "H"
    m.close()


def test_shutdown_cancels_or_completes_every_copy(kvx):
    m = queued_host_mgr(kvx)
    futs = [m.d2h([0], [0], [1]) for _ in range(2000)]
    m.close()
    codes = set()
    for f in futs:
        with pytest.raises(kvx.KvxError) as e:
            f.Await()
        codes.add(e.value.code)
    assert codes <= {1, 9}  # CANCELLED (never dispatched) or the dispatch's own error
