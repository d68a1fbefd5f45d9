"""Concurrency of the host library on the CPU, from several Python threads at
once (ctypes releases the GIL during each call, so the calls run in the
library concurrently); the Makefile's tsan target runs these under
ThreadSanitizer.

* queued dispatch (kv_cache_manager_base.cc:452-512) fed by four threads,
  every future observed through OnReady on the library's poller thread
  (raw_transfer_core.h:491-530): each callback runs exactly once, with the
  dispatch's own status;
* the store's local flows (kv_cache_store.cc:977-1200) driven by four threads
  on disjoint hashes, with a transfer hook that records the block moves: every
  save and load completes and moves exactly its blocks.
"""
import os
import threading

import pytest


def test_queued_dispatch_from_threads_with_on_ready(kvx):
    os.environ["RAIDEN_ENABLE_ASYNC_DISPATCH"] = "1"
    try:
        m = kvx.KVCacheManager.create_host_only_for_testing(
            num_layers=2, slice_byte_size=64, host_blocks=4)
    finally:
        del os.environ["RAIDEN_ENABLE_ASYNC_DISPATCH"]
    assert m.queued_dispatch
    lock = threading.Lock()
    codes = []
    futures = []

    def submit(t):
        mine = []
        for k in range(150):
            f = (m.d2h if (k + t) % 2 else m.h2d)([0], [1], [1])

            def cb(code):
                with lock:
                    codes.append(code)

            f.on_ready(cb)
            mine.append(f)
        with lock:
            futures.extend(mine)

    threads = [threading.Thread(target=submit, args=(t,)) for t in range(4)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    for f in futures:
        with pytest.raises(kvx.KvxError):
            f.Await()
    m.wait_for_pending_work()
    for _ in range(2000):
        with lock:
            if len(codes) == len(futures):
                break
        threading.Event().wait(0.005)
    assert len(futures) == 600 and len(codes) == 600
    assert set(codes) == {9}  # the host-only manager's FailedPrecondition
    m.close()


def test_store_flows_from_threads(kvx):
    cap = 256
    store = kvx.KVCacheStore(capacity=cap, num_shards=1, store_server_ip="127.0.0.1",
                             metadata_shm_key="")
    moves = []
    mlock = threading.Lock()

    def transfer(d2h, src, dst):
        with mlock:
            moves.append((d2h, tuple(src), tuple(dst)))
        return 0

    store.set_transfer_fn(transfer)
    rid = store.raiden_id
    errors = []
    # Polls return every thread's completions: they land in shared sets.
    saved, loaded, failed = set(), set(), []
    plock = threading.Lock()

    def wait_for(hs, poll, into):
        for _ in range(100000):
            done, bad = poll()[:2]
            with plock:
                into.update(done)
                failed.extend(bad)
                if failed or all(h in into for h in hs):
                    return
        raise AssertionError("poll timed out")

    def worker(t):
        try:
            for r in range(6):
                hs = [b"t%d:r%d:%d" % (t, r, i) for i in range(8)]
                dev = [t * 1000 + r * 10 + i for i in range(8)]
                sl = [kvx.RaidenBlockId(rid, -1, d, kvx.BlockStatus.HBM) for d in dev]
                assert store.insert(hs, sl, on_host=False)
                assert store.save(hs), store.last_error()
                wait_for(hs, store.poll_save_status, saved)
                found = store.lookup(hs, pin_found=True)
                assert [h for h, _ in found] == hs
                assert store.load(hs, [d + 500 for d in dev]), store.last_error()
                wait_for(hs, store.poll_load_status, loaded)
        except Exception as e:  # reported below, on the main thread
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(4)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    assert not errors, errors
    assert not failed
    assert len(saved) == 192 and len(loaded) == 192
    d2h_src = sorted(s for d2h, src, _ in moves if d2h for s in src)
    h2d_dst = sorted(d for d2h, _, dst in moves if not d2h for d in dst)
    want = sorted(t * 1000 + r * 10 + i for t in range(4) for r in range(6) for i in range(8))
    assert d2h_src == want
    assert h2d_dst == sorted(x + 500 for x in want)
    assert store.size() == 192
    store.close()
