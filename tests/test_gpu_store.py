"""GPU: the KV store's local save/load flows through the real KV manager
(gather/scatter kernels + DMA) on the MI355X.

Restates tpu_sync/api/torch/kv_cache_store_e2e_test.py:150-300 (save blocks
0,1 to host, load them into blocks 2,3, compare with [a, b, a, b]) and
kv_cache_store_recovery_e2e_test.py (save into a shared-memory host pool,
SIGKILL, restart, recover the index from the metadata table and load the
bytes back), and runs a prefix-cache churn with evict-on-save whose every
loaded block is checked byte-for-byte against what was saved.
"""
import os
import random
import subprocess
import sys
import uuid

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _poll(fn, want):
    for _ in range(5000):
        r = fn()
        done, failed = r[0], r[1]
        assert not failed, failed
        if len(done) >= want:
            return done
    raise AssertionError("poll timed out")


@pytest.mark.parametrize("use_slices", [False, True])
def test_e2e_save_and_load(kvx, cuda, use_slices):
    num_blocks = 4
    shape = (num_blocks, 128, 8, 8, 128)
    host_data = np.arange(np.prod(shape), dtype=np.float32).reshape(shape)
    cache = torch.tensor(host_data, device=cuda)
    expected = host_data.copy()
    expected[2] = host_data[0]
    expected[3] = host_data[1]
    rid = kvx.RaidenId(f"save_{uuid.uuid4().hex[:8]}_job", "0", "cache", 0)
    store = kvx.KVCacheStore(capacity=num_blocks, raiden_id=rid, num_shards=1,
                             store_server_ip="localhost", metadata_shm_key="")
    mgr = kvx.KVCacheManager([cache], max_blocks=num_blocks, num_slots=2,
                             raiden_controller_address=store.raiden_controller_address)
    hashes = [b"hash_0", b"hash_1"]
    slices = [kvx.RaidenBlockId(rid, -1, 0, kvx.BlockStatus.HBM),
              kvx.RaidenBlockId(rid, -1, 1, kvx.BlockStatus.HBM)]
    assert store.insert(hashes, slices, on_host=False)
    res = store.lookup(hashes, pin_found=False)
    assert [(b.status, b.device_block_id) for _, b in res] == \
        [(kvx.BlockStatus.HBM, 0), (kvx.BlockStatus.HBM, 1)]
    assert store.save(hashes)
    _poll(store.poll_save_status, 2)
    res = store.lookup(hashes, pin_found=False)
    assert [(b.status, b.host_block_id) for _, b in res] == \
        [(kvx.BlockStatus.HOST_AND_HBM, 0), (kvx.BlockStatus.HOST_AND_HBM, 1)]
    # The host mirror holds blocks 0 and 1 byte-for-byte.
    bb = cache[0].numel() * 4
    for i in range(2):
        assert mgr.read_block_bytes(0, i) == host_data[i].tobytes()
    if use_slices:
        load_slices = [b for _, b in store.lookup(hashes)]
        assert store.load(hashes, [2, 3], slices=load_slices)
    else:
        assert len(store.lookup(hashes)) == 2
        assert store.load(hashes, [2, 3])
    _poll(store.poll_load_status, 2)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(cache.cpu().numpy(), expected)
    assert store.get_pin_count(hashes[0]) == 0
    assert bb == host_data[0].nbytes
    mgr.close()
    store.close()


def test_prefix_cache_churn_with_eviction(kvx, cuda):
    """Random save/load/lookup churn over a host tier smaller than the set of
    hashes, so saves evict LRU entries; every completed load must place in
    the device block exactly the bytes that were saved under its hash."""
    rng = random.Random(3)
    layers, pool_blocks, bb, host_blocks = 6, 64, 4096, 24
    gen = torch.Generator(device=cuda).manual_seed(1)
    pools = [torch.randint(0, 256, (pool_blocks, bb), dtype=torch.uint8, device=cuda,
                           generator=gen) for _ in range(layers)]
    store = kvx.KVCacheStore(capacity=host_blocks, num_shards=1,
                             store_server_ip="127.0.0.1", metadata_shm_key="")
    mgr = kvx.KVCacheManager(pools, host_blocks_to_allocate=host_blocks,
                             raiden_controller_address=store.raiden_controller_address)
    rid = store.raiden_id
    content = {}  # hash -> bytes saved (layers x bb)
    free_dev = list(range(pool_blocks))
    rng.shuffle(free_dev)

    def dev_bytes(blk):
        torch.cuda.synchronize()
        return b"".join(p[blk].cpu().numpy().tobytes() for p in pools)

    saved = loaded = 0
    for step in range(60):
        # Offload a few fresh blocks under new hashes.
        n = rng.randint(1, 4)
        hs = [f"h{step}_{i}".encode() for i in range(n)]
        devs = [free_dev[(step * 4 + i) % pool_blocks] for i in range(n)]
        for h, d in zip(hs, devs):
            content[h] = dev_bytes(d)
        sl = [kvx.RaidenBlockId(rid, -1, d, kvx.BlockStatus.HBM) for d in devs]
        if not store.insert(hs, sl, on_host=False):
            continue
        if not store.save(hs):
            store.release(hs)
            continue
        saved += len(_poll(store.poll_save_status, len(hs)))
        # Reload a random earlier prefix of hashes that is still resident.
        want = rng.sample(sorted(content), min(3, len(content)))
        hits = store.lookup(want)
        if not hits:
            continue
        hit_hashes = [h for h, _ in hits]
        targets = rng.sample(range(pool_blocks), len(hit_hashes))
        assert store.load(hit_hashes, targets)
        _poll(store.poll_load_status, len(hit_hashes))
        for h, t in zip(hit_hashes, targets):
            assert dev_bytes(t) == content[h], (step, h)
            loaded += 1
    assert saved > host_blocks and loaded > 10
    mgr.close()
    store.close()


_RECOVERY_SCRIPT = r'''
import os, signal, sys
import numpy as np
import torch
import __graft_entry__
kvx = __graft_entry__.load_package()
N = 4
SHAPE = (N, 16, 8, 128)
HASHES = [b"hash_%d" % i for i in range(N)]

def stack(cache):
    store = kvx.KVCacheStore(N, raiden_id=kvx.RaidenId("rec", "0", "cache", 0),
                             num_shards=1, store_server_ip="localhost")
    mgr = kvx.KVCacheManager([cache], max_blocks=N, num_slots=2,
                             raiden_controller_address=store.raiden_controller_address)
    return store, mgr

def poll(fn, want):
    for _ in range(5000):
        done, failed = fn()[:2]
        assert not failed, failed
        if len(done) >= want:
            return
    raise SystemExit("poll timed out")

data = np.arange(np.prod(SHAPE), dtype=np.float32).reshape(SHAPE)
phase = sys.argv[1]
if phase == "a":
    cache = torch.tensor(data, device="cuda:0")
    store, mgr = stack(cache)
    rid = store.raiden_id
    sl = [kvx.RaidenBlockId(rid, -1, i, kvx.BlockStatus.HBM) for i in range(N)]
    assert store.insert(HASHES, sl, False)
    assert store.save(HASHES)
    poll(store.poll_save_status, N)
    torch.cuda.synchronize()
    got = store.lookup(HASHES, pin_found=False)
    assert [b.host_block_id for _, b in got] == list(range(N))
    print("PHASE_A_SAVED", flush=True)
    os.kill(os.getpid(), signal.SIGKILL)
else:
    cache = torch.zeros(SHAPE, dtype=torch.float32, device="cuda:0")
    store, mgr = stack(cache)
    got = store.lookup(HASHES)
    if phase == "cold":
        assert got == [], got
        print("PHASE_B_COLD", flush=True)
        raise SystemExit(0)
    assert len(got) == N, got
    for i, (h, b) in enumerate(got):
        assert h == HASHES[i] and b.status == kvx.BlockStatus.HOST and b.host_block_id == i
    print("PHASE_B_RECOVERED", flush=True)
    assert store.load(HASHES, list(range(N)))
    poll(store.poll_load_status, N)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(cache.cpu().numpy(), data)
    print("PHASE_B_BYTES", flush=True)
'''


def test_crash_recovery_e2e(kvx, cuda, tmp_path):
    key = f"kvx_gpu_recovery_{os.getpid()}_{uuid.uuid4().hex[:6]}"
    script = tmp_path / "phase.py"
    script.write_text(_RECOVERY_SCRIPT)
    env = dict(os.environ, RAIDEN_SHM_KEY=key, RAIDEN_SHM_MODEL_UID="recovery_model",
               PYTHONPATH=ROOT)
    try:
        a = subprocess.run([sys.executable, str(script), "a"], env=env,
                           capture_output=True, text=True, timeout=300)
        assert "PHASE_A_SAVED" in a.stdout, a.stderr[-3000:]
        assert a.returncode == -9, a.stderr[-3000:]
        b = subprocess.run([sys.executable, str(script), "b"], env=env,
                           capture_output=True, text=True, timeout=300)
        assert b.returncode == 0, b.stderr[-3000:]
        assert "PHASE_B_RECOVERED" in b.stdout and "PHASE_B_BYTES" in b.stdout
        env["RAIDEN_SHM_MODEL_UID"] = "other_model"
        c = subprocess.run([sys.executable, str(script), "cold"], env=env,
                           capture_output=True, text=True, timeout=300)
        assert c.returncode == 0, c.stderr[-3000:]
        assert "PHASE_B_COLD" in c.stdout
    finally:
        for name in os.listdir("/dev/shm"):
            if name.startswith(key):
                os.unlink(os.path.join("/dev/shm", name))
