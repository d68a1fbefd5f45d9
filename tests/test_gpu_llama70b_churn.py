"""GPU: Llama-3-70B-shaped prefix-cache churn through the KV store at full
size, every byte checked.

The pool is 80 layers of K and V: 160 storages of 12000 blocks of 32 KiB
(16 tokens x 8 KV heads x 128 x bf16), 58.6 GiB of HBM. Requests are
prefixes of document hash chains (document drawn Zipf(1.1), 64-2048 blocks,
log-uniform; the first request is 2048 blocks, 10 GiB per direction, the
second 64). Each request looks up its chain (pinning the cached prefix),
loads the host-resident prefix into random device blocks and saves the rest
from other device blocks, load and save issued together, as the reference's
local flows do (tpu_sync/kv_cache/kv_cache_store.cc:977-1200). The host tier
holds 2048 blocks, far fewer than the request stream saves, so saves evict
through candidates and the LRU tail (kv_cache_store.cc:1743-1781,
lru_cache.h:260); hashes demoted to candidates and requested again are
saved again.

The test runs on a pinned tier and on a /dev/shm tier, the second with the
benchmark's staging ring (16 chunks of 32 MiB), so its copies take the pageable bounce
lanes (host threads between the segment and pinned bounce buffers, SDMA
between those and device staging) that the benchmark's churn measures.

Checks, against device-side copies taken with torch (not the library):
  * every block a load places equals, in all 160 storages, the bytes its
    hash had on the device when it was saved;
  * at the end every device block holds either its initial bytes (never a
    load destination: compared through a 64-bit weighted word sum per
    (storage, block), taken before the run) or the bytes of the last hash
    loaded into it.
"""
import os

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

L, P, BB, HOST_BLOCKS = 80, 12000, 32768, 2048
S = 2 * L
DOCS, REQUESTS = 12, 20


def _fingerprints(pools, weights):
    """Per (storage, block): sum of the block's int64 words times fixed
    random odd weights, wrapping (any single changed word changes it)."""
    out = torch.empty(len(pools), P, dtype=torch.int64, device=weights.device)
    for s, p in enumerate(pools):
        out[s] = (p.view(torch.int64) * weights).sum(dim=1)
    return out


def _poll(fn, want, what):
    got = []
    for _ in range(200000):
        done, failed = fn()[:2]
        assert not failed, f"{what} failed for {len(failed)} blocks"
        got += done
        if len(got) >= want:
            return got
    raise AssertionError(f"{what}: {len(got)} of {want} done")


@pytest.mark.parametrize("host_alloc", ["pinned", "shm"])
def test_llama70b_prefix_cache_churn_bytes(kvx, cuda, host_alloc):
    rng = np.random.default_rng(2024)
    gen = torch.Generator(device=cuda).manual_seed(7)
    print(f"allocating {S} x {P} x {BB} B pool", flush=True)
    pools = [torch.randint(0, 256, (P, BB), dtype=torch.uint8, device=cuda, generator=gen)
             for _ in range(S)]
    weights = torch.randint(-(1 << 62), 1 << 62, (BB // 8,), dtype=torch.int64, device=cuda,
                            generator=gen) | 1
    initial = _fingerprints(pools, weights)
    store = kvx.KVCacheStore(capacity=HOST_BLOCKS, num_shards=1, store_server_ip="127.0.0.1",
                             metadata_shm_key="")
    tier = {}
    if host_alloc == "shm":
        tier = dict(host_alloc="shm", shm_key=f"kvx_test_churn_{os.getpid()}",
                    staging_chunk_bytes=32 << 20, staging_chunks=16)
    mgr = kvx.KVCacheManager(pools, host_blocks_to_allocate=HOST_BLOCKS,
                             raiden_controller_address=store.raiden_controller_address,
                             **tier)
    assert mgr.host_alloc == host_alloc
    rid = store.raiden_id
    on_host = (kvx.BlockStatus.HOST, kvx.BlockStatus.HOST_AND_HBM)
    w = 1.0 / np.arange(1, DOCS + 1) ** 1.1
    cdf = np.cumsum(w) / w.sum()

    snaps = []          # per request: [S, n_saved, BB] bytes of its saves
    saved_at = {}       # hash -> (snapshot index, row) of its latest save
    last_loaded = {}    # device block -> (snapshot, row) last loaded into it
    saves = loads = recycled = 0

    def check(blocks, where, what):
        """Device blocks `blocks` hold, in every storage, the snapshot rows
        `where` ((snapshot, row) pairs; one index_select per snapshot and
        storage)."""
        want_i = torch.tensor([t for t, _ in where])
        want_j = torch.tensor([j for _, j in where])
        dst = torch.as_tensor(np.asarray(blocks, dtype=np.int64)).to(cuda)
        for t in torch.unique(want_i).tolist():
            sel = (want_i == t).nonzero().flatten()
            rows = want_j[sel].to(cuda)
            got_blocks = dst[sel.to(cuda)]
            for s in range(S):
                if not torch.equal(pools[s].index_select(0, got_blocks),
                                   snaps[t][s].index_select(0, rows)):
                    raise AssertionError(f"{what}: storage {s} differs from the bytes "
                                         f"saved in snapshot {t}")

    for r in range(REQUESTS):
        doc = int(np.searchsorted(cdf, rng.random()))
        nb = 2048 if r == 0 else 64 if r == 1 else int(np.exp(rng.uniform(np.log(64),
                                                                          np.log(2048))))
        chain = [b"d%03d:%05d" % (doc, i) for i in range(nb)]
        dev_ids = rng.permutation(P)[:nb]
        candidates = set(store.candidate_keys())
        found = store.lookup(chain, pin_found=True)
        k = len(found)
        assert [h for h, _ in found] == chain[:k]
        assert all(b.status in on_host for _, b in found), r
        load_h = [h for h, _ in found]
        load_d = dev_ids[:k]
        # After the cached prefix, hashes still on the host past an evicted
        # one are not saved again; the others are inserted and saved.
        fresh = [(h, int(d)) for h, d in zip(chain[k:], dev_ids[k:])
                 if not store.lookup([h], pin_found=False)]
        recycled += sum(h in candidates for h, _ in fresh)
        if fresh:
            idx = torch.tensor([d for _, d in fresh], device=cuda)
            snaps.append(torch.stack([p.index_select(0, idx) for p in pools]))
            for j, (h, _) in enumerate(fresh):
                saved_at[h] = (len(snaps) - 1, j)
            sl = [kvx.RaidenBlockId(rid, -1, d, kvx.BlockStatus.HBM) for _, d in fresh]
            assert store.insert([h for h, _ in fresh], sl, on_host=False), r
        print(f"request {r}: doc {doc}, {nb} blocks, load {k}, save {len(fresh)}", flush=True)
        # Load and save issued together, then both polled to completion.
        if load_h:
            assert store.load(load_h, [int(d) for d in load_d]), store.last_error()
        if fresh:
            assert store.save([h for h, _ in fresh]), store.last_error()
        if load_h:
            _poll(store.poll_load_status, len(load_h), "load")
        if fresh:
            _poll(store.poll_save_status, len(fresh), "save")
        torch.cuda.synchronize()
        loads += len(load_h)
        saves += len(fresh)
        assert store.size() <= HOST_BLOCKS
        if load_h:
            where = [saved_at[h] for h in load_h]
            check(load_d, where, f"request {r}")
            for d, tj in zip(load_d, where):
                last_loaded[int(d)] = tj
    evicted = len(saved_at) - store.size()
    assert saves > 2 * HOST_BLOCKS and loads > 0 and evicted > HOST_BLOCKS, (saves, loads)

    # Every block: initial bytes, or those last loaded into it.
    final = _fingerprints(pools, weights)
    touched = torch.zeros(P, dtype=torch.bool, device=cuda)
    if last_loaded:
        touched[torch.tensor(sorted(last_loaded), device=cuda)] = True
    assert torch.equal(final[:, ~touched], initial[:, ~touched])
    if last_loaded:
        blocks = sorted(last_loaded)
        check(blocks, [last_loaded[d] for d in blocks], "final state")
    print(f"saves {saves}, loads {loads}, evicted {evicted}, candidates re-saved "
          f"{recycled}, blocks loaded into {len(last_loaded)}", flush=True)
    if host_alloc == "shm":
        # Every copy of the shm tier went through the bounce lanes.
        st = mgr.engine_stats()
        assert st["bounce_copies"] > 0 and st["bounce_copies"] == st["staged_copies"], st
    mgr.close()
    store.close()
    if tier:
        seg = f"/dev/shm/{tier['shm_key']}_dev_{cuda.index or 0}"
        if os.path.exists(seg):
            os.unlink(seg)
    del snaps, pools
    torch.cuda.empty_cache()
