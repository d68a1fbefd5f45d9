"""GPU: staging-slot flows. A push stages device blocks into a slot's host ids
layer by layer (StartPushInternal's D2H half), a receive assigns slot host
ids and builds the load plan (StartRead) and IssueH2D moves a slot's host
blocks into device ids; bytes are checked against numpy fancy indexing of the
pools and untouched blocks must keep their bytes."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


def dev_np(t):
    torch.cuda.synchronize()
    return t.detach().cpu().view(torch.uint8).numpy().reshape(t.shape[0], -1).copy()


def make_pools(cuda, rng, layers, blocks, block_bytes):
    host = [rng.integers(0, 256, (blocks, block_bytes), dtype=np.uint8) for _ in range(layers)]
    return host, [torch.from_numpy(h).to(cuda) for h in host]


@pytest.mark.parametrize("host_alloc", ["pinned", "malloc"])
def test_push_stage_then_issue_h2d_moves_blocks(kvx, cuda, host_alloc):
    rng = np.random.default_rng(21)
    host, dev = make_pools(cuda, rng, 4, 96, 4096)
    mgr = kvx.KVCacheManager(dev, max_blocks=16, num_slots=3, host_alloc=host_alloc)
    assert mgr.num_free_slots() == 3
    src = [int(x) for x in rng.choice(96, 12, replace=False)]
    src[3:7] = [40, 41, 42, 43]  # a run that coalesces
    st = mgr.stage_for_push(src)
    assert st["slot_idx"] == 0 and mgr.num_free_slots() == 2
    assert st["host_block_ids"] == mgr.slot_block_ids(0)[:12]
    assert len(st["layer_futures"]) == 4
    for f in st["layer_futures"]:
        f.Await()
    for l in range(4):
        hv = mgr.host_view(l).reshape(-1, 4096)
        assert np.array_equal(hv[st["host_block_ids"]], host[l][src])
    # Receive side: the staged host ids land in device ids `dst`.
    dst = [int(x) for x in rng.choice(96, 12, replace=False)]
    before = [dev_np(d) for d in dev]
    res = mgr.issue_h2d(st["slot_idx"], 12, dst)
    res["future"].Await()
    assert res["total_bytes"] == 4 * 12 * 4096
    assert res["copy_segments"] == len(kvx.copy_plan.build_coalesced_copy_spec(
        st["host_block_ids"], dst)["sizes"])
    for l in range(4):
        got = dev_np(dev[l])
        want = before[l].copy()
        want[dst] = host[l][src]
        assert np.array_equal(got, want)
    mgr.release_slot(st["slot_idx"])
    assert mgr.num_free_slots() == 3
    mgr.close()


def test_prepare_load_plan_drives_h2d(kvx, cuda):
    """StartRead's host ids + load plan, then the plan's H2D spec through the
    manager: every local id receives the block its host id holds, repeated
    local ids once."""
    rng = np.random.default_rng(22)
    host, dev = make_pools(cuda, rng, 2, 64, 2048)
    mgr = kvx.KVCacheManager(dev, max_blocks=8, num_slots=2)
    local = [9, 3, 9, 40, 41, 42, 7]
    remote = [5, 1, 5, 2, 3, 4, 0]
    r = mgr.prepare_load(remote, local)
    slot_ids = mgr.slot_block_ids(r["slot_idx"])
    # Fill the slot's host blocks as a transport would (host bytes per remote id).
    payload = [rng.integers(0, 256, (64, 2048), dtype=np.uint8) for _ in range(2)]
    for l in range(2):
        hv = mgr.host_view(l).reshape(-1, 2048)
        for rem, hid in zip(remote, r["host_block_ids"]):
            hv[hid] = payload[l][rem]
    assert set(r["host_block_ids"]) <= set(slot_ids)
    before = [dev_np(d) for d in dev]
    spec = r["plan"]["h2d_copy"]
    mgr.h2d(spec["src_offsets"], spec["dst_offsets"], spec["sizes"]).Await()
    for l in range(2):
        want = before[l].copy()
        for rem, loc in zip(remote, local):
            want[loc] = payload[l][rem]
        assert np.array_equal(dev_np(dev[l]), want)
    mgr.release_slot(r["slot_idx"])
    mgr.close()
