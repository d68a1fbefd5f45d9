"""GPU: hardware-queue placement of streams, probed on the device.

Work on one hardware queue runs in order, so two streams on one queue
serialize (an offload's DMA behind a reload's: 54 instead of 96 GB/s). The
probe launches one short clock-bounded kernel per stream at once; streams
whose kernels ran one after the other share a queue. A manager probes its
transfer engine's four streams at creation and creates them again while two
share a queue.
"""
import os

import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


def hw_queues():
    """Hardware queues per process the HIP runtime uses (its default: 4)."""
    try:
        v = int(os.environ.get("GPU_MAX_HW_QUEUES", "0"))
    except ValueError:
        v = 0
    return v if 1 <= v <= 64 else 4


def test_probe_sees_one_stream_as_one_queue(kvx, cuda):
    s = torch.cuda.Stream(cuda)
    assert kvx.probe_stream_queues([s, s]) == 1
    assert kvx.probe_stream_queues([s, s, s]) == 3
    assert kvx.probe_stream_queues([s]) == 0
    assert kvx.probe_stream_queues([]) == 0


def test_probe_finds_the_shared_queues_of_more_streams_than_queues(kvx, cuda):
    # 2q streams on at most q queues: at least q pairs share one.
    q = hw_queues()
    streams = [torch.cuda.Stream(cuda) for _ in range(2 * q)]
    pairs = kvx.probe_stream_queues(streams)
    assert q <= pairs <= (2 * q) * (2 * q - 1) // 2, pairs


def test_manager_streams_each_on_their_own_queue(kvx, cuda):
    pools = [torch.zeros(16, 4096, dtype=torch.uint8, device=cuda) for _ in range(2)]
    for _ in range(3):
        mgr = kvx.KVCacheManager(pools, host_blocks_to_allocate=4)
        p = mgr.stream_placement
        assert p["serialized_pairs"] == 0, p
        assert 1 <= p["attempts"] <= 3, p
        mgr.close()


def test_probe_rejects_more_than_64_streams(kvx, cuda):
    s = torch.cuda.Stream(cuda)
    with pytest.raises(kvx.KvxError):
        kvx.probe_stream_queues([s] * 65)


def test_link_peaks_on_the_lanes_engines(kvx, cuda):
    """Pinned copies on the lanes' fixed SDMA engines, one direction at a
    time and both at once: rates in a plausible range (the call checks that
    the bytes landed), both at once never much below one direction alone,
    and one engine bit per direction."""
    r = kvx.measure_link_peaks(64 << 20, 3)
    print(r, flush=True)
    for k in ("d2h_gbps", "h2d_gbps", "bidir_gbps"):
        assert 1.0 < r[k] < 1000.0, r
    assert r["bidir_gbps"] >= 0.9 * max(r["d2h_gbps"], r["h2d_gbps"]), r
    d2h_bit, h2d_bit = r["engines"] >> 16, r["engines"] & 0xFFFF
    for bit in (d2h_bit, h2d_bit):
        assert bit != 0 and bit & (bit - 1) == 0, r
