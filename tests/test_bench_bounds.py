"""The benchmark's PCIe bounds for the store churn (bench.py), on the CPU:
the windowed bound against closed forms that pin it from both ends, and a
small case worked by hand."""
import os
import sys

import numpy as np
import pytest

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import bench  # noqa: E402

PEAKS = {"pcie_h2d_gbps": 57.3, "pcie_d2h_gbps": 57.0, "pcie_bidir_gbps": 96.4}
BLOCK = 160 * 32768


def per_request_closed_form(reqs, peaks=PEAKS, blk=BLOCK):
    """One request at a time: each needs max(load / H2D, save / D2H,
    (load + save) / bidir) seconds."""
    h, d, b = (peaks[k] * 1e9 for k in ("pcie_h2d_gbps", "pcie_d2h_gbps", "pcie_bidir_gbps"))
    t = sum(max(l * blk / h, s * blk / d, (l + s) * blk / b) for l, s in reqs)
    return sum(l + s for l, s in reqs) * blk / t / 1e9


def overlapped_closed_form(reqs, peaks=PEAKS, blk=BLOCK):
    L = sum(l for l, _ in reqs) * blk
    S = sum(s for _, s in reqs) * blk
    t = max(L / (peaks["pcie_h2d_gbps"] * 1e9), S / (peaks["pcie_d2h_gbps"] * 1e9),
            (L + S) / (peaks["pcie_bidir_gbps"] * 1e9))
    return (L + S) / t / 1e9


def churn_like(seed, n=120):
    rng = np.random.default_rng(seed)
    reqs = []
    for _ in range(n):
        nb = int(np.exp(rng.uniform(np.log(64), np.log(2048))))
        f = 0.0 if rng.random() < 0.3 else rng.uniform(0.2, 1.0)
        reqs.append((int(f * nb), nb - int(f * nb)))
    return reqs


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_one_in_flight_is_the_per_request_bound(seed):
    reqs = churn_like(seed)
    got = bench.window_bound_gbps(reqs, 1, PEAKS, BLOCK)
    assert got == pytest.approx(per_request_closed_form(reqs), rel=1e-9)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_whole_stream_in_flight_is_the_overlapped_bound(seed):
    reqs = churn_like(seed)
    got = bench.window_bound_gbps(reqs, len(reqs), PEAKS, BLOCK)
    assert got == pytest.approx(overlapped_closed_form(reqs), rel=1e-9)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_a_wider_window_never_lowers_the_bound(seed):
    reqs = churn_like(seed)
    b = [bench.window_bound_gbps(reqs, w, PEAKS, BLOCK) for w in (1, 2, 3, 4, 8, len(reqs))]
    assert all(x <= y * (1 + 1e-9) for x, y in zip(b, b[1:]))
    assert b[0] < b[-1]


def test_two_requests_worked_by_hand():
    # Unit rates: H2D 2, D2H 2, both at once 3 (bytes and seconds in blocks).
    peaks = {"pcie_h2d_gbps": 2e-9, "pcie_d2h_gbps": 2e-9, "pcie_bidir_gbps": 3e-9}
    # A load of 6, then a save of 6. One in flight: 3 s + 3 s. Two in flight:
    # both queued at once share 3: 1.5 each, done together at 4 s.
    reqs = [(6, 0), (0, 6)]
    assert bench.window_bound_gbps(reqs, 1, peaks, 1) == pytest.approx(12 / 6 * 1e-9)
    assert bench.window_bound_gbps(reqs, 2, peaks, 1) == pytest.approx(12 / 4 * 1e-9)
    # Window of two over three requests: the third (a load of 6) waits for
    # the first: the first load and the save run at 1.5 each for 4 s, then
    # the third load runs alone at 2 for 3 s.
    reqs = [(6, 0), (0, 6), (6, 0)]
    assert bench.window_bound_gbps(reqs, 2, peaks, 1) == pytest.approx(18 / 7 * 1e-9)
    # An uneven pair in one request: load 8, save 2 ask for 2.4 and 0.6 of
    # the shared 3; the load is capped at 2, the save takes 1 and ends at
    # 2 s, the load at 4 s (8 / 2).
    assert bench.window_bound_gbps([(8, 2)], 1, peaks, 1) == pytest.approx(10 / 4 * 1e-9)


def test_empty_requests_and_stream():
    assert bench.window_bound_gbps([], 2, PEAKS, BLOCK) is None
    assert bench.window_bound_gbps([(0, 0), (0, 0)], 2, PEAKS, BLOCK) is None
    reqs = [(0, 0), (100, 0), (0, 0), (0, 50)]
    assert bench.window_bound_gbps(reqs, 1, PEAKS, BLOCK) == pytest.approx(
        per_request_closed_form(reqs), rel=1e-9)


@pytest.mark.parametrize("inflight", [1, 2, 3, 4, 8])
def test_the_churn_window_keeps_inflight_minus_one(inflight):
    """After issuing request j the churn leaves requests j - inflight + 2 .. j
    in flight (fewer at the start), so request j + 1 joins at most
    inflight - 1 others: replayed over a stream of requests."""
    window = []
    for j in range(20):
        window.append(j)
        keep = bench.requests_to_keep(window, inflight)
        want = list(range(max(0, j - inflight + 2), j + 1)) if inflight > 1 else []
        assert keep == want, (j, keep)
        window = keep
