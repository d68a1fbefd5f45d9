#!/usr/bin/env python3
"""KV offload/reload benchmark on one MI355X.

Workload (default): Llama-3-8B-shaped paged KV cache -- 32 layers with K and
V in separate buffers (64 storages), 8 KV heads, head_dim 128, 16-token
blocks, bf16, a pool of 16384 blocks (32 GiB of HBM). One step offloads a
batch of 512 random blocks (gather kernel + D2H into a pinned host slot) and
reloads the previous batch from the other host slot (H2D + scatter kernel
into 512 random free blocks); the two run at the same time in the two PCIe
directions. value = KV payload bytes offloaded + reloaded per second.

Printed as one JSON line, with the gather kernel's HBM roofline (HIP events
on the kernel's stream over the timed region), measured pinned PCIe peaks
per direction, and the CPU host pack/unpack baseline (the oracle's
restatement of the reference's ReadBlockBytes/WriteBlockBytes loop).
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
HBM_PEAK_GBPS = 8000.0

WORKLOADS = {
    "llama3-8b-kv": dict(layers=32, kv_heads=8, head_dim=128, block_tokens=16,
                         dtype="bf16", dtype_bytes=2, pool_blocks=16384, batch=512),
}


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse_args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--workload", default="llama3-8b-kv", choices=sorted(WORKLOADS))
    p.add_argument("--chunk-mib", type=int, default=256)
    p.add_argument("--chunks", type=int, default=4)
    p.add_argument("--cpu-seconds", type=float, default=5.0,
                   help="minimum seconds per CPU-baseline leg (0 skips it)")
    p.add_argument("--no-extras", action="store_true",
                   help="skip the one-direction and PCIe-peak measurements")
    return p.parse_args()


def timed_events(torch, fn, reps, stream):
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        fn()
        torch.cuda.synchronize()
        start.record(stream)
        for _ in range(reps):
            fn()
        stop.record(stream)
    stop.synchronize()
    return start.elapsed_time(stop) / 1e3 / reps


def pcie_peaks(torch, dev, nbytes=1 << 30, reps=5):
    """Large pinned hipMemcpyAsync per direction, and both at once."""
    h = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
    h2 = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
    d = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    d2 = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    s1 = torch.cuda.Stream(dev)
    s2 = torch.cuda.Stream(dev)
    t_d2h = timed_events(torch, lambda: h.copy_(d, non_blocking=True), reps, s1)
    t_h2d = timed_events(torch, lambda: d.copy_(h, non_blocking=True), reps, s1)
    # Both directions at once on two streams.
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        with torch.cuda.stream(s1):
            h.copy_(d, non_blocking=True)
        with torch.cuda.stream(s2):
            d2.copy_(h2, non_blocking=True)
    torch.cuda.synchronize()
    t_bi = (time.perf_counter() - t0) / reps
    # Device-to-device copy (read + write bytes).
    t_d2d = timed_events(torch, lambda: d2.copy_(d), reps, s1)
    out = {
        "pcie_d2h_gbps": nbytes / t_d2h / 1e9,
        "pcie_h2d_gbps": nbytes / t_h2d / 1e9,
        "pcie_bidir_gbps": 2 * nbytes / t_bi / 1e9,
        "hbm_d2d_copy_gbps": 2 * nbytes / t_d2d / 1e9,
    }
    del h, h2, d, d2
    return out


def cpu_baseline(oracle, S, bb, n, min_seconds):
    """The reference's host block pack/unpack (oracle restatement of
    ReadBlockBytes/WriteBlockBytes per block per storage) on host pools of
    the workload's block shape, single-threaded and on every allowed core."""
    pool_blocks = 1024
    rng = np.random.default_rng(7)
    pools = [rng.integers(0, 256, pool_blocks * bb, dtype=np.uint8) for _ in range(S)]
    staging = np.empty(S * n * bb, np.uint8)
    try:
        ncores = len(os.sched_getaffinity(0))
    except AttributeError:
        ncores = os.cpu_count() or 1
    ncores = max(1, min(ncores, 64))
    legs = {}
    for threads in sorted({1, ncores}):
        iters, t_total = 0, 0.0
        while t_total < min_seconds or iters < 2:
            ids = rng.choice(pool_blocks, size=n, replace=False)
            dst = rng.choice(pool_blocks, size=n, replace=False)
            t0 = time.perf_counter()
            rc, _ = oracle.extract(pools, bb, ids, nthreads=threads, staging=staging)
            rc2 = oracle.insert(pools, bb, dst, staging, nthreads=threads)
            t_total += time.perf_counter() - t0
            assert rc == 0 and rc2 == 0
            iters += 1
        legs[threads] = (2 * iters * S * n * bb / t_total / 1e9, iters)
        log(f"cpu baseline threads={threads}: {legs[threads][0]:.2f} GB/s ({iters} iters)")
    best = legs[ncores]
    return {
        "value": round(best[0], 3),
        "unit": "GB/s",
        "cores": ncores,
        "kind": "port",
        "single_thread_gbps": round(legs[1][0], 3),
        "sample": (f"{S} storages x {pool_blocks}-block host pools x {bb} B blocks; "
                   f"per iteration extract {n} random ids into a contiguous buffer and "
                   f"insert it at {n} other ids; {best[1]} iterations"),
    }


def main():
    args = parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "bench.py measures one GPU; this build has no "
                                   "multi-GPU path (--gpus must be 1)"}))
        sys.exit(2)
    import torch
    sys.path.insert(0, ROOT)
    import __graft_entry__
    pkg = __graft_entry__.load_package()

    w = WORKLOADS[args.workload]
    L, n, P = w["layers"], w["batch"], w["pool_blocks"]
    S = 2 * L
    bb = w["block_tokens"] * w["kv_heads"] * w["head_dim"] * w["dtype_bytes"]
    dev = torch.device("cuda:0")
    log(f"allocating {S} x {P} x {bb} B pool ({S * P * bb / 2**30:.1f} GiB)")
    gen = torch.Generator(device=dev).manual_seed(0)
    pools = [torch.randint(-2**31, 2**31 - 1, (P, bb // 4), dtype=torch.int32, device=dev,
                           generator=gen).view(torch.uint8) for _ in range(S)]
    torch.cuda.synchronize()
    mgr = pkg.KVCacheManager(pools, host_blocks_to_allocate=2 * n,
                             staging_chunk_bytes=args.chunk_mib << 20,
                             staging_chunks=args.chunks, profile_kernels=True)
    log("manager ready")
    rng = np.random.default_rng(0)
    slots = [list(range(0, n)), list(range(n, 2 * n))]

    def batch():
        perm = rng.permutation(P)
        return perm[:n].tolist(), perm[n:2 * n].tolist()

    # Prime slot 1 so the first reload reads offloaded data.
    mgr.d2h(batch()[0], slots[1]).Await()
    pending = []

    def step(k):
        for f in pending:
            f.Await()
        pending.clear()
        ids, free = batch()
        pending.append(mgr.d2h(ids, slots[k % 2]))
        pending.append(mgr.h2d(slots[(k + 1) % 2], free))

    for k in range(args.warmup):
        step(k)
    for f in pending:
        f.Await()
    pending.clear()
    mgr.wait_for_pending_work()
    torch.cuda.synchronize()
    mgr.kernel_times(True, reset=True)
    mgr.kernel_times(False, reset=True)
    log(f"timing {args.steps} steps")
    t0 = time.perf_counter()
    for k in range(args.steps):
        step(args.warmup + k)
    for f in pending:
        f.Await()
    pending.clear()
    mgr.wait_for_pending_work()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    step_bytes = 2 * n * S * bb
    value = args.steps * step_bytes / elapsed / 1e9
    kg = mgr.kernel_times(True, reset=True)
    ks = mgr.kernel_times(False, reset=True)
    log(f"offload+reload: {value:.2f} GB/s, {elapsed / args.steps * 1e3:.2f} ms/step")

    def kernel_roofline(kt):
        if kt["launches"] == 0:
            return None
        avg_s = kt["total_ms"] / kt["launches"] / 1e3
        per_launch = kt["bytes"] / kt["launches"]
        ach = per_launch / avg_s / 1e9
        return {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBPS,
                "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBPS, 4), "traffic": None,
                "kernel": "block_copy_kernel (gather)", "launches": kt["launches"],
                "avg_launch_us": round(avg_s * 1e6, 2), "bytes_per_launch": int(per_launch)}

    roof = kernel_roofline(kg)
    scatter_roof = kernel_roofline(ks)
    if scatter_roof:
        scatter_roof["kernel"] = "block_copy_kernel (scatter)"

    extras = {}
    if not args.no_extras:
        reps = max(3, args.steps // 2)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            mgr.d2h(batch()[0], slots[0]).Await()
        t_off = (time.perf_counter() - t0) / reps
        t0 = time.perf_counter()
        for _ in range(reps):
            mgr.h2d(slots[0], batch()[1]).Await()
        t_rel = (time.perf_counter() - t0) / reps
        mgr.kernel_times(True, reset=True)
        mgr.kernel_times(False, reset=True)
        log("measuring pinned PCIe peaks")
        peaks = pcie_peaks(torch, dev)
        half = n * S * bb
        extras = {
            "offload_gbps": round(half / t_off / 1e9, 2),
            "reload_gbps": round(half / t_rel / 1e9, 2),
            **{k: round(v, 2) for k, v in peaks.items()},
        }
        extras["offload_frac_of_pcie_d2h"] = round(extras["offload_gbps"] / peaks["pcie_d2h_gbps"], 4)
        extras["reload_frac_of_pcie_h2d"] = round(extras["reload_gbps"] / peaks["pcie_h2d_gbps"], 4)
        extras["duplex_frac_of_pcie_bidir"] = round(value / peaks["pcie_bidir_gbps"], 4)
    mgr.close()
    del pools
    torch.cuda.empty_cache()

    cpu = None
    if args.cpu_seconds > 0:
        log("CPU baseline (oracle host pack/unpack)")
        cpu = cpu_baseline(__graft_entry__.load_oracle(), S, bb, n, args.cpu_seconds)

    out = {
        "metric": "KV offload/reload GB/s (HBM gather + PCIe) and % of roofline, 1 GPU",
        "value": round(value, 3),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed / args.steps * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8",
        "data": "synthetic",
        "config": {
            "workload": "llama3-8b-kv offload+reload (Llama-3-8B-shaped paged KV, 1 GPU)",
            "layers": L, "kv_heads": w["kv_heads"], "head_dim": w["head_dim"],
            "block_tokens": w["block_tokens"], "kv_dtype": w["dtype"], "storages": S,
            "block_bytes": bb, "pool_blocks": P, "batch_blocks": n,
            "staging_chunk_mib": args.chunk_mib,
        },
        "blocks_per_s": round(args.steps * 2 * n / elapsed, 1),
        "roofline": roof,
        "scatter_roofline": scatter_roof,
        "cpu_baseline": cpu,
        **extras,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
