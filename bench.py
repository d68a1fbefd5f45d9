#!/usr/bin/env python3
"""KV offload/reload benchmark on one MI355X.

Workload (default): Llama-3-8B-shaped paged KV cache -- 32 layers with K and
V in separate buffers (64 storages), 8 KV heads, head_dim 128, 16-token
blocks, bf16, a pool of 16384 blocks (32 GiB of HBM). One step offloads a
batch of 512 random blocks into a pinned host slot and reloads the previous
batch from the other host slot into 512 random free blocks; the two run at
the same time in the two PCIe directions. value = KV payload bytes
offloaded + reloaded per second. The headline mode (auto) picks per copy:
a batch's host runs here average 16 MiB per storage, so it stages (gather
kernel + hipMemcpyAsync through a device staging ring, and H2D + scatter);
headline_path reports the copies it issued. The staged and zero-copy modes
(one kernel between pool and pinned host over PCIe) are measured in the same
run.

Printed as one JSON line, with the gather kernel's HBM roofline (HIP events
on the kernel's stream over the timed region), measured pinned PCIe peaks
per direction, and the CPU host pack/unpack baseline (the oracle's
restatement of the reference's ReadBlockBytes/WriteBlockBytes loop).

Every number comes from checked bytes. Before timing, one offload + reload
with the headline manager is compared with a torch snapshot (the
reference's perf gate, tpu_sync/benchmarks/perf_core.py:112-142); after
each timed workload, outside its timed region, the bytes it moved are
compared with torch indexing (the last duplex step's offload and reload,
each isolated kernel's last launch, the extra configs' outputs). A mismatch
raises and the benchmark exits non-zero; each workload that passed carries
"verified": true.

The kernels are also set against the box itself: box_copy is the library's
strided copy over one contiguous buffer of the same bytes in this process,
and every HBM kernel reports frac_of_box_copy beside its fraction of the
8 TB/s peak. placement times the same kernels over the pool allocated the
other way (one buffer sliced per storage, or one allocation per storage),
alternating in this process.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
HBM_PEAK_GBPS = 8000.0

# HBM bytes per launch measured with rocprofv3 --pmc FETCH_SIZE and, in a
# second run, WRITE_SIZE (KiB per dispatch), each divided by the factor the
# same counter reads for a plain 1 GiB device copy in the same runs (FETCH
# 0.50001, WRITE 1.000): profiles/block_copy_llama3_8b_pmc.txt. Keyed by
# (kernel, algorithmic bytes per launch).
MEASURED_TRAFFIC = {
    ("gather", 2 * 512 * 64 * 32768): int((524452.0 / 0.50001 + 1048621.8 / 1.0) * 1024),
    ("scatter", 2 * 512 * 64 * 32768): int((524348.2 / 0.50001 + 1048598.9 / 1.0) * 1024),
    # The ascending and shuffled runs of ids (profiles/hbm_dram_stall_counters.txt,
    # calibrated by the same run's 1 GiB copy: 0.500011 / 1.0).
    ("scatter_contiguous", 2 * 512 * 64 * 32768): int((524345.0 / 0.500011 + 1048587.5) * 1024),
    ("scatter_shuffled", 2 * 512 * 64 * 32768): int((524345.0 / 0.500011 + 1048604.5) * 1024),
}

WORKLOADS = {
    "llama3-8b-kv": dict(layers=32, kv_heads=8, head_dim=128, block_tokens=16,
                         dtype="bf16", dtype_bytes=2, pool_blocks=16384, batch=512),
}


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


POOL_ALLOC_TEXT = {
    "single": "one device buffer sliced into one [pool_blocks, block_bytes] view per storage",
    "per_storage": "one device allocation per storage",
}


def make_pool(torch, dev, gen, S, P, bb, how):
    """S storages of [P, bb] random bytes: views of one buffer ("single", as
    a serving engine that allocates its whole KV cache at once) or one
    allocation each ("per_storage")."""
    if how == "single":
        buf = torch.randint(-2**31, 2**31 - 1, (S * P * bb // 4,), dtype=torch.int32, device=dev,
                            generator=gen).view(torch.uint8)
        return [buf[k * P * bb:(k + 1) * P * bb].view(P, bb) for k in range(S)]
    return [torch.randint(-2**31, 2**31 - 1, (P, bb // 4), dtype=torch.int32, device=dev,
                          generator=gen).view(torch.uint8) for _ in range(S)]


def parse_args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=1000,
                   help="timed offload+reload steps of the headline workload (its "
                        "configuration runs 1000 iterations); the extra configs and "
                        "mode comparisons run min(steps, 20)")
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--workload", default="llama3-8b-kv", choices=sorted(WORKLOADS))
    p.add_argument("--chunk-mib", type=int, default=256)
    p.add_argument("--chunks", type=int, default=4)
    p.add_argument("--cpu-seconds", type=float, default=5.0,
                   help="minimum seconds per CPU-baseline leg (0 skips it)")
    p.add_argument("--pool-alloc", default="single", choices=["single", "per_storage"],
                   help="how the headline pool is allocated: one buffer sliced per storage "
                        "(measured faster for the scatter) or one allocation per storage")
    p.add_argument("--placement-rounds", type=int, default=3,
                   help="rounds of the gather/scatter kernels over the headline pool and a "
                        "pool allocated the other way, alternating in this process (0: skip)")
    p.add_argument("--no-extras", action="store_true",
                   help="skip the per-mode, one-direction and PCIe-peak measurements")
    p.add_argument("--mode", default="auto", choices=["auto", "staged", "zero_copy"],
                   help="transfer mode of the headline offload/reload loop")
    p.add_argument("--configs", default="scenarios,fp8,weights,tiled,pools,lanes,zipf",
                   help="comma list of extra workloads to measure after the headline "
                        "(scenarios, fp8, weights, tiled, pools, lanes, zipf; empty for none)")
    p.add_argument("--zipf-host-blocks", type=int, default=0,
                   help="host tier of the Zipf churn, in 5 MiB Llama-3-70B blocks (0: "
                        "the configured 256 GB budget, capped by free /dev/shm, available "
                        "RAM and a 160 GiB process budget)")
    p.add_argument("--zipf-batches", type=int, default=240)
    p.add_argument("--pools-host-alloc", default="pinned", choices=["pinned", "malloc"],
                   help="host mirror of the sparse-pool config (malloc: pageable, through "
                        "the bounce lanes)")
    p.add_argument("--zipf-host-alloc", default="shm", choices=["pinned", "shm"],
                   help="host tier memory: a /dev/shm segment (the reference's shared-"
                        "memory tier) or pinned (hipHostMalloc)")
    p.add_argument("--zipf-docs", type=int, default=160,
                   help="documents whose hash-chain prefixes the churn requests")
    p.add_argument("--zipf-chunk-mib", type=int, default=32,
                   help="staging chunk of the churn's manager (0: --chunk-mib); "
                        "32 MiB measured best for its 64-2048-block requests")
    p.add_argument("--zipf-chunks", type=int, default=16,
                   help="staging chunks (ring depth) of the churn's and the lanes' "
                        "managers; their pageable lanes carry a load and a save at once "
                        "at 93.0 / 94.8 / 96.2 GB/s with 4 / 8 / 16 chunks of 32 MiB")
    p.add_argument("--zipf-host-threads", type=int, default=0,
                   help="host copy threads of the churn's bounce lanes (0: the library's 8)")
    p.add_argument("--zipf-mode", default="auto", choices=["auto", "staged", "zero_copy", "lanes"],
                   help="transfer mode of the churn's manager")
    p.add_argument("--zipf-inflight", type=int, default=1,
                   help="requests whose copies may be in flight at once (1: each "
                        "request's load and save finish before the next is issued)")
    p.add_argument("--zipf-more-inflight", default="2,4",
                   help="then continue the churn on the warm tier with this many "
                        "requests in flight, one run per comma-separated count "
                        "(counts below 2 are skipped)")
    p.add_argument("--configs-only", action="store_true",
                   help="measure only the --configs workloads (no headline, no CPU "
                        "baseline) and print them; for profiling one of them")
    p.add_argument("--rocpd-summary", metavar="DB",
                   help="print per-kernel (name, grid) duration statistics of a "
                        "rocprofv3 results database and exit")
    return p.parse_args()


def rocpd_summary(db_path):
    """Kernel durations grouped by (kernel, grid size) and memory copies by
    direction, from a rocprofv3 --kernel-trace results database."""
    import sqlite3
    con = sqlite3.connect(db_path)
    cur = con.cursor()
    print(f"{'kernel':<72} {'grid':>9} {'calls':>6} {'avg_us':>9} {'min_us':>9} {'max_us':>9}")
    q = ("select name, grid_x, count(*), avg(end - start), min(end - start), "
         "max(end - start), sum(end - start) from kernels group by name, grid_x "
         "order by sum(end - start) desc")
    for name, grid, cnt, avg, mn, mx, _ in cur.execute(q):
        short = (name.replace("void ", "").replace("(anonymous namespace)::", "")
                 .replace("unsigned int __vector(4)", "u32x4"))
        if ">(" in short:
            short = short[:short.index(">(") + 1]
        short = short if len(short) <= 72 else short[:69] + "..."
        print(f"{short:<72} {grid:>9} {cnt:>6} {avg / 1e3:>9.2f} {mn / 1e3:>9.2f} {mx / 1e3:>9.2f}")
    q = ("select p.name, k.grid_x, p.counter_name, count(*), avg(p.counter_value), "
         "min(p.counter_value), max(p.counter_value) from pmc_events p left join kernels k "
         "on p.dispatch_id = k.dispatch_id group by p.name, k.grid_x, p.counter_name")
    rows = list(cur.execute(q))
    if rows:
        print(f"\n{'kernel (pmc)':<60} {'grid':>9} {'counter':>11} {'calls':>6} "
              f"{'avg':>13} {'min':>13} {'max':>13}")
        for name, grid, counter, cnt, avg, mn, mx in rows:
            short = (name.replace("void ", "").replace("(anonymous namespace)::", "")
                     .replace("unsigned int __vector(4)", "u32x4"))
            if ">(" in short:
                short = short[:short.index(">(") + 1]
            short = short if len(short) <= 60 else short[:57] + "..."
            print(f"{short:<60} {grid or 0:>9} {counter:>11} {cnt:>6} {avg:>13.1f} "
                  f"{mn:>13.1f} {mx:>13.1f}")
    # Per dispatch of this library's kernels, each counter. Counters collected
    # without _sum come back one row per hardware instance (a TCC counter: one
    # per L2 channel): their spread over instances.
    q = ("select p.dispatch_id, p.name, k.grid_x, k.end - k.start, p.counter_name, "
         "count(*), sum(p.counter_value), min(p.counter_value), max(p.counter_value), "
         "avg(p.counter_value * p.counter_value) from pmc_events p left join kernels k "
         "on p.dispatch_id = k.dispatch_id where p.name like '%kvx::%' "
         "group by p.dispatch_id, p.counter_name "
         "order by p.dispatch_id, p.counter_name")
    rows = list(cur.execute(q))
    if rows:
        print(f"\n{'dispatch':>8} {'kernel (pmc per dispatch)':<48} {'grid':>9} {'dur_us':>8} "
              f"{'counter':>30} {'inst':>5} {'sum':>13} {'min':>11} {'max':>11} "
              f"{'cv':>7} {'max/mean':>8}")
        for did, name, grid, dur, counter, cnt, tot, mn, mx, sq in rows:
            short = name.replace("void ", "").replace("(anonymous namespace)::", "")
            if ">(" in short:
                short = short[:short.index(">(") + 1]
            short = short if len(short) <= 48 else short[:45] + "..."
            mean = tot / cnt
            cv = max(sq - mean * mean, 0.0) ** 0.5 / mean if mean else 0.0
            print(f"{did:>8} {short:<48} {grid or 0:>9} {(dur or 0) / 1e3:>8.1f} "
                  f"{counter:>30} {cnt:>5} {tot:>13.0f} {mn:>11.0f} {mx:>11.0f} "
                  f"{cv:>7.4f} {mx / mean if mean else 0:>8.2f}")
    # Streams and the hardware queues their kernels ran on (memory copies that
    # run on SDMA engines have no compute queue).
    q = ("select stream_id, queue_id, name, count(*) from kernels "
         "group by stream_id, queue_id, name order by stream_id, count(*) desc")
    rows = list(cur.execute(q))
    if rows:
        print(f"\n{'stream':>6} {'queue':>5} {'launches':>8}  kernel")
        for sid, qid, name, cnt in rows:
            short = (name.replace("void ", "").replace("(anonymous namespace)::", "")
                     .replace("unsigned int __vector(4)", "u32x4"))
            if ">(" in short:
                short = short[:short.index(">(") + 1]
            print(f"{sid:>6} {qid if qid is not None else '-':>5} {cnt:>8}  {short[:70]}")
        q = ("select stream_id, name, count(*), sum(size) from memory_copies "
             "group by stream_id, name order by stream_id")
        print(f"\n{'stream':>6} {'copies':>8} {'GB':>9}  direction (SDMA or blit)")
        for sid, name, cnt, size in cur.execute(q):
            print(f"{sid:>6} {cnt:>8} {size / 1e9:>9.3f}  {name}")
    q = ("select name, count(*), sum(size), avg(end - start), sum(end - start) "
         "from memory_copies group by name")
    rows = list(cur.execute(q))
    if rows:
        print(f"\n{'memory copy':<32} {'calls':>6} {'GB':>9} {'avg_us':>9} {'GB/s':>9}")
        for name, cnt, size, avg, tot in rows:
            print(f"{name:<32} {cnt:>6} {size / 1e9:>9.3f} {avg / 1e3:>9.2f} "
                  f"{size / tot if tot else 0:>9.2f}")
        # How long copies of both directions were in flight together, against
        # the time any copy was: a load and a save issued at once should
        # overlap for nearly all of their shorter side.
        ev = []
        for name, start, end in cur.execute("select name, start, end from memory_copies"):
            d = "h2d" if "HOST_TO_DEVICE" in name else ("d2h" if "DEVICE_TO_HOST" in name else None)
            if d:
                ev += [(start, 1, d), (end, -1, d)]
        ev.sort()
        act = {"h2d": 0, "d2h": 0}
        both = anyt = 0
        last = ev[0][0] if ev else 0
        for ts, k, d in ev:
            if act["h2d"] and act["d2h"]:
                both += ts - last
            if act["h2d"] or act["d2h"]:
                anyt += ts - last
            act[d] += k
            last = ts
        if anyt:
            print(f"\ncopies in flight: any {anyt / 1e6:.1f} ms, both directions at once "
                  f"{both / 1e6:.1f} ms ({both / anyt:.1%})")


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


def timed_each(torch, fn, reps, stream):
    """Mean duration of one launch of fn on `stream`, with an event pair
    around each launch (the way the library's profiled kernel launches are
    timed), so a yardstick and the kernels it is compared with carry the same
    per-launch event overhead."""
    with torch.cuda.stream(stream):
        fn()
        torch.cuda.synchronize()
        pairs = []
        for _ in range(reps):
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record(stream)
            fn()
            b.record(stream)
            pairs.append((a, b))
    pairs[-1][1].synchronize()
    return sum(a.elapsed_time(b) for a, b in pairs) / 1e3 / reps


def pcie_peaks(torch, dev, nbytes=1 << 30, reps=5):
    """Large pinned hipMemcpyAsync per direction, and both at once, on random
    bytes like the workload's."""
    h = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
    h2 = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
    gen = torch.Generator(device=dev).manual_seed(1)
    d = torch.randint(-2**31, 2**31 - 1, (nbytes // 4,), dtype=torch.int32, device=dev,
                      generator=gen).view(torch.uint8)
    d2 = torch.randint(-2**31, 2**31 - 1, (nbytes // 4,), dtype=torch.int32, device=dev,
                       generator=gen).view(torch.uint8)
    h.copy_(d)
    h2.copy_(d2)
    torch.cuda.synchronize()
    s1 = torch.cuda.Stream(dev)
    s2 = torch.cuda.Stream(dev)
    # Peaks are bounds: the best of three timed rounds, each after a warm-up.
    t_d2h = min(timed_events(torch, lambda: h.copy_(d, non_blocking=True), reps, s1)
                for _ in range(3))
    t_h2d = min(timed_events(torch, lambda: d.copy_(h, non_blocking=True), reps, s1)
                for _ in range(3))

    def both():  # both directions at once on two streams
        with torch.cuda.stream(s1):
            h.copy_(d, non_blocking=True)
        with torch.cuda.stream(s2):
            d2.copy_(h2, non_blocking=True)

    both()
    t_bi = float("inf")
    for _ in range(3):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            both()
        torch.cuda.synchronize()
        t_bi = min(t_bi, (time.perf_counter() - t0) / reps)
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


def link_peaks_both_ways(torch, dev, pkg, runtime, nbytes=1 << 30, reps=5):
    """The pinned peaks by both methods: `runtime` (pcie_peaks: the runtime's
    hipMemcpyAsync, which picks the DMA engine per copy) and the library's
    copies on the lanes' fixed SDMA engines (measure_link_peaks). Returns
    (the best of the two per figure, the figures by method). The runtime has
    run the two directions of its bidirectional measurement one after the
    other in some processes (one direction's rate), which the fixed engines
    do not."""
    torch.cuda.synchronize()
    fixed = pkg.measure_link_peaks(nbytes, reps)
    by = {"runtime_copies": {k: round(v, 2) for k, v in runtime.items()},
          "fixed_sdma_engines": {"pcie_d2h_gbps": round(fixed["d2h_gbps"], 2),
                                 "pcie_h2d_gbps": round(fixed["h2d_gbps"], 2),
                                 "pcie_bidir_gbps": round(fixed["bidir_gbps"], 2),
                                 "engines": hex(fixed["engines"])}}
    best = dict(runtime)
    for k, f in (("pcie_d2h_gbps", "d2h_gbps"), ("pcie_h2d_gbps", "h2d_gbps"),
                 ("pcie_bidir_gbps", "bidir_gbps")):
        best[k] = max(best[k], fixed[f])
    return best, by

def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def cpu_baseline(oracle, S, bb, n, pool_blocks, min_seconds):
    """The reference's host block pack/unpack (oracle restatement of
    ReadBlockBytes/WriteBlockBytes per block per storage) on host pools of
    the workload's shape (the full pool when the host has room for it, else
    1024 blocks per storage), single-threaded and on every allowed core."""
    try:
        with open("/proc/meminfo") as f:
            kb = {ln.split(":")[0]: int(ln.split()[1]) for ln in f if ln.strip()}
        avail = kb["MemAvailable"] * 1024
    except (OSError, KeyError, ValueError):
        avail = 0
    if S * pool_blocks * bb * 3 > avail:
        pool_blocks = 1024
    rng = np.random.default_rng(7)
    # Every page is written once (the values do not matter to a byte copy).
    pools = [np.full(pool_blocks * bb, k & 0xFF, np.uint8) for k in range(S)]
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
        legs[threads] = (2 * iters * S * n * bb / t_total / 1e9, iters,
                         2 * iters * n / t_total)
        log(f"cpu baseline threads={threads}: {legs[threads][0]:.2f} GB/s ({iters} iters)")
    best = legs[ncores]
    del pools, staging
    return {
        "value": round(best[0], 3),
        "unit": "GB/s",
        "cores": ncores,
        "kind": "port",
        "blocks_per_s": round(best[2], 1),
        "cpu_model": cpu_model(),
        "single_thread_gbps": round(legs[1][0], 3),
        "single_thread_blocks_per_s": round(legs[1][2], 1),
        "sample": (f"{S} storages x {pool_blocks}-block host pools x {bb} B blocks; "
                   f"per iteration extract {n} random ids into a contiguous buffer and "
                   f"insert it at {n} other ids (a block = all {S} storages, "
                   f"{S * bb} B); {best[1]} iterations on {ncores} threads"),
    }


def short_run_duplex(torch, pkg, pools, make_mgr, rng, P, n, args, peaks):
    """Offload + reload at once, as run_duplex, but every host id random
    (host runs of one block, 2 MiB over the 64 storages), through a manager
    in each mode: auto (zero-copy for a lone short-run copy, the lanes while
    both directions are at work), zero_copy and lanes. Then a lone 64-block
    offload, one at a time after an idle pause longer than auto's duplex
    window, to show the lone copy keeps the zero-copy path. Each duplex run's
    last step is checked against torch."""
    out = {}
    hosts = np.split(rng.permutation(4 * n), 4)
    slots = [h.tolist() for h in hosts]
    for mode in ("auto", "zero_copy", "lanes"):
        m = make_mgr(mode)
        batch = batch_source(rng, P, n)
        el, last = run_duplex(torch, m, batch, slots, args.sub_steps, args.warmup)
        verify_duplex(torch, m, pools, slots, last)
        step_bytes = 2 * n * sum(rows_u8(t).shape[1] for t in pools)
        st0 = m.engine_stats()
        time.sleep(0.35)  # past the duplex window: the next copies are lone
        lone = []
        for _ in range(max(5, args.sub_steps // 2)):
            ids = rng.permutation(P)[:64].tolist()
            hid = rng.permutation(4 * n)[:64].tolist()
            t0 = time.perf_counter()
            m.d2h(ids, hid, [1] * 64).Await()
            lone.append(time.perf_counter() - t0)
        st1 = m.engine_stats()
        lone_path = "+".join(k for k in ("zero_copy", "staged", "bounce")
                             if st1[f"{k}_copies"] > st0[f"{k}_copies"]) or "none"
        r = {"duplex_gbps": round(args.sub_steps * step_bytes / el / 1e9, 2),
             "lone_64_block_offload_ms": round(float(np.median(lone)) * 1e3, 3),
             "lone_copy_path": lone_path, "verified": True}
        if peaks:
            r["duplex_frac_of_pcie_bidir"] = round(r["duplex_gbps"] / peaks["pcie_bidir_gbps"], 4)
        out[mode] = r
        log(f"short runs, {mode}: {r}")
        m.close()
    return out


def run_duplex(torch, mgr, batch, slots, steps, warmup):
    """Step k offloads batch k into host slot k%4 and reloads slot (k+2)%4
    (offloaded at step k-2) into fresh free blocks. Step k waits only for the
    copies of step k-2, the last ones touching its slots, so step k-1's copies
    are still in flight when step k is issued: the steady state of a serving
    loop, with no drain between steps (batch() keeps consecutive steps'
    blocks disjoint). Returns the seconds the timed steps took (all of them
    finished) and the last step (k, offloaded ids, reload targets)."""
    for s in (2, 3):
        mgr.d2h(batch()[0], slots[s]).Await()  # the first reloads read real data
    inflight = {}
    last = [None]

    def step(k):
        for f in inflight.pop(k - 2, []):
            f.Await()
        ids, free = batch()
        inflight[k] = [mgr.d2h(ids, slots[k % 4]), mgr.h2d(slots[(k + 2) % 4], free)]
        last[0] = (k, ids, free)

    def drain():
        for fs in inflight.values():
            for f in fs:
                f.Await()
        inflight.clear()
        mgr.wait_for_pending_work()
        torch.cuda.synchronize()

    for k in range(warmup):
        step(k)
    drain()
    mgr.kernel_times(True, reset=True)
    mgr.kernel_times(False, reset=True)
    t0 = time.perf_counter()
    for k in range(steps):
        step(k)
    drain()
    return time.perf_counter() - t0, last[0]


def one_direction(mgr, batch, slots, reps):
    """Offload alone, then reload alone, one copy at a time, after two
    untimed copies each way: the first D2H copies of a fresh manager, and
    those right after the runtime has freed device memory, run 6-13 %
    slower (measured 50.4 and 46.6 against 53.8 GB/s)."""
    for _ in range(2):
        mgr.d2h(batch()[0], slots[0]).Await()
        mgr.h2d(slots[0], batch()[1]).Await()
    t0 = time.perf_counter()
    for _ in range(reps):
        mgr.d2h(batch()[0], slots[0]).Await()
    t_off = (time.perf_counter() - t0) / reps
    t0 = time.perf_counter()
    for _ in range(reps):
        mgr.h2d(slots[0], batch()[1]).Await()
    t_rel = (time.perf_counter() - t0) / reps
    return t_off, t_rel


def kernel_gbps(kt):
    """GB/s of profiled launches: algorithmic bytes / summed event time."""
    if kt["launches"] == 0 or kt["total_ms"] <= 0:
        return None
    return kt["bytes"] / (kt["total_ms"] / 1e3) / 1e9


class Mismatch(AssertionError):
    """Bytes a timed workload moved differ from what torch says they should
    be; the benchmark exits non-zero (as the reference's perf gate does,
    tpu_sync/benchmarks/perf_core.py:112-142)."""


def check(ok, what):
    if not ok:
        raise Mismatch(f"verification failed: {what}")


def rows_u8(t):
    """A [major, ...] device tensor as [major, row bytes] uint8."""
    import torch
    return t.reshape(t.shape[0], -1).view(torch.uint8)


def batch_source(rng, P, n):
    """Per step, n random blocks to offload and n other random free blocks to
    reload into, all 2n disjoint from the previous step's 2n. Consecutive
    steps overlap in flight (step k waits only for step k-2), so a block the
    previous step is still reloading into is never offloaded, and a block it
    is still offloading is never reloaded into: every step's bytes are then
    well defined and the last step can be checked."""
    prev = np.empty(0, np.int64)

    def batch():
        nonlocal prev
        perm = rng.permutation(P)
        if prev.size:
            perm = perm[~np.isin(perm, prev)]
        sel = perm[:2 * n]
        prev = sel
        return sel[:n].tolist(), sel[n:].tolist()
    return batch


def host_rows(mgr, w, bb, first, count):
    """Host mirror blocks [first, first + count) of storage w, as a uint8
    numpy view [count, bb]."""
    return mgr.host_view(w).reshape(-1, bb)[first:first + count]


def verify_duplex(torch, mgr, storages, slots, last):
    """After a duplex run has drained, the last step's copies are checked
    against torch indexing: its offload left the bytes of its source blocks
    in its host slot, and its reload left the bytes of the slot it read
    (offloaded two steps before) in its free blocks."""
    k, ids, free = last
    dev = storages[0].device
    ids_t = torch.tensor(ids, device=dev)
    free_t = torch.tensor(free, device=dev)
    s_off, s_rel = list(slots[k % 4]), list(slots[(k + 2) % 4])
    for w, t in enumerate(storages):
        r = rows_u8(t)
        bb = r.shape[1]
        mirror = mgr.host_view(w).reshape(-1, bb)
        h_off = torch.from_numpy(mirror[s_off]).to(dev)
        check(torch.equal(r[ids_t], h_off), f"offload of the last step, storage {w}")
        h_rel = torch.from_numpy(mirror[s_rel]).to(dev)
        check(torch.equal(r[free_t], h_rel), f"reload of the last step, storage {w}")


def verify_round_trip(torch, mgr, storages, src, host, dst):
    """One offload + reload with the manager, outside any timed region (the
    reference's verify_roundtrip, perf_core.py:112-142): the device blocks
    dst must then hold the bytes src held before (a torch snapshot)."""
    dev = storages[0].device
    src_t = torch.tensor(src, device=dev)
    dst_t = torch.tensor(dst, device=dev)
    snap = [rows_u8(t)[src_t].clone() for t in storages]
    mgr.d2h(src, host, [1] * len(src)).Await()
    mgr.h2d(host, dst, [1] * len(dst)).Await()
    torch.cuda.synchronize()
    for w, t in enumerate(storages):
        check(torch.equal(rows_u8(t)[dst_t], snap[w]), f"round trip, storage {w}")


def box_copy(torch, pkg, src, dst, reps, stream):
    """The box's streaming-copy yardstick: the library's strided kernel over
    one contiguous entry (src -> dst, the same bytes as a gather launch),
    timed by HIP events right around each launch on the stream it runs on,
    as the block-copy launches are; read + write bytes per second (the best
    of 3 rounds). The copy is checked against its source."""
    plan = pkg.StridedPlan([pkg.StridedEntry(src.data_ptr(), dst.data_ptr(), src.numel())],
                           profile_kernels=True)
    pkg.copy_strided(plan, stream=stream).Await()
    plan.kernel_times(reset=True)
    best = 0.0
    for _ in range(3):
        for f in [pkg.copy_strided(plan, stream=stream) for _ in range(reps)]:
            f.Await()
        best = max(best, kernel_gbps(plan.kernel_times(reset=True)) or 0.0)
    torch.cuda.synchronize()
    check(torch.equal(dst, src), "box copy")
    plan.close()
    return best


def frac_of_box(gbps, box_gbps):
    return round(gbps / box_gbps, 4) if gbps and box_gbps else None


def torch_detile(torch, tiled, H, W, tH=8, tW=128, P=2):
    """The row-major [H, W] image of a 16-bit tensor stored in the
    {T(tH,tW)(P,1)} layout, by torch reshapes (an independent formulation of
    the nested tiling: pad to whole tiles, tiles row-major, P rows of a tile
    interleaved element by element)."""
    nT0, nT1 = -(-H // tH), -(-W // tW)
    t = tiled.view(nT0, nT1, tH // P, tW, P).transpose(-1, -2)
    t = t.reshape(nT0, nT1, tH, tW).permute(0, 2, 1, 3).reshape(nT0 * tH, nT1 * tW)
    return t[:H, :W]


def torch_tile(torch, x, tH=8, tW=128, P=2):
    """The inverse of torch_detile, padding written as zero."""
    H, W = x.shape
    nT0, nT1 = -(-H // tH), -(-W // tW)
    pad = torch.zeros(nT0 * tH, nT1 * tW, dtype=x.dtype, device=x.device)
    pad[:H, :W] = x
    t = pad.view(nT0, tH, nT1, tW).permute(0, 2, 1, 3).reshape(nT0, nT1, tH // P, P, tW)
    return t.transpose(-1, -2).contiguous().reshape(-1)


def bench_fp8_scales(torch, pkg, dev, args, rng):
    """fp8 KV (32 layers, 8 KV heads, head_dim 128, 16-token blocks, e4m3
    bytes) plus one fp32 scale per (layer, block, head): 512-block offload +
    reload at once, and the gather kernel moving payload and scales in one
    launch. Random payload bytes cover every e4m3 pattern (NaN, denormals);
    every moved byte is checked against torch indexing outside the timed
    regions."""
    L, P, H, n = 32, 16384, 8, 512
    bb = 16 * H * 128
    log(f"fp8: allocating {2 * L} x {P} x {bb} B pool + {L} scale tables")
    gen = torch.Generator(device=dev).manual_seed(1)
    kv = [torch.randint(0, 256, (P, bb), dtype=torch.uint8, device=dev, generator=gen)
          for _ in range(2 * L)]
    sc = [torch.randn(P, H, device=dev, generator=gen) for _ in range(L)]
    storages = kv + sc
    torch.cuda.synchronize()
    mgr = pkg.KVCacheManager(kv, host_blocks_to_allocate=4 * n, scale_tables=sc,
                             staging_chunk_bytes=args.chunk_mib << 20,
                             staging_chunks=args.chunks, profile_kernels=True)
    slots = [list(range(k * n, (k + 1) * n)) for k in range(4)]
    batch = batch_source(rng, P, n)
    ids, free = batch()
    verify_round_trip(torch, mgr, storages, ids, slots[0], free)
    step_bytes = 2 * n * (2 * L * bb + L * H * 4)
    el, last = run_duplex(torch, mgr, batch, slots, args.sub_steps, args.warmup)
    verify_duplex(torch, mgr, storages, slots, last)
    staging = torch.empty(n * (2 * L * bb + L * H * 4), dtype=torch.uint8, device=dev)
    s = torch.cuda.Stream(dev)
    id_sets = [batch()[0] for _ in range(16)]
    mgr.gather(id_sets[0], staging, stream=s).Await()
    mgr.kernel_times(True, reset=True)
    for f in [mgr.gather(id_sets[k % 16], staging, stream=s) for k in range(args.sub_steps)]:
        f.Await()
    g = kernel_gbps(mgr.kernel_times(True, reset=True))
    # The last gather's staging: payload then scales, storage by storage.
    last_ids = torch.tensor(id_sets[(args.sub_steps - 1) % 16], device=dev)
    want = torch.cat([rows_u8(t)[last_ids].reshape(-1) for t in storages])
    torch.cuda.synchronize()
    check(torch.equal(staging, want), "fp8 payload + scales gather")
    out = {"workload": "fp8 e4m3 KV + fp32 scale per (layer, block, head), Llama-3-8B shape",
           "offload_reload_gbps": round(args.sub_steps * step_bytes / el / 1e9, 2),
           "blocks_per_s": round(args.sub_steps * 2 * n / el, 1),
           "gather_payload_and_scales_gbps": round(g, 1) if g else None,
           "gather_frac_of_hbm_peak": round(g / HBM_PEAK_GBPS, 4) if g else None,
           "gather_frac_of_box_copy": frac_of_box(g, args.box_copy_gbps),
           "bytes_per_block": 2 * L * bb + L * H * 4,
           "verified": True}
    log(f"fp8: {out}")
    mgr.close()
    del kv, sc, storages, staging
    torch.cuda.empty_cache()
    return out


def llama3_8b_param_shapes():
    h, kvh, ffn, vocab = 4096, 1024, 14336, 128256
    shapes = [(vocab, h)]
    for _ in range(32):
        shapes += [(h,), (h, h), (kvh, h), (kvh, h), (h, h), (h,), (ffn, h), (ffn, h), (h, ffn)]
    return shapes + [(h,), (vocab, h)]


def verify_weight_image(torch, ws, tensors_u8, staging, what):
    """Every tensor's bytes at its offset-table position of `staging` (a
    device buffer holding the packed image)."""
    for k, t in enumerate(tensors_u8):
        _, nbytes, off = ws.host_buffer_info(k, 0)
        check(nbytes == t.numel() and torch.equal(staging[off:off + nbytes], t),
              f"{what}, tensor {k}")


def bench_weight_sync(torch, pkg, dev, args):
    """Llama-3-8B parameter set (291 bf16 tensors, 8.03e9 elements): device
    pack into one contiguous staging buffer via the offset table, pipelined
    pack + D2H to pinned host, H2D + unpack, and an 8-way column split of the
    226 2-D weights. Each is checked against torch outside its timed region:
    the packed image against the tensors, the host image against the packed
    image, H2D and unpack against a device copy of the tensors, the split
    chunks against torch column slices."""
    shapes = llama3_8b_param_shapes()
    log("weights: allocating 291 bf16 tensors (16.06 GB)")
    params = [torch.empty(s, dtype=torch.bfloat16, device=dev).normal_(0, 0.02)
              for s in shapes]
    ref = [t.clone() for t in params]
    as_u8 = [t.reshape(-1).view(torch.uint8) for t in params]
    torch.cuda.synchronize()  # the pack runs on a stream of its own
    total = sum(t.numel() * 2 for t in params)
    t0 = time.perf_counter()
    ws = pkg.WeightSynchronizer([[t] for t in params], profile_kernels=True)
    setup_s = time.perf_counter() - t0
    staging = torch.empty(ws.total_bytes, dtype=torch.uint8, device=dev)
    s = torch.cuda.Stream(dev)
    reps = max(3, args.sub_steps // 4)
    ws.pack(staging, stream=s).Await()
    ws.kernel_times(True, reset=True)
    for f in [ws.pack(staging, stream=s) for _ in range(reps)]:
        f.Await()
    pack_gbps = kernel_gbps(ws.kernel_times(True, reset=True))  # read+write counted once
    pack_gbps = pack_gbps * 2 if pack_gbps else None
    torch.cuda.synchronize()
    verify_weight_image(torch, ws, as_u8, staging, "pack")
    ws.d2h().Await()
    ws.kernel_times(True, reset=True)
    t0 = time.perf_counter()
    for _ in range(reps):
        ws.d2h().Await()
    d2h_gbps = reps * total / (time.perf_counter() - t0) / 1e9
    check(torch.equal(torch.from_numpy(ws.host_image()).to(dev), staging), "d2h host image")
    t0 = time.perf_counter()
    for _ in range(reps):
        ws.h2d().Await()
    h2d_gbps = reps * total / (time.perf_counter() - t0) / 1e9
    ws.kernel_times(True, reset=True)
    ws.kernel_times(False, reset=True)
    # H2D and unpack must restore tensors that were overwritten.
    for t in params:
        t.fill_(7)
    torch.cuda.synchronize()
    ws.h2d().Await()
    torch.cuda.synchronize()
    check(all(torch.equal(a, b) for a, b in zip(params, ref)), "h2d")
    for t in params:
        t.fill_(9)
    torch.cuda.synchronize()  # the unpack runs on s, which does not wait for the fill
    ws.unpack(staging, stream=s).Await()
    torch.cuda.synchronize()
    check(all(torch.equal(a, b) for a, b in zip(params, ref)), "unpack")
    del staging, ref
    # Column split: one launch over every 2-D weight.
    mats = [t for t in params if t.dim() == 2]
    entries, outs = [], []
    for m in mats:
        bounds = pkg.compute_nd_shard_slices(tuple(m.shape), (1, 8))
        chunk = [torch.empty(m.shape[0], b[1][1] - b[1][0], dtype=m.dtype, device=dev)
                 for b in bounds]
        entries += pkg.column_split_entries(m, chunk)
        outs.append(chunk)
    split_bytes = sum(m.numel() * 2 for m in mats)
    plan = pkg.StridedPlan(entries)  # the same split every sync: convert once
    pkg.copy_strided(plan, stream=s).Await()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record(s)
    for _ in range(reps):
        pkg.copy_strided(plan, stream=s)
    ev1.record(s)
    ev1.synchronize()
    split_s = ev0.elapsed_time(ev1) / 1e3 / reps
    for m, chunk in zip(mats, outs):
        c0 = 0
        for c in chunk:
            check(torch.equal(c, m[:, c0:c0 + c.shape[1]]), "column split")
            c0 += c.shape[1]
    split_gbps = 2 * split_bytes / split_s / 1e9
    out = {"workload": "Llama-3-8B parameter set, 291 bf16 tensors, 16.06 GB",
           "bytes": total, "pinned_host_setup_s": round(setup_s, 2),
           "pack_kernel_gbps": round(pack_gbps, 1) if pack_gbps else None,
           "pack_frac_of_hbm_peak": round(pack_gbps / HBM_PEAK_GBPS, 4) if pack_gbps else None,
           "pack_frac_of_box_copy": frac_of_box(pack_gbps, args.box_copy_gbps),
           "d2h_gbps": round(d2h_gbps, 2), "h2d_gbps": round(h2d_gbps, 2),
           "column_split_gbps": round(split_gbps, 1),
           "column_split_frac_of_hbm_peak": round(split_gbps / HBM_PEAK_GBPS, 4),
           "column_split_frac_of_box_copy": frac_of_box(split_gbps, args.box_copy_gbps),
           "column_split_entries": len(entries),
           "verified": True}
    log(f"weights: {out}")
    ws.close()
    del params, outs, mats
    torch.cuda.empty_cache()
    return out


def bench_weight_sync_tiled(torch, pkg, dev, args):
    """The Llama-3-8B parameter set stored tiled on the device, every tensor
    in the bf16 {T(8,128)(2,1)} layout (1-D norms as (1, 4096), padded to whole
    tiles): device detile + pack into one contiguous staging buffer, tile +
    unpack back (padding cleared), and the pipelined D2H / H2D whose host
    copies are the row-major images. Algorithmic bytes of a pack or unpack:
    2 x the logical bytes (16.06 GB read + written)."""
    shapes = llama3_8b_param_shapes()
    layouts = [pkg.tiling.TiledLayout(2, sh, [(8, 128), (2, 1)]) for sh in shapes]
    log("weights_tiled: allocating 291 tiled bf16 tensors")
    params = [torch.empty(L.tiled_bytes // 2, dtype=torch.int16, device=dev).random_()
              for L in layouts]
    torch.cuda.synchronize()  # the detile + pack runs on a stream of its own
    total = sum(L.logical_bytes for L in layouts)
    ws = pkg.WeightSynchronizer([[t] for t in params], layouts=[[L] for L in layouts],
                                profile_kernels=True)
    staging = torch.empty(ws.total_bytes, dtype=torch.uint8, device=dev)
    s = torch.cuda.Stream(dev)
    reps = max(3, args.sub_steps // 4)
    hw = [(1, sh[0]) if len(sh) == 1 else sh for sh in shapes]  # rank 1 tiles as (1, d0)

    def image(k):  # tensor k's row-major image in the packed staging buffer
        _, nbytes, off = ws.host_buffer_info(k, 0)
        return staging[off:off + nbytes].view(torch.int16).view(hw[k])

    ws.pack(staging, stream=s).Await()
    ws.kernel_times(True, reset=True)
    for f in [ws.pack(staging, stream=s) for _ in range(reps)]:
        f.Await()
    kt = ws.kernel_times(True, reset=True)
    detile_ms = kt["total_ms"] / reps if kt["launches"] else None
    torch.cuda.synchronize()
    for k, t in enumerate(params):
        check(torch.equal(image(k), torch_detile(torch, t, *hw[k])), f"detile + pack, tensor {k}")
    for f in [ws.unpack(staging, stream=s) for _ in range(reps)]:
        f.Await()
    kt = ws.kernel_times(False, reset=True)
    tile_ms = kt["total_ms"] / reps if kt["launches"] else None
    torch.cuda.synchronize()
    tiled_want = [torch_tile(torch, image(k)) for k in range(len(params))]
    for k, t in enumerate(params):
        check(torch.equal(t, tiled_want[k]), f"tile + unpack (padding zero), tensor {k}")
    ws.d2h().Await()
    t0 = time.perf_counter()
    for _ in range(reps):
        ws.d2h().Await()
    d2h_gbps = reps * total / (time.perf_counter() - t0) / 1e9
    check(torch.equal(torch.from_numpy(ws.host_image()).to(dev), staging), "tiled d2h host image")
    t0 = time.perf_counter()
    for _ in range(reps):
        ws.h2d().Await()
    h2d_gbps = reps * total / (time.perf_counter() - t0) / 1e9
    ws.kernel_times(True, reset=True)
    ws.kernel_times(False, reset=True)
    for t in params:
        t.fill_(3)
    torch.cuda.synchronize()
    ws.h2d().Await()
    torch.cuda.synchronize()
    check(all(torch.equal(t, w) for t, w in zip(params, tiled_want)), "tiled h2d")
    del tiled_want
    # The reference detiles on the host after the raw DMA (DetileBufferNDOptimized,
    # 4 threads): its restatement in the oracle, timed on one MLP weight.
    import numpy as np
    sys.path.insert(0, ROOT)
    import oracle
    H, W = 14336, 4096
    src = np.random.default_rng(0).integers(0, 256, H * W * 2, dtype=np.uint8)
    dst = np.empty_like(src)
    cpu = {}
    for nthreads in (4, min(16, os.cpu_count() or 1)):
        oracle.detile_std(2, 1, H, W, 8, 128, 2, src, dst, nthreads)
        reps, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < 1.0:
            oracle.detile_std(2, 1, H, W, 8, 128, 2, src, dst, nthreads)
            reps += 1
        cpu[nthreads] = 2 * src.nbytes * reps / (time.perf_counter() - t0) / 1e9
    out = {"workload": "Llama-3-8B parameter set, 291 bf16 tensors in the T(8,128)(2,1) tiled "
                       "layout, 16.06 GB logical",
           "bytes": total, "tiled_bytes": sum(L.tiled_bytes for L in layouts),
           "detile_pack_ms": round(detile_ms, 3) if detile_ms else None,
           "detile_pack_gbps": round(2 * total / detile_ms / 1e6, 1) if detile_ms else None,
           "detile_pack_frac_of_hbm_peak": round(2 * total / detile_ms / 1e6 / HBM_PEAK_GBPS, 4)
           if detile_ms else None,
           "detile_pack_frac_of_box_copy": frac_of_box(2 * total / detile_ms / 1e6, args.box_copy_gbps)
           if detile_ms else None,
           "tile_unpack_ms": round(tile_ms, 3) if tile_ms else None,
           "tile_unpack_gbps": round(2 * total / tile_ms / 1e6, 1) if tile_ms else None,
           "tile_unpack_frac_of_hbm_peak": round(2 * total / tile_ms / 1e6 / HBM_PEAK_GBPS, 4)
           if tile_ms else None,
           "tile_unpack_frac_of_box_copy": frac_of_box(2 * total / tile_ms / 1e6, args.box_copy_gbps)
           if tile_ms else None,
           "verified": True,
           # HBM bytes per launch from rocprofv3 FETCH_SIZE / WRITE_SIZE with the
           # same calibration (profiles/tiled_copy_weight_sync_trace.txt).
           "detile_pack_traffic": int((7844374.1 / 0.50001 + 15684196.2) * 1024),
           "tile_unpack_traffic": int((7844090.4 / 0.50001 + 15692041.6) * 1024),
           "d2h_gbps": round(d2h_gbps, 2), "h2d_gbps": round(h2d_gbps, 2),
           "cpu_baseline": {"value": round(cpu[4], 2), "unit": "GB/s", "cores": 4, "kind": "port",
                            "all_threads_gbps": round(cpu[max(cpu)], 2), "all_threads": max(cpu),
                            "cpu_model": cpu_model(),
                            "sample": "one [14336, 4096] bf16 weight detiled from T(8,128)(2,1) "
                                      "on the host by the oracle's restatement of the reference's "
                                      "threaded routine (4 threads, as the reference), GB/s counted "
                                      "as 2 x bytes like the kernel"}}
    ws.close()
    del params, staging
    torch.cuda.empty_cache()
    out["int8_quads"] = bench_tiled_int8(torch, pkg, dev, args)
    log(f"weights_tiled: {out}")
    return out


def bench_tiled_int8(torch, pkg, dev, args):
    """Weights packed four 8-bit elements to a word: 8 int8 [14336, 8192]
    matrices (0.94 GB) in T(8,128)(4,1), detile + pack and tile + unpack
    through the weight synchronizer's device pack / unpack, each checked
    against the torch formulation of the tiling."""
    H, W, n = 14336, 8192, 8
    lay = pkg.tiling.TiledLayout(1, (H, W), [(8, 128), (4, 1)])
    params = [torch.empty(lay.tiled_bytes, dtype=torch.uint8, device=dev).random_(0, 256)
              for _ in range(n)]
    torch.cuda.synchronize()
    total = n * lay.logical_bytes
    ws = pkg.WeightSynchronizer([[t] for t in params], layouts=[[lay]] * n, profile_kernels=True)
    staging = torch.empty(ws.total_bytes, dtype=torch.uint8, device=dev)
    s = torch.cuda.Stream(dev)
    reps = max(3, args.sub_steps // 2)

    def image(k):
        _, nbytes, off = ws.host_buffer_info(k, 0)
        return staging[off:off + nbytes].view(H, W)

    out = {"workload": f"{n} int8 [{H}, {W}] matrices in T(8,128)(4,1), {total / 1e9:.2f} GB"}
    ws.pack(staging, stream=s).Await()
    ws.kernel_times(True, reset=True)
    for f in [ws.pack(staging, stream=s) for _ in range(reps)]:
        f.Await()
    kt = ws.kernel_times(True, reset=True)
    torch.cuda.synchronize()
    for k, t in enumerate(params):
        check(torch.equal(image(k), torch_detile(torch, t, H, W, 8, 128, 4)),
              f"int8 detile + pack, tensor {k}")
    for f in [ws.unpack(staging, stream=s) for _ in range(reps)]:
        f.Await()
    kt2 = ws.kernel_times(False, reset=True)
    torch.cuda.synchronize()
    for k, t in enumerate(params):
        check(torch.equal(t, torch_tile(torch, image(k), 8, 128, 4)),
              f"int8 tile + unpack, tensor {k}")
    for name, kt_ in (("detile_pack", kt), ("tile_unpack", kt2)):
        ms = kt_["total_ms"] / reps
        g = 2 * total / ms / 1e6
        out[f"{name}_gbps"] = round(g, 1)
        out[f"{name}_frac_of_hbm_peak"] = round(g / HBM_PEAK_GBPS, 4)
        out[f"{name}_frac_of_box_copy"] = frac_of_box(g, args.box_copy_gbps)
    # HBM bytes per launch from rocprofv3 FETCH_SIZE / WRITE_SIZE with the
    # same calibration (profiles/tiled_copy_weight_sync_trace.txt).
    out["detile_pack_traffic"] = int((458919.1 / 0.50001 + 917621.9) * 1024)
    out["tile_unpack_traffic"] = int((458925.5 / 0.50001 + 917616.7) * 1024)
    out["verified"] = True
    ws.close()
    del params, staging
    torch.cuda.empty_cache()
    return out


def bench_pools(torch, pkg, dev, args, rng):
    """Pool-addressed copies of a sparse (FA-like) pool: per block 4 head
    groups of 64 tokens x (K 256 B + V 256 B) packed at 70 KiB pitch inside a
    320 KiB block stride (40 % live). 32 storages x 512 blocks; each step
    copies 128 random blocks of every pool device->host, then host->device,
    moving only the live bytes (one strided-copy launch per pool over the
    pinned mirror; with a malloc mirror the live bytes are packed into staging
    chunks and cross PCIe through the bounce lanes), against whole-block
    copies of the same ids."""
    L, NB, stride = 32, 512, 327680
    regions = tuple(pkg.RegionSpec("fa%d" % g, g * 71680, 512, 256, 64, 2) for g in range(4))
    live = sum(r.live_bytes for r in regions)
    log(f"pools: allocating {L} x {NB} x {stride} B storages")
    pools = [torch.empty(NB, stride, dtype=torch.uint8, device=dev) for _ in range(L)]
    for p in pools:
        p.random_(0, 256)
    torch.cuda.synchronize()
    mgr = pkg.KVCacheManager(pools, host_blocks_to_allocate=NB,
                             host_alloc=args.pools_host_alloc)
    specs = [pkg.PoolSpec("fa", l, 0, stride, NB, regions) for l in range(L)]
    mgr.register_pools(specs)
    n = 128

    def timed(fn, reps):
        fn()
        mgr.wait_for_pending_work()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        mgr.wait_for_pending_work()
        return (time.perf_counter() - t0) / reps

    ids = sorted(rng.choice(NB, n, replace=False).tolist())
    reps = max(3, args.sub_steps // 2)

    def pool_copy(d2h):
        fn = mgr.d2h_pool_blocks if d2h else mgr.h2d_pool_blocks
        futs = [fn(l, ids) for l in range(L)]
        for f in futs:
            f.Await()

    t_d2h = timed(lambda: pool_copy(True), reps)
    t_h2d = timed(lambda: pool_copy(False), reps)
    t_dense = timed(lambda: mgr.d2h(ids, ids).Await(), reps)
    # Live bytes by the regions' definition: unit u of a region covers
    # [offset + u * stride, offset + u * stride + units_per_stride * unit).
    mask_np = np.zeros(stride, bool)
    for r in regions:
        for u in range(r.num_units):
            a = r.offset_bytes + u * r.stride_bytes
            mask_np[a:a + r.units_per_stride * r.unit_bytes] = True
    mask = torch.from_numpy(mask_np).to(dev)
    ids_t = torch.tensor(ids, device=dev)
    # D2H onto zeroed host blocks: the live bytes arrive, the padding stays 0.
    for l in range(L):
        host_rows(mgr, l, stride, 0, NB)[ids] = 0
    pool_copy(True)
    for l in range(L):
        h = torch.from_numpy(host_rows(mgr, l, stride, 0, NB)[ids]).to(dev)
        d = pools[l][ids_t]
        check(torch.equal(h[:, mask], d[:, mask]) and not h[:, ~mask].any(),
              f"pool d2h, storage {l}")
    # H2D of new host bytes: live bytes land, the device padding is untouched.
    for l in range(L):
        hr = host_rows(mgr, l, stride, 0, NB)
        hr[ids] = rng.integers(0, 256, (n, stride), dtype=np.uint8)
    before = [pools[l][ids_t].clone() for l in range(L)]
    pool_copy(False)
    torch.cuda.synchronize()
    for l in range(L):
        h = torch.from_numpy(host_rows(mgr, l, stride, 0, NB)[ids]).to(dev)
        d = pools[l][ids_t]
        check(torch.equal(d[:, mask], h[:, mask]) and torch.equal(d[:, ~mask], before[l][:, ~mask]),
              f"pool h2d, storage {l}")
    del before
    live_bytes = L * n * live
    out = {"workload": "FA-like sparse pool (4 head groups x 32 KiB live per 320 KiB block), "
                       f"{L} storages x {NB} blocks, {n} random blocks per copy",
           "live_fraction": round(live / stride, 3),
           "host_mirror": args.pools_host_alloc,
           "pool_d2h_live_gbps": round(live_bytes / t_d2h / 1e9, 2),
           "pool_h2d_live_gbps": round(live_bytes / t_h2d / 1e9, 2),
           "pool_d2h_ms": round(t_d2h * 1e3, 3),
           "whole_block_d2h_ms": round(t_dense * 1e3, 3),
           "speedup_vs_whole_blocks": round(t_dense / t_d2h, 2),
           "verified": True}
    log(f"pools: {out}")
    mgr.close()
    del pools
    torch.cuda.empty_cache()
    return out


def zipf_host_blocks(args, block_bytes):
    """Host tier of the churn in blocks, and what set it: the configuration's
    256 GB budget, capped by free /dev/shm (for the shm tier), available RAM
    and a 160 GiB process budget (the pool's pinned staging, the bounce lanes
    and the interpreter need the rest of the host memory a process may use)."""
    if args.zipf_host_blocks > 0:
        return args.zipf_host_blocks, "--zipf-host-blocks"
    if args.zipf_host_alloc == "pinned":
        # Page-locked allocations much beyond this were refused (out of memory).
        return 2048, "pinned tier: 10 GiB"
    limits = {"configured 256 GB budget": 256e9, "160 GiB process budget": float(160 << 30)}
    st = os.statvfs("/dev/shm")
    limits["80% of free /dev/shm"] = 0.8 * st.f_bavail * st.f_frsize
    try:
        with open("/proc/meminfo") as f:
            kb = {ln.split(":")[0]: int(ln.split()[1]) for ln in f if ln.strip()}
        limits["60% of MemAvailable"] = 0.6 * kb["MemAvailable"] * 1024
    except (OSError, KeyError, ValueError):
        pass
    name, lim = min(limits.items(), key=lambda kv: kv[1])
    return int(lim // block_bytes), name


def percentiles_ms(xs):
    if not xs:
        return None
    a = np.sort(np.asarray(xs)) * 1e3
    return {"count": len(xs), "p50": round(float(np.percentile(a, 50)), 2),
            "p99": round(float(np.percentile(a, 99)), 2), "max": round(float(a[-1]), 2)}


def requests_to_keep(window, inflight):
    """The requests a caller with at most `inflight` in flight may leave in
    flight after issuing the newest of `window` (oldest first): the newest
    inflight - 1 of them, or all while there are fewer."""
    if inflight <= 1:
        return []
    return window[max(0, len(window) - (inflight - 1)):]

def pcie_rates(q_load, q_save, peaks):
    """Bytes/s of the H2D and D2H directions with q_load and q_save bytes
    queued: a direction alone runs at its pinned peak; both at once share the
    bidirectional peak in proportion to their queued bytes, each capped at its
    own peak (the split that drains both queues together)."""
    h2d, d2h = peaks["pcie_h2d_gbps"] * 1e9, peaks["pcie_d2h_gbps"] * 1e9
    bidir = peaks["pcie_bidir_gbps"] * 1e9
    if q_load <= 0 or q_save <= 0:
        return h2d, d2h
    rl = bidir * q_load / (q_load + q_save)
    if rl > h2d:
        return h2d, min(d2h, bidir - h2d)
    if bidir - rl > d2h:
        return min(h2d, bidir - d2h), d2h
    return rl, bidir - rl


def window_bound_gbps(per_request, inflight, peaks, block_bytes):
    """PCIe bound of a request stream issued as the churn issues it: request
    j is issued once every request before j - inflight + 1 has finished both
    copies; its load (H2D) and save (D2H) join their direction's queue at
    issue and each queue runs in order, at pcie_rates. Host time between
    requests and per-copy latencies count as zero, so no copy engine can do
    better under that window. With one in flight this is the per-request
    bound sum(max(load / H2D, save / D2H, (load + save) / bidir)); with every
    request issued at once it is the fully overlapped bound."""
    from collections import deque
    n = len(per_request)
    pending = [0] * n  # copies of each request not yet finished
    loads, saves = deque(), deque()  # [request, bytes left], in issue order
    q_load = q_save = 0.0
    t = 0.0
    issued = oldest = 0  # oldest: first request with a copy unfinished
    while True:
        while issued < n and issued - oldest < inflight:
            nl, ns = per_request[issued]
            if nl > 0:
                loads.append([issued, float(nl) * block_bytes])
                q_load += float(nl) * block_bytes
                pending[issued] += 1
            if ns > 0:
                saves.append([issued, float(ns) * block_bytes])
                q_save += float(ns) * block_bytes
                pending[issued] += 1
            issued += 1
            while oldest < issued and pending[oldest] == 0:
                oldest += 1
        if not loads and not saves:
            break
        rl, rs = pcie_rates(q_load, q_save, peaks)
        dl = loads[0][1] / rl if loads else float("inf")
        ds = saves[0][1] / rs if saves else float("inf")
        dt = min(dl, ds)
        t += dt
        for q, r, first in ((loads, rl, dl <= ds), (saves, rs, ds <= dl)):
            if not q:
                continue
            q[0][1] = 0.0 if first else q[0][1] - r * dt
            if q is loads:
                q_load = max(0.0, q_load - r * dt)
            else:
                q_save = max(0.0, q_save - r * dt)
            if q[0][1] <= 0.0:
                pending[q.popleft()[0]] -= 1
        if not loads:
            q_load = 0.0
        if not saves:
            q_save = 0.0
        while oldest < issued and pending[oldest] == 0:
            oldest += 1
    moved = sum(nl + ns for nl, ns in per_request) * block_bytes
    return moved / t / 1e9 if t > 0 else None


def bench_zipf_store(torch, pkg, dev, args, rng, peaks=None):
    """Llama-3-70B-shaped KV (80 layers, K and V: 160 storages of 12000 x 32
    KiB blocks, 58.6 GiB) with a host LRU tier (default: a /dev/shm segment of
    the configured 256 GB budget, or as much of it as the machine allows)
    behind the KVCacheStore; prefix-cache churn: each request is a prefix of
    one of --zipf-docs documents' block-hash chains (document drawn Zipf(1.1),
    length 64-2048 blocks log-uniform). Lookup returns the cached prefix,
    which is loaded into device blocks; the rest is inserted and saved
    (evicting LRU entries once the host tier is full). Load (H2D) and save
    (D2H) of a request are issued together; up to --zipf-inflight requests
    have copies in flight (the next request is looked up and issued while the
    previous one's copies run), as in a server with several requests in
    progress. With one request in flight, each request's latency (lookup to
    both copies polled done) is recorded. Then the same request stream
    continues on the warm tier with --zipf-more-inflight requests in flight."""
    L, P, bb = 80, 12000, 32768
    S = 2 * L
    host_blocks, tier_limit = zipf_host_blocks(args, S * bb)
    log(f"zipf: allocating {S} x {P} x {bb} B pool ({S * P * bb / 2**30:.1f} GiB), "
        f"{host_blocks} host blocks ({host_blocks * S * bb / 2**30:.1f} GiB "
        f"{args.zipf_host_alloc}, limit: {tier_limit})")
    pools = [torch.empty(P, bb, dtype=torch.uint8, device=dev) for _ in range(S)]
    for p in pools:
        p.random_(0, 256)
    torch.cuda.synchronize()
    store = pkg.KVCacheStore(capacity=host_blocks, num_shards=1, store_server_ip="127.0.0.1",
                             metadata_shm_key="")
    tier = {}
    if args.zipf_host_alloc == "shm":
        tier = {"host_alloc": "shm", "shm_key": f"kvx_bench_{os.getpid()}"}
    t_tier = time.perf_counter()
    mgr = pkg.KVCacheManager(pools, host_blocks_to_allocate=host_blocks,
                             staging_chunk_bytes=(args.zipf_chunk_mib or args.chunk_mib) << 20,
                             staging_chunks=args.zipf_chunks,
                             host_copy_threads=args.zipf_host_threads,
                             transfer_mode=args.zipf_mode,
                             raiden_controller_address=store.raiden_controller_address,
                             **tier)
    t_tier = time.perf_counter() - t_tier
    log(f"zipf: host tier ready in {t_tier:.1f} s")
    rid = store.raiden_id
    docs = args.zipf_docs
    w = 1.0 / np.arange(1, docs + 1) ** 1.1
    cdf = np.cumsum(w) / w.sum()

    done_l = done_s = 0
    loading = set()  # hashes whose load has not been polled done

    def poll_until(want_load, want_save):
        nonlocal done_l, done_s
        while done_l < want_load or done_s < want_save:
            if done_l < want_load:
                done, failed = store.poll_load_status()[:2]
                if failed:
                    raise RuntimeError(f"store load failed: {len(failed)} blocks")
                done_l += len(done)
                loading.difference_update(done)
            if done_s < want_save:
                done, failed = store.poll_save_status()[:2]
                if failed:
                    raise RuntimeError(f"store save failed: {len(failed)} blocks")
                done_s += len(done)

    def run(inflight, batches):
        """batches requests with up to `inflight` in flight; returns the
        phase's counters, per-request latencies (one in flight) and sizes."""
        nonlocal done_l, done_s
        done_l = done_s = 0
        saved = loaded = hits = asked = skipped = device_hits = replaced = 0
        window = []  # (loads, saves) of the requests possibly still in flight
        latency = []  # (blocks, seconds) per request, one request in flight
        # Per request, seconds from its lookup until both copies are issued,
        # and of that the store's load and save calls.
        issue = []
        per_request = []  # (blocks loaded, blocks saved) per request
        t0 = time.perf_counter()
        for step in range(batches):
            doc = int(np.searchsorted(cdf, rng.random()))
            nb = int(np.exp(rng.uniform(np.log(64), np.log(2048))))
            chain = [b"d%03d:%05d" % (doc, i) for i in range(nb)]
            dev_ids = rng.permutation(P)[:nb].tolist()
            # A request's latency runs from its lookup (the request itself is
            # drawn above) until both of its copies are polled done.
            t_req = time.perf_counter()
            found = store.lookup(chain, pin_found=True)
            k = len(found)
            rest = chain[k:]
            # Host-resident hits are loaded; an HBM-only entry (inserted by a
            # request whose save could not get host blocks, or whose save is
            # still in flight) names a device block the caller owns: a hit
            # with nothing to move. A block another request in flight is
            # loading arrives with that load: also a hit with nothing to move.
            on_host = (pkg.BlockStatus.HOST, pkg.BlockStatus.HOST_AND_HBM)
            to_load = [b.status in on_host and h not in loading for h, b in found]
            load_h = [h for (h, _), t in zip(found, to_load) if t]
            load_d = [dev_ids[i] for i, t in enumerate(to_load) if t]
            in_hbm = [h for (h, _), t in zip(found, to_load) if not t]
            if in_hbm:
                store.release(in_hbm)
                device_hits += len(in_hbm)
            t_call = time.perf_counter()
            if load_h and not store.load(load_h, load_d):
                raise RuntimeError(f"store load of {len(load_h)} blocks failed: "
                                   f"{store.last_error()}")
            t_load_call = time.perf_counter() - t_call
            loading.update(load_h)
            n_save = 0
            t_save_call = 0.0
            if rest:
                # Chain blocks past the cached prefix that are still on the
                # host (their prefix was evicted first) cannot be reached
                # through a prefix lookup any more; the request's fresh
                # copies replace them.
                replaced += store.evict(rest)
                sl = [pkg.RaidenBlockId(rid, -1, d, pkg.BlockStatus.HBM) for d in dev_ids[k:]]
                if store.insert(rest, sl, on_host=False):
                    t_call = time.perf_counter()
                    saved_ok = store.save(rest)
                    t_save_call = time.perf_counter() - t_call
                    if saved_ok:
                        n_save = len(rest)
                    else:  # no host blocks to spare, or a block pinned by another request
                        store.release(rest)
                        skipped += len(rest)
                else:  # another request in flight inserted some of them
                    skipped += len(rest)
            loaded += len(load_h)
            saved += n_save
            hits += k
            asked += nb
            window.append((len(load_h), n_save))
            issue.append((time.perf_counter() - t_req, t_load_call, t_save_call))
            # Keep at most `inflight` requests in flight: wait until every
            # copy but those of the newest inflight - 1 requests has landed.
            keep = requests_to_keep(window, inflight)
            poll_until(loaded - sum(x[0] for x in keep), saved - sum(x[1] for x in keep))
            window = keep
            if inflight == 1:
                latency.append((nb, time.perf_counter() - t_req))
            per_request.append((len(load_h), n_save))
        poll_until(loaded, saved)
        t_run = time.perf_counter() - t0
        return dict(saved=saved, loaded=loaded, hits=hits, asked=asked, skipped=skipped,
                    device_hits=device_hits, replaced=replaced, t_run=t_run,
                    latency=latency, issue=issue, per_request=per_request)

    inflight = max(1, args.zipf_inflight)
    r = run(inflight, args.zipf_batches)
    saved, loaded, hits, asked = r["saved"], r["loaded"], r["hits"], r["asked"]
    skipped, device_hits, replaced = r["skipped"], r["device_hits"], r["replaced"]
    latency, per_request, t_run = r["latency"], r["per_request"], r["t_run"]
    issue = r["issue"]
    moved = (saved + loaded) * S * bb
    # PCIe bound of this request stream: a request's load (H2D) and save (D2H)
    # run at once, each at most at its direction's measured pinned peak and
    # together at most at the measured bidirectional peak, and requests
    # follow one another, so the stream needs at least
    # sum(max(load / H2D peak, save / D2H peak, (load + save) / bidir peak)).
    # pcie_bound_per_direction_gbps leaves out the bidirectional term.
    pcie_bound = pcie_bound_dir = None
    small_vs_bound = None
    if peaks and inflight == 1:
        t_dir = t_min = 0.0
        req_bound = []  # each request's own PCIe time at the measured peaks
        for l, sv in per_request:
            tl = l * S * bb / (peaks["pcie_h2d_gbps"] * 1e9)
            ts = sv * S * bb / (peaks["pcie_d2h_gbps"] * 1e9)
            t_dir += max(tl, ts)
            req_bound.append(max(tl, ts, (l + sv) * S * bb / (peaks["pcie_bidir_gbps"] * 1e9)))
            t_min += req_bound[-1]
        if t_min > 0:
            pcie_bound = moved / t_min / 1e9
            pcie_bound_dir = moved / t_dir / 1e9
        # Small requests (64-127 blocks): latency against the request's own
        # PCIe time, which separates per-request overhead from bytes moved.
        small = [(t, b, l + sv, ti) for (nb, t), b, (l, sv), ti
                 in zip(latency, req_bound, per_request, issue) if nb < 128 and b > 0]
        if small:
            ratios = sorted(t / b for t, b, _, _ in small)
            over_ms = sorted((t - b) * 1e3 for t, b, _, _ in small)
            small_vs_bound = {
                "count": len(small),
                "median_blocks_moved": int(np.median([m for _, _, m, _ in small])),
                "median_pcie_bound_ms": round(float(np.median([b for _, b, _, _ in small])) * 1e3, 2),
                "median_latency_over_bound": round(ratios[len(ratios) // 2], 3),
                "median_ms_above_bound": round(over_ms[len(over_ms) // 2], 2),
                # Host time from the lookup until the load and save are
                # issued (store lookup / release / evict / insert / save /
                # load calls), part of the time above the bound; and of it
                # the load and save calls (which plan and enqueue the copies).
                "median_issue_ms": round(float(np.median([ti[0] for *_, ti in small])) * 1e3, 2),
                "median_load_call_ms": round(float(np.median([ti[1] for *_, ti in small])) * 1e3, 2),
                "median_save_call_ms": round(float(np.median([ti[2] for *_, ti in small])) * 1e3, 2)}
    out = {"workload": "Llama-3-70B-shaped KV (80 layers, 12000-block pool), prefix-cache "
                       "churn through the KV store: requests are prefixes (64-2048 blocks) of "
                       f"{docs} documents' hash chains, document drawn Zipf(1.1)",
           "host_tier_blocks": host_blocks, "host_tier_memory": args.zipf_host_alloc,
           "host_tier_gib": round(host_blocks * S * bb / 2**30, 1),
           "host_tier_limit": tier_limit, "host_tier_setup_s": round(t_tier, 1),
           "batches": args.zipf_batches, "requests_in_flight": inflight,
           "staging_chunk_mib": args.zipf_chunk_mib or args.chunk_mib,
           "staging_chunks": args.zipf_chunks,
           "transfer_mode": args.zipf_mode, "engine_stats": mgr.engine_stats(),
           "host_copy_threads": args.zipf_host_threads or 8,
           "blocks_saved": saved, "blocks_loaded": loaded,
           "blocks_skipped": skipped, "device_hits": device_hits,
           "stale_suffix_blocks_replaced": replaced,
           "blocks_evicted_lru": max(0, saved - replaced - store.size()),
           "hit_rate": round(hits / max(asked, 1), 4),
           "gbps": round(moved / t_run / 1e9, 2),
           "pcie_bound_gbps": round(pcie_bound, 2) if pcie_bound else None,
           "frac_of_pcie_bound": round(moved / t_run / 1e9 / pcie_bound, 4)
                                 if pcie_bound else None,
           "pcie_bound_per_direction_gbps": round(pcie_bound_dir, 2) if pcie_bound_dir else None,
           "blocks_per_s": round((saved + loaded) / t_run, 1),
           "latency_ms": ({"all_requests": percentiles_ms([t for _, t in latency]),
                           "requests_64_to_127_blocks": percentiles_ms(
                               [t for nb, t in latency if nb < 128])}
                          if latency else None),
           "requests_64_to_127_blocks_vs_pcie_bound": small_vs_bound}
    more = []
    for m in (int(x) for x in str(args.zipf_more_inflight).split(",") if x.strip()):
        if m < 2:
            continue
        # The same request stream continued on the warm tier with more
        # requests in flight, as a server with several requests in progress.
        r2 = run(m, args.zipf_batches)
        moved2 = (r2["saved"] + r2["loaded"]) * S * bb
        e = {"requests_in_flight": m, "batches": args.zipf_batches,
             "blocks_saved": r2["saved"], "blocks_loaded": r2["loaded"],
             "blocks_skipped": r2["skipped"], "device_hits": r2["device_hits"],
             "hit_rate": round(r2["hits"] / max(r2["asked"], 1), 4),
             "gbps": round(moved2 / r2["t_run"] / 1e9, 2),
             "blocks_per_s": round((r2["saved"] + r2["loaded"]) / r2["t_run"], 1)}
        if peaks:
            # With requests overlapping freely the stream can do no better
            # than all loads on H2D, all saves on D2H and everything on the
            # bidirectional peak at once.
            t_lo = max(r2["loaded"] * S * bb / (peaks["pcie_h2d_gbps"] * 1e9),
                       r2["saved"] * S * bb / (peaks["pcie_d2h_gbps"] * 1e9),
                       moved2 / (peaks["pcie_bidir_gbps"] * 1e9))
            if t_lo > 0:
                e["pcie_bound_overlapped_gbps"] = round(moved2 / t_lo / 1e9, 2)
                e["frac_of_overlapped_bound"] = round(moved2 / r2["t_run"] / (moved2 / t_lo), 4)
            # The bound of this stream under its own window: requests are
            # issued only as older ones finish, so a direction idles when the
            # requests in flight have nothing queued for it.
            wb = window_bound_gbps(r2["per_request"], m, peaks, S * bb)
            if wb:
                e["pcie_bound_window_gbps"] = round(wb, 2)
                e["frac_of_window_bound"] = round(moved2 / r2["t_run"] / 1e9 / wb, 4)
        more.append(e)
        log(f"zipf: {m} in flight: {e}")
    if more:
        out["more_in_flight"] = more
    # One offload + reload through the same manager and host tier after the
    # churn (its lanes, chunking and /dev/shm tier), checked against torch.
    perm = rng.permutation(P)
    verify_round_trip(torch, mgr, pools, perm[:512].tolist(),
                      rng.permutation(host_blocks)[:512].tolist(), perm[512:1024].tolist())
    out["verified"] = True
    log(f"zipf: {out}")
    mgr.close()
    store.close()
    if tier:
        # The library never unlinks a host-tier segment (it outlives the
        # process by design); the benchmark removes its own.
        seg = f"/dev/shm/{tier['shm_key']}_dev_{dev.index or 0}"
        if os.path.exists(seg):
            os.unlink(seg)
    del pools
    torch.cuda.empty_cache()
    return out


def bench_lanes(torch, pkg, dev, args, rng):
    """Loads and saves through the pageable lanes on the Llama-3-70B block
    shape (160 storages x 32 KiB per block): a 2048-block /dev/shm tier,
    requests of 64 and 512 random blocks, each direction alone and both at
    once (a store request issues its load and save together), 32 MiB staging
    chunks. Median over the repetitions; GB/s counts both directions' bytes."""
    S, P, bb, HB = 160, 4096, 32768, 2048
    log(f"lanes: {S} x {P} x {bb} B pool, {HB}-block /dev/shm tier")
    pools = [torch.empty(P, bb, dtype=torch.uint8, device=dev) for _ in range(S)]
    for p in pools:
        p.random_(0, 256)
    torch.cuda.synchronize()
    key = f"kvx_lanes_{os.getpid()}"
    mgr = pkg.KVCacheManager(pools, host_blocks_to_allocate=HB, staging_chunk_bytes=32 << 20,
                             staging_chunks=args.zipf_chunks, host_alloc="shm", shm_key=key)
    out = {"workload": "Llama-3-70B block shape (160 storages x 32 KiB), /dev/shm tier of "
                       f"{HB} blocks, random device and host ids, {args.zipf_chunks} staging "
                       "chunks of 32 MiB"}
    for nb, reps in ((64, 12), (512, 6)):
        t = {"save_ms": [], "load_ms": [], "load_and_save_ms": []}
        one = [1] * nb
        for r in range(reps + 1):
            dev_ids = rng.permutation(P)[:nb].tolist()
            host_ids = rng.permutation(HB)[:nb].tolist()
            dev2 = rng.permutation(P)[:nb].tolist()
            host2 = rng.permutation(HB)[:nb].tolist()
            t0 = time.perf_counter()
            mgr.d2h(dev_ids, host_ids, one).Await()
            a = time.perf_counter() - t0
            t0 = time.perf_counter()
            mgr.h2d(host_ids, dev2, one).Await()
            b = time.perf_counter() - t0
            t0 = time.perf_counter()
            f1 = mgr.h2d(host_ids, dev_ids, one)
            f2 = mgr.d2h(dev2, host2, one)
            f1.Await()
            f2.Await()
            c = time.perf_counter() - t0
            if r > 0:  # the first round warms the lanes
                t["save_ms"].append(a * 1e3)
                t["load_ms"].append(b * 1e3)
                t["load_and_save_ms"].append(c * 1e3)
        nbytes = nb * S * bb
        res = {}
        for k, v in t.items():
            med = float(np.median(v))
            res[k] = round(med, 2)
            res[k.replace("_ms", "_gbps")] = round((2 if "and" in k else 1) * nbytes / med / 1e6, 2)
        out[f"requests_of_{nb}_blocks"] = res
        log(f"lanes {nb} blocks: {res}")
    out["lane_dma_engines"] = mgr.lane_dma_engines
    perm = rng.permutation(P)
    verify_round_trip(torch, mgr, pools, perm[:512].tolist(),
                      rng.permutation(HB)[:512].tolist(), perm[512:1024].tolist())
    out["verified"] = True
    mgr.close()
    seg = f"/dev/shm/{key}_dev_{dev.index or 0}"
    if os.path.exists(seg):
        os.unlink(seg)
    del pools
    torch.cuda.empty_cache()
    return out


# The reference's published raw-transfer figures on Ironwood (8 chips, 256
# layers, 32 blocks), aggregate over the 8 chips: (H2D, D2H) GB/s per dtype
# (examples/microbenchmarks/RAW_TRANSFER.md, "Benchmark Results").
REFERENCE_SCENARIO_GBPS = {
    "A": {"fp8": (78.50, 78.95), "bf16": (154.67, 148.79), "f32": (189.27, 184.97),
          "int32": (190.62, 186.07)},
    "B": {"fp8": (176.75, 173.43), "bf16": (183.38, 182.56), "f32": (192.88, 188.24),
          "int32": (193.89, 189.00)},
}


def bench_reference_scenarios(torch, pkg, dev, args, peaks):
    """The reference's raw-transfer microbenchmark at one device's share
    (tpu_sync/core/kv_cache_manager_perf_test.cc:146-185, 336-366): 32 layers
    x 32 blocks of [128 tokens, 8 heads, K/V, 128]. Scenario A: one array per
    layer, [32, 128, 8, 2, 128]; Scenario B: one block-major array
    [32, 32, 128, 8, 2, 128]. D2H copies the 16 odd blocks to the same host
    blocks and H2D the 16 odd host blocks to the even device blocks, each as
    one KVCacheManager.d2h / h2d call; afterwards every even device block
    must equal its odd neighbour (the reference's own check). GB/s = bytes
    moved / mean call time (the reference reports the mean), beside the
    published figure per chip (the 8-chip aggregate / 8)."""
    dtypes = {"fp8": torch.float8_e4m3fn, "bf16": torch.bfloat16, "f32": torch.float32,
              "int32": torch.int32}
    odd, even, ones = list(range(1, 32, 2)), list(range(0, 32, 2)), [1] * 16
    iters, warm = max(5, args.sub_steps), 3
    out = {"workload": "reference raw-transfer scenarios, one device's share: 32 layers x "
                       "32 blocks of [128, 8, 2, 128]; odd blocks D2H, then H2D into the "
                       "even blocks",
           "iterations": iters}
    for sc in ("A", "B"):
        res = {}
        for name, dt in dtypes.items():
            if sc == "A":
                tensors = [torch.empty((32, 128, 8, 2, 128), dtype=dt, device=dev)
                           for _ in range(32)]
            else:
                tensors = [torch.empty((32, 32, 128, 8, 2, 128), dtype=dt, device=dev)]
            for t in tensors:
                rows_u8(t).random_(0, 256)
            torch.cuda.synchronize()
            mgr = pkg.KVCacheManager(tensors, host_blocks_to_allocate=32)
            bb = rows_u8(tensors[0]).shape[1]
            moved = 16 * bb * len(tensors)
            for _ in range(warm):
                mgr.d2h(odd, odd, ones).Await()
                mgr.h2d(odd, even, ones).Await()
            t0 = time.perf_counter()
            for _ in range(iters):
                mgr.d2h(odd, odd, ones).Await()
            t_d2h = (time.perf_counter() - t0) / iters
            ev, od = torch.tensor(even, device=dev), torch.tensor(odd, device=dev)
            for t in tensors:  # the timed H2D copies must rewrite the even blocks
                rows_u8(t)[ev] = 0
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(iters):
                mgr.h2d(odd, even, ones).Await()
            t_h2d = (time.perf_counter() - t0) / iters
            torch.cuda.synchronize()
            for w, t in enumerate(tensors):
                r = rows_u8(t)
                check(torch.equal(r[ev], r[od]), f"scenario {sc} {name}: even == odd, layer {w}")
                h = torch.from_numpy(host_rows(mgr, w, bb, 0, 32)[odd]).to(dev)
                check(torch.equal(h, r[od]), f"scenario {sc} {name}: host odd blocks, layer {w}")
            st = mgr.engine_stats()
            path = "+".join(k for k in ("direct", "staged", "zero_copy")
                            if st.get(f"{k}_copies", 0)) or "none"
            pub_h2d, pub_d2h = REFERENCE_SCENARIO_GBPS[sc][name]
            r = {"bytes_per_copy": moved, "d2h_gbps": round(moved / t_d2h / 1e9, 2),
                 "h2d_gbps": round(moved / t_h2d / 1e9, 2), "path": path,
                 "reference_per_chip_d2h_gbps": round(pub_d2h / 8, 2),
                 "reference_per_chip_h2d_gbps": round(pub_h2d / 8, 2)}
            if peaks:
                r["d2h_frac_of_pcie_d2h"] = round(moved / t_d2h / 1e9 / peaks["pcie_d2h_gbps"], 4)
                r["h2d_frac_of_pcie_h2d"] = round(moved / t_h2d / 1e9 / peaks["pcie_h2d_gbps"], 4)
            res[name] = r
            log(f"scenario {sc} {name}: {r}")
            mgr.close()
            del tensors
        out[f"scenario_{sc}"] = res
    out["verified"] = True
    torch.cuda.empty_cache()
    return out


def run_configs(torch, pkg, dev, args, rng, peaks):
    configs = {}
    wanted = [c for c in args.configs.split(",") if c]
    if "scenarios" in wanted:
        configs["reference_scenarios"] = bench_reference_scenarios(torch, pkg, dev, args, peaks)
    if "fp8" in wanted:
        configs["fp8_kv_scales"] = bench_fp8_scales(torch, pkg, dev, args, rng)
    if "weights" in wanted:
        configs["weight_sync_pack"] = bench_weight_sync(torch, pkg, dev, args)
    if "tiled" in wanted:
        configs["weight_sync_tiled"] = bench_weight_sync_tiled(torch, pkg, dev, args)
    if "pools" in wanted:
        configs["sparse_pool_copies"] = bench_pools(torch, pkg, dev, args, rng)
    if "lanes" in wanted:
        configs["shm_lanes_load_and_save"] = bench_lanes(torch, pkg, dev, args, rng)
    if "zipf" in wanted:
        configs["llama3_70b_zipf_churn"] = bench_zipf_store(torch, pkg, dev, args, rng,
                                                            peaks=peaks)
    return configs


def main():
    args = parse_args()
    args.sub_steps = max(1, min(args.steps, 20))
    args.box_copy_gbps = None  # set once the box copy has been measured
    if args.rocpd_summary:
        rocpd_summary(args.rocpd_summary)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "bench.py measures one GPU; this build has no "
                                   "multi-GPU path (--gpus must be 1)"}))
        sys.exit(2)
    import torch
    sys.path.insert(0, ROOT)
    import __graft_entry__
    pkg = __graft_entry__.load_package()
    if args.configs_only:
        # Only the extra workloads (for traces of one of them): no headline,
        # no CPU baseline; not the benchmark's result line.
        dev = torch.device("cuda:0")
        # The churn's PCIe bound needs the link's measured peaks.
        peaks = by_method = None
        if "zipf" in args.configs.split(","):
            peaks, by_method = link_peaks_both_ways(torch, dev, pkg, pcie_peaks(torch, dev))
            log(f"pinned PCIe peaks: {by_method}")
        configs = run_configs(torch, pkg, dev, args, np.random.default_rng(1), peaks)
        print(json.dumps({"configs_only": True, "pcie_peaks_by_method": by_method,
                          "configs": configs}), flush=True)
        return

    w = WORKLOADS[args.workload]
    L, n, P = w["layers"], w["batch"], w["pool_blocks"]
    S = 2 * L
    bb = w["block_tokens"] * w["kv_heads"] * w["head_dim"] * w["dtype_bytes"]
    dev = torch.device("cuda:0")
    # The link's pinned peaks, measured before the headline and again after
    # it; each peak is the better of the two (peaks are bounds). Measuring
    # first keeps the headline clear of a box's transient: right after
    # another process has freed tens of GiB of device and host memory, a
    # fresh process's first ~0.5 s of offload + reload measured 72.8 against
    # 96.6 GB/s for every later 20-step window (and 96.5 from the start in
    # the process after). Measuring again later is needed for the
    # bidirectional peak: first in a process, the runtime ran the two
    # directions' copies one after the other (56.8 GB/s, one direction's
    # rate), and 96.7 once the managers' streams existed.
    measured_peaks = None
    if not args.no_extras:
        log("measuring pinned PCIe peaks (before the headline)")
        measured_peaks = pcie_peaks(torch, dev)
        log(f"pinned PCIe peaks: {measured_peaks}")
    gen = torch.Generator(device=dev).manual_seed(0)
    log(f"allocating {S} x {P} x {bb} B pool ({S * P * bb / 2**30:.1f} GiB, {args.pool_alloc})")
    pools = make_pool(torch, dev, gen, S, P, bb, args.pool_alloc)
    torch.cuda.synchronize()

    def make_mgr(mode, storages=pools, host_blocks=4 * n):
        return pkg.KVCacheManager(storages, host_blocks_to_allocate=host_blocks,
                                  staging_chunk_bytes=args.chunk_mib << 20,
                                  staging_chunks=args.chunks, profile_kernels=True,
                                  transfer_mode=mode)

    mgr = make_mgr(args.mode)
    nodes = [d for d in os.listdir("/sys/devices/system/node") if d.startswith("node")] \
        if os.path.isdir("/sys/devices/system/node") else []
    host_info = {"gpu_numa_node": int(pkg._capi.load().kvx_gpu_numa_node(0)),
                 "mirror_numa_node": mgr.assigned_numa_node,
                 "numa_nodes": len(nodes), "cpus": os.cpu_count()}
    log(f"manager ready (mode {args.mode})")
    rng = np.random.default_rng(0)
    slots = [list(range(k * n, (k + 1) * n)) for k in range(4)]
    batch = batch_source(rng, P, n)

    # The reference's gate: one offload + reload with the same manager,
    # checked before anything is timed.
    ids0, free0 = batch()
    verify_round_trip(torch, mgr, pools, ids0, slots[0], free0)
    step_bytes = 2 * n * S * bb
    log(f"timing {args.steps} offload+reload steps")
    elapsed, last = run_duplex(torch, mgr, batch, slots, args.steps, args.warmup)
    value = args.steps * step_bytes / elapsed / 1e9
    stats = mgr.engine_stats()
    log(f"offload+reload: {value:.2f} GB/s, {elapsed / args.steps * 1e3:.2f} ms/step "
        f"({stats})")
    verify_duplex(torch, mgr, pools, slots, last)
    log("last step's offload and reload verified")
    # What the headline copies actually did (the auto mode decides per copy).
    kinds = {"staged": stats["staged_copies"], "zero_copy": stats["zero_copy_copies"],
             "direct": stats["direct_copies"]}
    headline_path = {"mode": args.mode, **{f"{k}_copies": v for k, v in kinds.items()},
                     "path": "+".join(k for k, v in kinds.items() if v) or "none",
                     # Gather, D2H, H2D and scatter streams: pairs probed on
                     # one hardware queue at creation (0: all apart).
                     "stream_placement": mgr.stream_placement}
    kg = mgr.kernel_times(True, reset=True)
    ks = mgr.kernel_times(False, reset=True)

    def loop_kernel(kt, name):
        if kt["launches"] == 0:
            return None
        avg_s = kt["total_ms"] / kt["launches"] / 1e3
        per_launch = kt["bytes"] / kt["launches"]
        return {"kernel": f"block copy kernels ({name}) inside the offload/reload loop",
                "achieved_gbps": round(per_launch / avg_s / 1e9, 1),
                "launches": kt["launches"], "avg_launch_us": round(avg_s * 1e6, 2),
                "bytes_per_launch": int(per_launch)}

    loop_gather = loop_kernel(kg, "gather")
    loop_scatter = loop_kernel(ks, "scatter")

    # The gather/scatter kernels alone: one launch moves the whole batch
    # (n blocks x S storages, 2 * n * S * B algorithmic HBM bytes) between the
    # pool and a device staging buffer, on a stream of its own. Inside the
    # offload loop the same kernel shares the GPU with PCIe traffic (D2H blit
    # kernels in staged mode; the zero-copy kernels are PCIe-bound), so those
    # launches are reported separately.
    log("timing the gather/scatter kernels alone")
    staging = torch.empty(n * S * bb, dtype=torch.uint8, device=dev)
    copy_dst = torch.empty_like(staging)
    ks_stream = torch.cuda.Stream(dev)
    # The box's streaming-copy yardstick, same bytes per launch.
    staging.random_(0, 256)
    torch.cuda.synchronize()
    args.box_copy_gbps = box_copy(torch, pkg, staging, copy_dst, max(5, args.sub_steps),
                                  ks_stream)
    log(f"box copy (strided kernel, one contiguous {staging.numel() >> 20} MiB entry): "
        f"{args.box_copy_gbps:.0f} GB/s")
    # A fresh batch of random ids for each launch (16 in rotation): repeating
    # one batch keeps its pages' translations warm (gather +0.7 points).
    id_sets = [batch()[0] for _ in range(16)]
    gen_c = np.random.default_rng(5)
    contig_sets = [list(range(s0, s0 + n)) for s0 in gen_c.integers(0, P - n, 16)]
    # The same runs of ids in a shuffled order: the same blocks and pages as
    # the ascending launches, written in random order.
    shuffled_sets = [gen_c.permutation(ids).tolist() for ids in contig_sets]

    def time_kernel(m, gather, idsets, launches):
        fn = m.gather if gather else m.scatter
        for _ in range(2):
            fn(idsets[0], staging, stream=ks_stream).Await()
        # The engine brackets each launch with HIP events on ks_stream (the
        # stream the kernel runs on); the id-table upload before it is not
        # inside the bracket.
        m.kernel_times(gather, reset=True)
        futs = [fn(idsets[k % len(idsets)], staging, stream=ks_stream) for k in range(launches)]
        for f in futs:
            f.Await()
        kt = m.kernel_times(gather, reset=True)
        check(kt["bytes"] / kt["launches"] == 2 * n * S * bb, "bytes per launch")
        return kt["total_ms"] / kt["launches"] / 1e3, idsets[(launches - 1) % len(idsets)]

    def verify_kernel(storages, gather, ids):
        torch.cuda.synchronize()
        ids_t = torch.tensor(ids, device=dev)
        stg = staging.view(S, n, bb)
        for w_, t in enumerate(storages):
            check(torch.equal(t[ids_t], stg[w_]), f"{'gather' if gather else 'scatter'}, "
                                                   f"storage {w_}")

    iso = {}
    for name, idsets in (("gather", id_sets), ("scatter", id_sets),
                         ("scatter_contiguous", contig_sets),
                         ("scatter_shuffled", shuffled_sets)):
        gather = name == "gather"
        avg_s, last_ids = time_kernel(mgr, gather, idsets, args.steps)
        verify_kernel(pools, gather, last_ids)
        per_launch = 2 * n * S * bb
        ach = per_launch / avg_s / 1e9
        what = {"scatter_contiguous": "a fresh contiguous run of ids per launch, ascending",
                "scatter_shuffled": "the same contiguous runs of ids, each in a shuffled "
                                    "order"}.get(name, "a fresh random id batch per launch")
        iso[name] = {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBPS, 4),
                     "frac_of_box_copy": frac_of_box(ach, args.box_copy_gbps),
                     "traffic": MEASURED_TRAFFIC.get((name, per_launch)),
                     "kernel": (("block_copy_sliced_gather_kernel (a quarter of each of 4 ids "
                                 "per workgroup)" if gather else "block_copy_fast_kernel (scatter)")
                                + f", {n} ids x {S} storages per launch, {what}"),
                     "launches": args.steps, "avg_launch_us": round(avg_s * 1e6, 2),
                     "bytes_per_launch": int(per_launch), "verified": True}
        log(f"{name} alone: {ach:.0f} GB/s ({ach / HBM_PEAK_GBPS:.1%} of HBM peak, "
            f"{ach / args.box_copy_gbps:.1%} of the box copy)")
    # A plain runtime device copy of the same byte count (the runtime's blit
    # kernel), and the calibration kernel for the FETCH_SIZE / WRITE_SIZE
    # counters.
    t_copy = timed_each(torch, lambda: copy_dst.copy_(staging), max(3, args.sub_steps // 4),
                          ks_stream)
    hbm_copy_gbps = 2 * staging.numel() / t_copy / 1e9
    log(f"runtime device copy of {staging.numel() >> 20} MiB: {hbm_copy_gbps:.0f} GB/s")

    # Placement: the same kernels over a pool allocated the other way (one
    # buffer sliced per storage, or one allocation per storage), alternating
    # with the headline pool in this process.
    placement = None
    if args.placement_rounds > 0:
        other = "per_storage" if args.pool_alloc == "single" else "single"
        log(f"placement: allocating the pool as {other}")
        pools2 = make_pool(torch, dev, gen, S, P, bb, other)
        mgr2 = make_mgr(args.mode, storages=pools2, host_blocks=8)
        pm = {args.pool_alloc: (mgr, pools), other: (mgr2, pools2)}
        res = {k: {"gather": [], "scatter": [], "scatter_contiguous": []} for k in pm}
        for r in range(args.placement_rounds):
            for k in (list(pm) if r % 2 == 0 else list(pm)[::-1]):
                m, st = pm[k]
                for name, idsets in (("gather", id_sets), ("scatter", id_sets),
                                     ("scatter_contiguous", contig_sets)):
                    avg_s, last_ids = time_kernel(m, name == "gather", idsets, args.sub_steps)
                    res[k][name].append(avg_s)
                    if r == 0:
                        verify_kernel(st, name == "gather", last_ids)
        placement = {"rounds": args.placement_rounds, "launches_per_round": args.sub_steps,
                     "note": "median launch time per kernel, rounds alternating between the "
                             "two pools in one process"}
        for k, kinds_ in res.items():
            placement[k] = {}
            for name, xs in kinds_.items():
                med = float(np.median(xs))
                g_ = 2 * n * S * bb / med / 1e9
                placement[k][name] = {"avg_launch_us": round(med * 1e6, 2),
                                      "frac": round(g_ / HBM_PEAK_GBPS, 4),
                                      "frac_of_box_copy": frac_of_box(g_, args.box_copy_gbps)}
        log(f"placement: {placement}")
        mgr2.close()
        del pools2, mgr2, pm
    del staging, copy_dst
    mgr.kernel_times(True, reset=True)
    mgr.kernel_times(False, reset=True)

    extras = {}
    if not args.no_extras:
        half = n * S * bb
        reps = max(3, args.sub_steps // 2)
        modes = {}
        for mode in [args.mode] + [x for x in ("zero_copy", "staged") if x != args.mode]:
            m = mgr if mode == args.mode else make_mgr(mode)
            t_off, t_rel = one_direction(m, batch, slots, reps)
            el_steps = args.steps if m is mgr else args.sub_steps
            if m is mgr:
                el = elapsed
            else:
                el, last_m = run_duplex(torch, m, batch, slots, el_steps, args.warmup)
                verify_duplex(torch, m, pools, slots, last_m)
            modes[mode] = {"duplex_gbps": round(el_steps * step_bytes / el / 1e9, 2),
                           "offload_gbps": round(half / t_off / 1e9, 2),
                           "reload_gbps": round(half / t_rel / 1e9, 2)}
            log(f"{mode}: {modes[mode]}")
            if m is not mgr:
                m.close()
        log("measuring pinned PCIe peaks (after the headline)")
        later = pcie_peaks(torch, dev)
        log(f"pinned PCIe peaks: {later}")
        runtime_peaks = {k: max(v, later[k]) for k, v in measured_peaks.items()}
        measured_peaks, peaks_by_method = link_peaks_both_ways(torch, dev, pkg, runtime_peaks)
        log(f"pinned PCIe peaks by method: {peaks_by_method}")
        peaks = measured_peaks
        for mode, r in modes.items():
            r["offload_frac_of_pcie_d2h"] = round(r["offload_gbps"] / peaks["pcie_d2h_gbps"], 4)
            r["reload_frac_of_pcie_h2d"] = round(r["reload_gbps"] / peaks["pcie_h2d_gbps"], 4)
            r["duplex_frac_of_pcie_bidir"] = round(r["duplex_gbps"] / peaks["pcie_bidir_gbps"], 4)
        # Per direction: the headline manager itself (its mode), one copy at a
        # time; the path it took is in headline_path.
        extras = {
            "offload_gbps": modes[args.mode]["offload_gbps"],
            "reload_gbps": modes[args.mode]["reload_gbps"],
            "offload_frac_of_pcie_d2h": modes[args.mode]["offload_frac_of_pcie_d2h"],
            "reload_frac_of_pcie_h2d": modes[args.mode]["reload_frac_of_pcie_h2d"],
            "duplex_frac_of_pcie_bidir": round(value / peaks["pcie_bidir_gbps"], 4),
            **{k: round(v, 2) for k, v in peaks.items()},
            "pcie_peaks_by_method": peaks_by_method,
            "modes": modes,
        }
        # Short host runs (every host id a run of its own, as a store's
        # fragmented tier gives) with offload and reload at once.
        extras["short_runs"] = short_run_duplex(torch, pkg, pools, make_mgr, rng, P, n, args,
                                                peaks)
    mgr.close()
    del pools
    torch.cuda.empty_cache()

    # The other workloads of the path, each measured on its own shape.
    configs = run_configs(torch, pkg, dev, args, rng, measured_peaks)

    cpu = None
    if args.cpu_seconds > 0:
        log("CPU baseline (oracle host pack/unpack)")
        cpu = cpu_baseline(__graft_entry__.load_oracle(), S, bb, n, P, args.cpu_seconds)

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
            "transfer_mode": args.mode, "staging_chunk_mib": args.chunk_mib,
            "pool_allocation": POOL_ALLOC_TEXT[args.pool_alloc],
        },
        "blocks_per_s": round(args.steps * 2 * n / elapsed, 1),
        "verified": True,
        "headline_path": headline_path,
        "roofline": iso["gather"],
        "scatter_roofline": iso["scatter"],
        "scatter_contiguous": iso["scatter_contiguous"],
        "scatter_shuffled": iso["scatter_shuffled"],
        "box_copy": {"kernel": "strided_copy_kernel over one contiguous entry of the same "
                               "bytes (sliced tile groups, 2 workgroups per CU), HIP events "
                               "on its stream",
                     "achieved": round(args.box_copy_gbps, 1),
                     "frac": round(args.box_copy_gbps / HBM_PEAK_GBPS, 4), "verified": True},
        "placement": placement,
        "loop_gather": loop_gather,
        "loop_scatter": loop_scatter,
        "hbm_copy_same_bytes_gbps": round(hbm_copy_gbps, 1),
        "cpu_baseline": cpu,
        "host": host_info,
        **extras,
        "configs": configs,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
