"""NUMA placement helpers on the CPU: the node preference of host
allocations (checked with get_mempolicy on the touched pages of this
machine's node 0), thread pinning to a node's CPUs, and the manager's
placement options (the GPU's node is checked in test_gpu_numa.py). The reference detects
the node of its devices (tpu_sync/core/raiden_manager_base.cc:47-76) and
allocates under a thread mempolicy with first touch
(tpu_sync/core/host_memory_allocator.cc:86-121)."""
import ctypes
import os

import numpy as np
import pytest


def node0_exists():
    return os.path.isdir("/sys/devices/system/node/node0")


def test_manager_numa_options(kvx):
    # Host-only managers: AUTO has no GPU to follow; an explicit node is kept.
    m = kvx.KVCacheManager.create_host_only_for_testing(num_layers=1, slice_byte_size=4096,
                                                        host_blocks=64)
    assert m.assigned_numa_node == -1
    lib = kvx._capi.load()
    cfg = kvx._capi.ManagerConfig()
    cfg.num_layers, cfg.num_shards, cfg.slice_byte_size, cfg.host_blocks = 1, 1, 4096, 256
    cfg.host_alloc = kvx._capi.HOST_MALLOC
    cfg.numa_policy, cfg.numa_node = 2, -1
    h = ctypes.c_void_p()
    with pytest.raises(kvx.KvxError, match="numa_node must be non-negative"):
        kvx._capi.check(lib.kvx_manager_create(ctypes.byref(cfg), ctypes.byref(h)))
    cfg.numa_policy = 7
    with pytest.raises(kvx.KvxError, match="unknown numa_policy"):
        kvx._capi.check(lib.kvx_manager_create(ctypes.byref(cfg), ctypes.byref(h)))
    if not node0_exists():
        pytest.skip("no NUMA node 0 on this host")
    cfg.numa_policy, cfg.numa_node = 2, 0
    kvx._capi.check(lib.kvx_manager_create(ctypes.byref(cfg), ctypes.byref(h)))
    try:
        assert lib.kvx_manager_numa_node(h) == 0
        base = lib.kvx_manager_block_array_host_ptr(h, 0, 0)
        size = lib.kvx_manager_block_array_host_size(h, 0, 0)
        assert size == 256 * 4096
        # Every page of the zeroed mirror was touched while preferring node 0.
        for off in range(0, size, 64 * 4096):
            assert lib.kvx_host_page_numa_node(base + off) == 0
    finally:
        lib.kvx_manager_destroy(h)


def test_gpu_numa_node_without_gpu_is_minus_one(kvx):
    assert kvx._capi.load().kvx_gpu_numa_node(0) in (-1,) + tuple(range(64))
    assert kvx._capi.load().kvx_host_page_numa_node(0) == -1


def test_pin_current_thread(kvx):
    import threading
    if not node0_exists():
        pytest.skip("no NUMA node 0 on this host")
    cpus = open("/sys/devices/system/node/node0/cpulist").read().strip()
    want = set()
    for part in cpus.split(","):
        lo, _, hi = part.partition("-")
        want |= set(range(int(lo), int(hi or lo) + 1))
    got = {}

    def run():
        kvx._capi.check(kvx._capi.load().kvx_numa_pin_current_thread(0))
        got["cpus"] = os.sched_getaffinity(0)
        got["bad"] = kvx._capi.load().kvx_numa_pin_current_thread(100000)

    t = threading.Thread(target=run)
    t.start()
    t.join()
    assert got["cpus"] == want & os.sched_getaffinity(0) or got["cpus"] == want
    assert got["bad"] == 5  # NOT_FOUND: no such node


def test_topology_lookups_on_a_two_node_tree(tmp_path):
    """The GPU-node and CPU-list lookups of libkvx (tests/numa_topology_check.cc)
    against a made-up sysfs tree of a two-node machine: this machine may have
    one node, so the two-node cases are checked on the lookups themselves."""
    import shutil
    import subprocess
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    cxx = shutil.which("g++") or shutil.which("c++")
    libdir = os.path.join(root, "tpu-sync_amd")
    if cxx is None or not os.path.exists(os.path.join(libdir, "libkvx.so")):
        pytest.skip("no C++ compiler or libkvx.so not built")
    exe = tmp_path / "numa_topology_check"
    env = {k: v for k, v in os.environ.items() if k != "LD_PRELOAD"}
    r = subprocess.run([cxx, "-O1", "-std=c++17", "-Wall", "-Werror", "-D__HIP_PLATFORM_AMD__",
                        "-I/opt/rocm/include",
                        "-I", os.path.join(root, "tpu-sync_amd", "csrc", "host"),
                        os.path.join(root, "tests", "numa_topology_check.cc"), "-o", str(exe),
                        "-L", libdir, "-lkvx", f"-Wl,-rpath,{libdir}"],
                       capture_output=True, text=True, env=env)
    assert r.returncode == 0, r.stdout + r.stderr
    tree = tmp_path / "sys"
    tree.mkdir()
    r = subprocess.run([str(exe), str(tree)], capture_output=True, text=True, timeout=60, env=env)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all checks passed" in r.stdout

