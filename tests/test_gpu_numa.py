"""GPU: the manager and the weight synchronizer place their host memory on
the GPU's NUMA node (DetectAndAssignNumaNode,
tpu_sync/core/raiden_manager_base.cc:47-76): the node comes from the GPU's PCI
function in sysfs, read here independently from torch's device properties,
and every touched page of the mirrors reports that node."""
import os

import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


def sysfs_node():
    p = torch.cuda.get_device_properties(0)
    if not hasattr(p, "pci_bus_id") or not hasattr(p, "pci_device_id"):
        return None
    bdf = "%04x:%02x:%02x.0" % (getattr(p, "pci_domain_id", 0), p.pci_bus_id, p.pci_device_id)
    path = f"/sys/bus/pci/devices/{bdf}/numa_node"
    if not os.path.exists(path):
        return None
    v = int(open(path).read().strip())
    return v if v >= 0 else -1


def test_host_mirrors_on_gpu_node(kvx, cuda):
    want = sysfs_node()
    lib = kvx._capi.load()
    got = lib.kvx_gpu_numa_node(0)
    print("gpu numa node", got, "sysfs", want, flush=True)
    if want is not None:
        assert got == want
    kv = [torch.zeros(64, 65536, dtype=torch.uint8, device=cuda) for _ in range(2)]
    for alloc in ("pinned", "malloc"):
        mgr = kvx.KVCacheManager(kv, host_blocks_to_allocate=64, host_alloc=alloc)
        assert mgr.assigned_numa_node == got
        if got >= 0:
            for layer in range(2):
                base = lib.kvx_manager_block_array_host_ptr(mgr._h, layer, 0)
                for off in range(0, 64 * 65536, 1 << 20):
                    assert lib.kvx_host_page_numa_node(base + off) == got, (alloc, layer, off)
        mgr.close()
        off_mgr = kvx.KVCacheManager(kv, host_blocks_to_allocate=4, host_alloc=alloc, numa="off")
        assert off_mgr.assigned_numa_node == -1
        off_mgr.close()
    ws = kvx.WeightSynchronizer([[t] for t in kv])
    if got >= 0:
        assert lib.kvx_host_page_numa_node(lib.kvx_weight_sync_host_base(ws._h)) == got
    ws.close()
