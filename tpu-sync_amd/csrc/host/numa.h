// NUMA placement of host buffers next to the GPU: the MI355X counterpart of
// the reference's DetectAndAssignNumaNode (tpu_sync/core/raiden_manager_base.cc:47-76),
// its allocate-under-thread-mempolicy + first touch
// (tpu_sync/core/host_memory_allocator.cc:86-121) and the node-pinned issue
// threads of NumaThreadPool (tpu_sync/core/numa_thread_pool.h:36-80).
//
// The GPU's node comes from its PCI function in sysfs. Host mirrors are
// allocated and first touched while the allocating thread prefers that node
// (MPOL_PREFERRED rather than the reference's MPOL_BIND, so a host tier
// larger than one node's free memory spills instead of failing); shared
// memory segments get the same preference on their mapping (mbind), which
// governs pages faulted in later by any thread.
#ifndef KVX_HOST_NUMA_H_
#define KVX_HOST_NUMA_H_

#include <cstddef>
#include <string>

#include "status.h"

namespace kvx {

// <sysfs_root>/bus/pci/devices/<bus_id>/numa_node, or -1 when absent or
// negative. bus_id is matched in lower case ("0000:c1:00.0").
int NumaNodeOfPciDevice(const std::string& sysfs_root, const std::string& bus_id);

// NUMA node of HIP device `device`, or -1 (no GPU, no NUMA information).
int GpuNumaNode(int device);

// Number of the NUMA node holding the page at `addr` (after it has been
// touched), or -1.
int PageNumaNode(const void* addr);

// While alive, the calling thread's new pages prefer `node` (no-op for
// node < 0); the previous policy is restored on destruction.
class ScopedNumaPreference {
 public:
  explicit ScopedNumaPreference(int node);
  ~ScopedNumaPreference();
  ScopedNumaPreference(const ScopedNumaPreference&) = delete;
  ScopedNumaPreference& operator=(const ScopedNumaPreference&) = delete;
  bool active() const { return active_; }

 private:
  bool active_ = false;
  int saved_mode_ = 0;
  unsigned long saved_mask_[16] = {};
};

// Applies a preference for `node` to the page-aligned range [addr, addr+len)
// (pages faulted in afterwards land there). No-op for node < 0.
Status PreferNodeForRange(void* addr, size_t len, int node);

// CPUs of <sysfs_root>/devices/system/node/node<N>/cpulist ("0-7,16-23").
StatusOr<std::string> NumaNodeCpuList(const std::string& sysfs_root, int node);
// Restricts the calling thread to the CPUs of `node`.
Status PinCurrentThreadToNumaNode(int node);

}  // namespace kvx

#endif  // KVX_HOST_NUMA_H_
