// Host-side checks of the NUMA topology lookups in libkvx (numa.h) against a
// made-up sysfs tree of a two-node machine with two GPUs, on the CPU (no
// device calls): the GPU's node from its PCI function (upper- or lower-case
// bus ids, missing, negative or malformed files) and a node's CPU list.
//   argv[1]: an empty directory to build the tree in.
#include <cstdio>
#include <fstream>
#include <string>
#include <sys/stat.h>

#include "numa.h"

namespace {

int failures = 0;

void expect(bool ok, const std::string& what) {
  if (!ok) {
    std::printf("FAIL: %s\n", what.c_str());
    ++failures;
  }
}

void mkdirs(const std::string& path) {
  std::string cur;
  for (size_t i = 0; i <= path.size(); ++i) {
    if (i == path.size() || path[i] == '/') {
      if (!cur.empty()) mkdir(cur.c_str(), 0755);
    }
    if (i < path.size()) cur += path[i];
  }
}

void write(const std::string& dir, const std::string& name, const std::string& text) {
  mkdirs(dir);
  std::ofstream(dir + "/" + name) << text;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 2) {
    std::printf("usage: numa_topology_check <empty dir>\n");
    return 2;
  }
  const std::string root = argv[1];
  const std::string pci = root + "/bus/pci/devices/";
  // GPU 0 on node 0, GPU 1 on node 1, a device whose firmware reports no
  // node (-1), one with a malformed file, one with a node beyond the mask.
  write(pci + "0000:05:00.0", "numa_node", "0\n");
  write(pci + "0000:c1:00.0", "numa_node", "1\n");
  write(pci + "0000:11:00.0", "numa_node", "-1\n");
  write(pci + "0000:12:00.0", "numa_node", "node\n");
  write(pci + "0000:13:00.0", "numa_node", "100000\n");
  write(root + "/devices/system/node/node0", "cpulist", "0-63,128-191\n");
  write(root + "/devices/system/node/node1", "cpulist", "64-127,192-255\n");

  expect(kvx::NumaNodeOfPciDevice(root, "0000:05:00.0") == 0, "GPU on node 0");
  expect(kvx::NumaNodeOfPciDevice(root, "0000:c1:00.0") == 1, "GPU on node 1");
  // hipDeviceGetPCIBusId may report the bus id in upper case.
  expect(kvx::NumaNodeOfPciDevice(root, "0000:C1:00.0") == 1, "upper-case bus id");
  expect(kvx::NumaNodeOfPciDevice(root, "0000:11:00.0") == -1, "no node reported");
  expect(kvx::NumaNodeOfPciDevice(root, "0000:12:00.0") == -1, "malformed numa_node");
  expect(kvx::NumaNodeOfPciDevice(root, "0000:13:00.0") == -1, "node beyond the mask");
  expect(kvx::NumaNodeOfPciDevice(root, "0000:99:00.0") == -1, "unknown device");
  expect(kvx::NumaNodeOfPciDevice(root + "/missing", "0000:05:00.0") == -1, "no sysfs tree");

  auto l0 = kvx::NumaNodeCpuList(root, 0);
  expect(l0.ok() && l0.value() == "0-63,128-191", "node 0 cpulist");
  auto l1 = kvx::NumaNodeCpuList(root, 1);
  expect(l1.ok() && l1.value() == "64-127,192-255", "node 1 cpulist");
  auto l2 = kvx::NumaNodeCpuList(root, 2);
  expect(!l2.ok() && l2.status().code() == kvx::Code::kNotFound, "node 2 has no cpulist");
  auto lneg = kvx::NumaNodeCpuList(root, -1);
  expect(!lneg.ok() && lneg.status().code() == kvx::Code::kInvalidArgument, "negative node");

  // A preference for a node that does not exist on this machine, and for a
  // negative node, leave the thread's policy alone.
  {
    kvx::ScopedNumaPreference none(-1);
    expect(!none.active(), "no preference for node -1");
  }
  expect(kvx::PreferNodeForRange(nullptr, 4096, 1).ok(), "empty range is a no-op");
  expect(!kvx::PreferNodeForRange(reinterpret_cast<void*>(4096), 4096, 5000).ok(),
         "node beyond the mask refused");

  if (failures == 0) std::printf("all checks passed\n");
  return failures == 0 ? 0 : 1;
}
