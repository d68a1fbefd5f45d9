#include "numa.h"

#include <hip/hip_runtime_api.h>
#include <linux/mempolicy.h>
#include <sched.h>
#include <sys/syscall.h>
#include <unistd.h>

#include <cctype>
#include <cerrno>
#include <cstdint>
#include <cstring>
#include <fstream>
#include <sstream>

namespace kvx {
namespace {

constexpr unsigned long kMaskBits = 16 * 8 * sizeof(unsigned long);

long GetMempolicy(int* mode, unsigned long* mask, unsigned long maxnode, const void* addr,
                  unsigned long flags) {
  return syscall(SYS_get_mempolicy, mode, mask, maxnode, addr, flags);
}

long SetMempolicy(int mode, const unsigned long* mask, unsigned long maxnode) {
  return syscall(SYS_set_mempolicy, mode, mask, maxnode);
}

std::string ReadFirstLine(const std::string& path) {
  std::ifstream f(path);
  std::string line;
  if (!f || !std::getline(f, line)) return "";
  return line;
}

}  // namespace

int NumaNodeOfPciDevice(const std::string& sysfs_root, const std::string& bus_id) {
  std::string id = bus_id;
  for (char& c : id) c = static_cast<char>(std::tolower(static_cast<unsigned char>(c)));
  const std::string line = ReadFirstLine(sysfs_root + "/bus/pci/devices/" + id + "/numa_node");
  if (line.empty()) return -1;
  char* end = nullptr;
  const long v = std::strtol(line.c_str(), &end, 10);
  if (end == line.c_str() || v < 0 || v >= static_cast<long>(kMaskBits)) return -1;
  return static_cast<int>(v);
}

int GpuNumaNode(int device) {
  char bus[64] = {};
  if (hipDeviceGetPCIBusId(bus, sizeof(bus), device) != hipSuccess) {
    (void)hipGetLastError();
    return -1;
  }
  return NumaNodeOfPciDevice("/sys", bus);
}

int PageNumaNode(const void* addr) {
  int node = -1;
  if (GetMempolicy(&node, nullptr, 0, addr, MPOL_F_NODE | MPOL_F_ADDR) != 0) return -1;
  return node;
}

ScopedNumaPreference::ScopedNumaPreference(int node) {
  if (node < 0 || node >= static_cast<int>(kMaskBits)) return;
  if (GetMempolicy(&saved_mode_, saved_mask_, kMaskBits, nullptr, 0) != 0) return;
  unsigned long mask[16] = {};
  mask[node / (8 * sizeof(unsigned long))] = 1ul << (node % (8 * sizeof(unsigned long)));
  active_ = SetMempolicy(MPOL_PREFERRED, mask, kMaskBits) == 0;
}

ScopedNumaPreference::~ScopedNumaPreference() {
  if (!active_) return;
  // A default policy carries no node mask.
  (void)SetMempolicy(saved_mode_, saved_mode_ == MPOL_DEFAULT ? nullptr : saved_mask_,
                     saved_mode_ == MPOL_DEFAULT ? 0 : kMaskBits);
}

Status PreferNodeForRange(void* addr, size_t len, int node) {
  if (node < 0 || addr == nullptr || len == 0) return OkStatus();
  if (node >= static_cast<int>(kMaskBits)) return InvalidArgumentError("NUMA node out of range");
  const long page = sysconf(_SC_PAGESIZE);
  const uintptr_t start = reinterpret_cast<uintptr_t>(addr) & ~static_cast<uintptr_t>(page - 1);
  const uintptr_t end = reinterpret_cast<uintptr_t>(addr) + len;
  unsigned long mask[16] = {};
  mask[node / (8 * sizeof(unsigned long))] = 1ul << (node % (8 * sizeof(unsigned long)));
  if (syscall(SYS_mbind, reinterpret_cast<void*>(start), end - start, MPOL_PREFERRED, mask,
              kMaskBits, 0) != 0) {
    return InternalError(std::string("mbind failed: ") + std::strerror(errno));
  }
  return OkStatus();
}

StatusOr<std::string> NumaNodeCpuList(const std::string& sysfs_root, int node) {
  if (node < 0) return InvalidArgumentError("NUMA node must be non-negative");
  const std::string line =
      ReadFirstLine(sysfs_root + "/devices/system/node/node" + std::to_string(node) + "/cpulist");
  if (line.empty()) return NotFoundError("no cpulist for NUMA node " + std::to_string(node));
  return line;
}

Status PinCurrentThreadToNumaNode(int node) {
  KVX_ASSIGN_OR_RETURN(std::string list, NumaNodeCpuList("/sys", node));
  cpu_set_t set;
  CPU_ZERO(&set);
  std::stringstream ss(list);
  std::string part;
  int count = 0;
  while (std::getline(ss, part, ',')) {
    if (part.empty()) continue;
    const size_t dash = part.find('-');
    char* end = nullptr;
    const long lo = std::strtol(part.c_str(), &end, 10);
    long hi = lo;
    if (dash != std::string::npos) hi = std::strtol(part.c_str() + dash + 1, &end, 10);
    if (lo < 0 || hi < lo) return InvalidArgumentError("malformed cpulist: " + list);
    for (long c = lo; c <= hi && c < CPU_SETSIZE; ++c) {
      CPU_SET(static_cast<int>(c), &set);
      ++count;
    }
  }
  if (count == 0) return NotFoundError("NUMA node " + std::to_string(node) + " has no CPUs");
  if (sched_setaffinity(0, sizeof(set), &set) != 0) {
    return InternalError(std::string("sched_setaffinity failed: ") + std::strerror(errno));
  }
  return OkStatus();
}

}  // namespace kvx
