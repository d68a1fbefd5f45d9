// Classification of the raw addresses handed across the C-ABI.
//
// The C-ABI takes device buffers as plain addresses. One that is host
// memory (pageable or pinned), memory of another device, or no allocation
// at all would reach a kernel or a DMA and fault or corrupt memory there.
// The reference validates every argument before it issues any copy
// (tpu_sync/kv_cache/kv_cache_manager_base.cc:72-102); here the addresses
// are part of that validation: each is looked up in the HIP runtime, which
// knows every device allocation (hipPointerGetAttributes: memory type and
// device; hipMemGetAddressRange: the allocation's extent), and a bad one is
// refused with INVALID_ARGUMENT before anything is issued.
//
// The lookup is a replaceable function so that tests on a machine without a
// GPU can drive the C-ABI's checks with addresses of their own making.
#ifndef KVX_HOST_DEVICE_MEMORY_H_
#define KVX_HOST_DEVICE_MEMORY_H_

#include <cstdint>
#include <utility>
#include <vector>

#include "status.h"

namespace kvx {

enum class MemKind : int {
  kUnknown = 0,  // no allocation the runtime knows (e.g. pageable host memory)
  kHost = 1,     // host memory registered with or allocated by the runtime
  kDevice = 2,   // device memory
  kOther = 3,    // managed, array or other memory the kernels do not take
};

struct AddressInfo {
  MemKind kind = MemKind::kUnknown;
  int device = -1;
  uint64_t base = 0;  // the allocation's extent; size 0: not known
  uint64_t size = 0;
};

using AddressQuery = AddressInfo (*)(uint64_t addr);

// Installs `q` as the lookup behind every check (nullptr restores the HIP
// runtime's). For tests: the C-ABI then classifies addresses without a GPU.
void SetAddressQueryForTesting(AddressQuery q);

// Checks ranges [addr, addr + bytes) of one call. Each must lie in one
// device allocation of `device` (-1: of the device of the first range
// checked, for calls that name no device); a range inside an allocation
// already found in this call is not looked up again. Empty ranges are not
// accessed and pass. `what` names the argument in the error.
class DeviceRangeChecker {
 public:
  explicit DeviceRangeChecker(int device) : device_(device) {}
  Status Check(uint64_t addr, uint64_t bytes, const char* what);
  int device() const { return device_; }

 private:
  int device_;
  std::vector<std::pair<uint64_t, uint64_t>> known_;  // [base, end)
};

inline Status CheckDeviceRange(int device, uint64_t addr, uint64_t bytes, const char* what) {
  return DeviceRangeChecker(device).Check(addr, bytes, what);
}

// Bytes from the first to the last byte a strided run touches: count rows
// of `size` bytes, `stride` apart (count >= 1, size > 0, stride >= 0);
// false on overflow.
bool StridedExtent(int64_t size, int64_t count, int64_t stride, uint64_t* bytes);

}  // namespace kvx

#endif  // KVX_HOST_DEVICE_MEMORY_H_
