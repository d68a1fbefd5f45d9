// Small HIP helpers shared by the host-side library.
#ifndef KVX_HOST_HIP_UTIL_H_
#define KVX_HOST_HIP_UTIL_H_

#include <hip/hip_runtime_api.h>

#include <string>

#include "status.h"

namespace kvx {

inline Status HipStatus(hipError_t e, const char* what) {
  if (e == hipSuccess) return OkStatus();
  return InternalError(std::string(what) + ": " + hipGetErrorName(e) + " (" +
                       hipGetErrorString(e) + ")");
}

#define KVX_HIP_RETURN_IF_ERROR(expr) \
  KVX_RETURN_IF_ERROR(::kvx::HipStatus((expr), #expr))

// Makes `device` current for the scope and restores the caller's device, so
// calls into the library never change the device a framework thread uses.
class DeviceGuard {
 public:
  explicit DeviceGuard(int device) {
    if (hipGetDevice(&prev_) != hipSuccess) prev_ = -1;
    if (prev_ != device) {
      ok_ = hipSetDevice(device) == hipSuccess;
      restore_ = ok_ && prev_ >= 0;
    }
  }
  ~DeviceGuard() {
    if (restore_) (void)hipSetDevice(prev_);
  }
  bool ok() const { return ok_; }
  DeviceGuard(const DeviceGuard&) = delete;
  DeviceGuard& operator=(const DeviceGuard&) = delete;

 private:
  int prev_ = -1;
  bool ok_ = true;
  bool restore_ = false;
};

}  // namespace kvx

#endif  // KVX_HOST_HIP_UTIL_H_
