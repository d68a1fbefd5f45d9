// Definitions shared by the extern "C" translation units: the opaque handle
// types and the status-to-code helpers (the message of the last failing call
// is kept per thread).
#ifndef KVX_CAPI_CAPI_INTERNAL_H_
#define KVX_CAPI_CAPI_INTERNAL_H_

#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../../include/kvx.h"
#include "../host/copy_future.h"
#include "../host/kv_cache_manager.h"
#include "../host/logical_block_manager.h"
#include "../host/status.h"

struct kvx_block_manager {
  kvx::LogicalBlockManager* lbm = nullptr;
  std::unique_ptr<kvx::LogicalBlockManager> owned;
  std::mutex* mu = nullptr;  // the owning object's lock, if any
};

struct kvx_manager {
  std::unique_ptr<kvx::KVCacheManager> impl;
  kvx_block_manager lbm_view;  // borrowed view of the manager's allocator
};

struct kvx_future {
  kvx::CopyFuture f;
};

struct kvx_strings {
  std::vector<std::string> items;
  // kvx_strings_flat: the items back to back and their offsets (built on
  // first use).
  std::string flat;
  std::vector<int64_t> offsets;
};

namespace kvx {
// Looks up this device's address of the no-alloc gather's scratch array
// (kvx_no_alloc.hip) once per device; the device must be current.
Status InitNoAllocScratch(int device);
}  // namespace kvx

namespace kvx_capi {

int Fail(const kvx::Status& s);
int Fail(int code, const char* msg);
int Done(const kvx::Status& s);
inline bool BadArray(const void* p, int64_t n) {
  return n < 0 || (n > 0 && p == nullptr);
}

}  // namespace kvx_capi

#endif  // KVX_CAPI_CAPI_INTERNAL_H_
