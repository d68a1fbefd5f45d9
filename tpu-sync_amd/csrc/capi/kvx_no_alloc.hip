// kvx_manager_gather_no_alloc: the device gather of kvx_manager_gather with
// its argument tables (block ids and storage base addresses) in a fixed
// device array instead of the library's argument ring, for callers that may
// not allocate (code under stream capture, serving loops that forbid
// hipMalloc).
//
// The tables reach the device through kernel arguments: a fill kernel
// receives up to kFillWords words by value (the runtime copies kernel
// arguments at launch) and stores them into `scratch`, then the block-copy
// kernel reads them from there. Nothing on the success path allocates host
// or device memory, and nothing reads the caller's host arrays after the call
// returns. Every launch goes on the caller's stream, in order.
//
// `scratch` is one array per GPU, shared by every call on that GPU, and it
// keeps the last call's contents. Every word a call reads is written by the
// same call first, so nothing needs clearing. Calls on one GPU are ordered:
// each records a per-device event after its last launch, and a call on
// another stream first makes its stream wait for that event, so its fills
// overwrite `scratch` only after the previous call's gather has read it
// (the event is created at set-up: a call allocates nothing). A per-device
// mutex keeps one call's wait, fills, launches and record together when
// host threads call at once. Calls on one stream are ordered by the stream
// and wait for nothing else.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdio>
#include <cstdint>
#include <mutex>
#include <string>

#include "../host/device_memory.h"
#include "../host/hip_util.h"
#include "../kernels/block_copy.h"
#include "capi_internal.h"

namespace kvx {
namespace {

// Scratch layout per call, in 8-byte words: the n block ids, then (from the
// next multiple of 32 words) one base-address table per block-size group.
constexpr int64_t kNoAllocMaxIds = KVX_NO_ALLOC_MAX_IDS;
constexpr int64_t kNoAllocMaxStorages = KVX_NO_ALLOC_MAX_STORAGES;
constexpr int64_t kScratchWords = kNoAllocMaxIds + 32 + kNoAllocMaxStorages;
constexpr int kMaxGroups = 16;
constexpr int kFillWords = 256;  // 2 KiB of kernel arguments per fill launch
constexpr int kMaxDevices = 64;

static __device__ __align__(256) uint64_t scratch[kScratchWords];

struct FillArgs {
  uint64_t words[kFillWords];
};

// Lane k stores word k of the launch's arguments (a vector store).
__global__ __launch_bounds__(kFillWords) void scratch_fill_kernel(FillArgs a, uint64_t* dst,
                                                                  uint32_t count) {
  const uint32_t k = threadIdx.x;
  if (k < count) dst[k] = a.words[k];
}

// Device address of `scratch` per device ordinal (0 = not looked up yet).
std::atomic<uint64_t> g_scratch_addr[kMaxDevices];
std::mutex g_scratch_mu;

// Per device: the event recorded after each call's last launch and the
// stream it was recorded on (the event lives as long as the process, like
// `scratch`).
struct CallOrder {
  std::mutex mu;
  hipEvent_t last = nullptr;
  hipStream_t stream = nullptr;
  bool recorded = false;
};
CallOrder g_order[kMaxDevices];

// Streams words into scratch[first..) through fill launches on `stream`.
class ScratchWriter {
 public:
  ScratchWriter(uint64_t base, hipStream_t stream) : base_(base), stream_(stream) {}
  hipError_t Push(uint64_t w) {
    buf_.words[count_++] = w;
    return count_ == kFillWords ? Flush() : hipSuccess;
  }
  hipError_t SkipTo(uint64_t word) {
    while (next_ + count_ < word) {
      const hipError_t e = Push(0);
      if (e != hipSuccess) return e;
    }
    return hipSuccess;
  }
  hipError_t Flush() {
    if (count_ == 0) return hipSuccess;
    uint64_t* dst = reinterpret_cast<uint64_t*>(base_) + next_;
    hipLaunchKernelGGL(scratch_fill_kernel, dim3(1), dim3(kFillWords), 0, stream_, buf_,
                       dst, count_);
    next_ += count_;
    count_ = 0;
    return hipGetLastError();
  }

 private:
  uint64_t base_;
  hipStream_t stream_;
  FillArgs buf_{};
  uint32_t count_ = 0;
  uint64_t next_ = 0;
};

}  // namespace

// Looks up this device's copy of `scratch` once; `device` must be current.
// Called when a device-backed manager is created.
Status InitNoAllocScratch(int device) {
  if (device < 0 || device >= kMaxDevices) {
    return InvalidArgumentError("device ordinal beyond the no-alloc scratch table");
  }
  std::lock_guard<std::mutex> l(g_scratch_mu);
  if (g_scratch_addr[device].load(std::memory_order_acquire) != 0) return OkStatus();
  {
    std::lock_guard<std::mutex> o(g_order[device].mu);
    if (g_order[device].last == nullptr) {
      KVX_HIP_RETURN_IF_ERROR(
          hipEventCreateWithFlags(&g_order[device].last, hipEventDisableTiming));
    }
  }
  void* ptr = nullptr;
  KVX_HIP_RETURN_IF_ERROR(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
  if (ptr == nullptr) return InternalError("hipGetSymbolAddress(scratch) returned null");
  g_scratch_addr[device].store(reinterpret_cast<uint64_t>(ptr), std::memory_order_release);
  return OkStatus();
}

}  // namespace kvx

using kvx_capi::BadArray;
using kvx_capi::Fail;

extern "C" int kvx_manager_gather_no_alloc(kvx_manager* m, const int64_t* ids, int64_t n,
                                           uint64_t staging, int64_t staging_bytes,
                                           int32_t order, int64_t layer_idx,
                                           int64_t shard_idx, void* stream) {
  using namespace kvx;
  if (m == nullptr) return Fail(KVX_INVALID_ARGUMENT, "null manager");
  if (BadArray(ids, n)) return Fail(KVX_INVALID_ARGUMENT, "null ids with a positive length");
  if (order != KVX_LAYER_MAJOR && order != KVX_BLOCK_MAJOR) {
    return Fail(KVX_INVALID_ARGUMENT, "unknown staging order");
  }
  const KVCacheManager& mgr = *m->impl;
  if (!mgr.device_backed()) {
    return Fail(KVX_FAILED_PRECONDITION,
                "Gather/Scatter requires a device-backed KVCacheManagerBase");
  }
  const int64_t L = static_cast<int64_t>(mgr.num_layers());
  const int64_t S = static_cast<int64_t>(mgr.num_shards());
  if (layer_idx >= L || shard_idx >= S) {
    return Fail(KVX_OUT_OF_RANGE, "layer or shard index out of range");
  }
  if (n > kNoAllocMaxIds) {
    return Fail(KVX_INVALID_ARGUMENT,
                "kvx_manager_gather_no_alloc: more block ids than its scratch holds");
  }
  const int device = mgr.device();
  const uint64_t scratch_addr =
      device >= 0 && device < kMaxDevices ? g_scratch_addr[device].load(std::memory_order_acquire)
                                          : 0;
  if (scratch_addr == 0) return Fail(KVX_INTERNAL, "no-alloc scratch was not set up");

  // Block-size groups of the selected storages in first-appearance order
  // (the staging layout of kvx_manager_gather), and the id check of its
  // storages in order: the first storage's check names the first bad id.
  int64_t gbytes[kMaxGroups];
  int64_t gpool[kMaxGroups];
  int64_t gcount[kMaxGroups];
  int ngroups = 0;
  int64_t nstorages = 0;
  uint64_t acc = staging;
  bool first = true;
  for (int64_t l = 0; l < L; ++l) {
    if (layer_idx >= 0 && l != layer_idx) continue;
    const int64_t B = mgr.LayerBlockByteSize(static_cast<size_t>(l));
    for (int64_t s = 0; s < S; ++s) {
      if (shard_idx >= 0 && s != shard_idx) continue;
      uint64_t dev = 0;
      int64_t dev_bytes = 0;
      if (!mgr.DeviceStorage(static_cast<size_t>(l), static_cast<size_t>(s), &dev, &dev_bytes)) {
        return Fail(KVX_INTERNAL, "storage lookup failed");
      }
      if (B <= 0) return Fail(KVX_INVALID_ARGUMENT, "zero-byte blocks");
      const int64_t pool = dev_bytes / B;
      if (first) {
        for (int64_t i = 0; i < n; ++i) {
          if (ids[i] < 0) {
            return Fail(KVX_INVALID_ARGUMENT, "block ids must be non-negative");
          }
          if (ids[i] >= pool) return Fail(KVX_OUT_OF_RANGE, "block id exceeds device buffer");
        }
        first = false;
      }
      int g = 0;
      while (g < ngroups && gbytes[g] != B) ++g;
      if (g == ngroups) {
        if (ngroups == kMaxGroups) {
          return Fail(KVX_INVALID_ARGUMENT, "more distinct block sizes than one call handles");
        }
        gbytes[g] = B;
        gpool[g] = pool;
        gcount[g] = 0;
        ++ngroups;
      }
      if (pool < gpool[g]) gpool[g] = pool;
      ++gcount[g];
      ++nstorages;
      acc |= dev;
    }
  }
  if (nstorages > kNoAllocMaxStorages) {
    return Fail(KVX_INVALID_ARGUMENT,
                "kvx_manager_gather_no_alloc: more storages than its scratch holds");
  }
  int64_t need = 0;
  for (int g = 0; g < ngroups; ++g) {
    if (gcount[g] * n > static_cast<int64_t>(UINT32_MAX)) {
      return Fail(KVX_INVALID_ARGUMENT, "copy too large for one launch");
    }
    need += gcount[g] * gbytes[g] * n;
  }
  for (int64_t i = 0; i < n; ++i) {
    for (int g = 0; g < ngroups; ++g) {
      if (ids[i] >= gpool[g]) return Fail(KVX_OUT_OF_RANGE, "block id exceeds device buffer");
    }
  }
  if (staging == 0 && need > 0) return Fail(KVX_INVALID_ARGUMENT, "null staging buffer");
  if (staging_bytes < need) {
    char msg[96];
    snprintf(msg, sizeof(msg), "staging buffer too small: need %lld bytes",
             static_cast<long long>(need));
    return Fail(KVX_INVALID_ARGUMENT, msg);
  }
  if (n == 0 || nstorages == 0) return KVX_OK;
  if (order == KVX_BLOCK_MAJOR && ngroups != 1) {
    return Fail(KVX_INVALID_ARGUMENT, "block-major staging needs one block size");
  }
  // The bytes this gather writes must be device memory of the manager's
  // device (a runtime lookup: it allocates nothing).
  Status chk = CheckDeviceRange(device, staging, static_cast<uint64_t>(need), "staging");
  if (!chk.ok()) return Fail(chk);

  DeviceGuard dg(device);
  if (!dg.ok()) return Fail(KVX_INTERNAL, "hipSetDevice failed");
  hipStream_t st = static_cast<hipStream_t>(stream);
  CallOrder& ord = g_order[device];
  std::lock_guard<std::mutex> order_lock(ord.mu);
  if (ord.last == nullptr) return Fail(KVX_INTERNAL, "no-alloc ordering event was not set up");
  hipError_t e = hipSuccess;
  if (ord.recorded && ord.stream != st) e = hipStreamWaitEvent(st, ord.last, 0);
  if (e != hipSuccess) {
    return Fail(KVX_INTERNAL, (std::string("stream wait failed: ") +
                               hipGetErrorString(e)).c_str());
  }
  // Whatever this call launches, the next call on another stream waits for
  // it (also after a failed launch, whose fills may have run).
  struct RecordOnExit {
    CallOrder& o;
    hipStream_t s;
    ~RecordOnExit() {
      if (hipEventRecord(o.last, s) == hipSuccess) {
        o.stream = s;
        o.recorded = true;
      }
    }
  } record_on_exit{ord, st};
  ScratchWriter wr(scratch_addr, st);
  for (int64_t i = 0; i < n && e == hipSuccess; ++i) e = wr.Push(static_cast<uint64_t>(ids[i]));
  const uint64_t table0 = (static_cast<uint64_t>(n) + 31) / 32 * 32;
  if (e == hipSuccess) e = wr.SkipTo(table0);
  for (int g = 0; g < ngroups && e == hipSuccess; ++g) {
    for (int64_t l = 0; l < L && e == hipSuccess; ++l) {
      if ((layer_idx >= 0 && l != layer_idx) ||
          mgr.LayerBlockByteSize(static_cast<size_t>(l)) != gbytes[g]) {
        continue;
      }
      for (int64_t s = 0; s < S && e == hipSuccess; ++s) {
        if (shard_idx >= 0 && s != shard_idx) continue;
        uint64_t dev = 0;
        int64_t dev_bytes = 0;
        mgr.DeviceStorage(static_cast<size_t>(l), static_cast<size_t>(s), &dev, &dev_bytes);
        e = wr.Push(dev);
      }
    }
  }
  if (e == hipSuccess) e = wr.Flush();
  if (e != hipSuccess) {
    return Fail(KVX_INTERNAL, (std::string("scratch fill launch failed: ") +
                               hipGetErrorString(e)).c_str());
  }

  // One block-copy launch per kMaxPieces groups, as kvx_manager_gather.
  uint64_t table = scratch_addr + table0 * 8;
  int64_t off = 0;
  for (int g0 = 0; g0 < ngroups; g0 += kMaxPieces) {
    CopyLaunch cl;
    cl.ids = reinterpret_cast<const int64_t*>(scratch_addr);
    cl.n = n;
    cl.gather_workgroups_per_cu = mgr.engine()->gather_workgroups_per_cu();
    for (int g = g0; g < ngroups && g < g0 + kMaxPieces; ++g) {
      const int64_t W = gcount[g];
      const int64_t B = gbytes[g];
      CopyPiece& c = cl.pieces[cl.npieces++];
      c.storages = table;
      c.staging = staging + static_cast<uint64_t>(off);
      c.stride_w = order == KVX_BLOCK_MAJOR ? B : n * B;
      c.stride_i = order == KVX_BLOCK_MAJOR ? W * B : B;
      c.f0 = 0;
      c.nblocks = W * n;
      c.block_bytes = B;
      c.pool_blocks = gpool[g];
      acc |= static_cast<uint64_t>(off);
      off += W * n * B;
      table += static_cast<uint64_t>(W) * 8;
    }
    const int vec = LaunchVectorBytes(cl, acc);
    e = LaunchBlockCopy(cl, CopyDir::kGather, vec, st);
    if (e != hipSuccess) {
      return Fail(e == hipErrorInvalidValue ? KVX_INVALID_ARGUMENT : KVX_INTERNAL,
                  (std::string("kernel launch failed: ") + hipGetErrorString(e)).c_str());
    }
  }
  return KVX_OK;
}
