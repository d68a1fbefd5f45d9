#include "link_peaks.h"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <chrono>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "hip_util.h"
#include "sdma_engines.h"

namespace kvx {
namespace {

constexpr int kRounds = 3;
constexpr size_t kMaxBytes = 16ull << 30;
constexpr int kMaxReps = 1000;
constexpr uint8_t kDevicePattern = 0xA5;
constexpr uint8_t kHostPattern = 0x3C;

// Buffers and signals of one measurement, released on every path out.
struct Buffers {
  void* dev[2] = {nullptr, nullptr};
  uint8_t* host[2] = {nullptr, nullptr};
  hsa_signal_t sig[2] = {};
  hipStream_t stream = nullptr;
  ~Buffers() {
    if (stream != nullptr) (void)hipStreamDestroy(stream);
    for (hsa_signal_t s : sig) SdmaEngines::DestroySignal(s);
    for (void* d : dev) {
      if (d != nullptr) (void)hipFree(d);
    }
    for (uint8_t* h : host) {
      if (h != nullptr) (void)hipHostFree(h);
    }
  }
};

double Seconds(std::chrono::steady_clock::time_point t0) {
  return std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
}

// Samples of `n` bytes at `p` (first, last and 62 spread between) equal `v`.
bool Sampled(const uint8_t* p, size_t n, uint8_t v) {
  for (int k = 0; k < 64; ++k) {
    const size_t i = k == 63 ? n - 1 : (n / 63) * static_cast<size_t>(k);
    if (p[i] != v) return false;
  }
  return true;
}

}  // namespace

StatusOr<LinkPeaks> MeasureLinkPeaks(size_t bytes, int reps) {
  if (bytes == 0 || bytes > kMaxBytes || reps <= 0 || reps > kMaxReps) {
    return InvalidArgumentError("link peaks: bytes must be 1..16 GiB and reps 1..1000");
  }
  int device = 0;
  KVX_HIP_RETURN_IF_ERROR(hipGetDevice(&device));
  KVX_ASSIGN_OR_RETURN(std::unique_ptr<SdmaEngines> engines, SdmaEngines::Create(device));
  Buffers b;
  for (int k = 0; k < 2; ++k) {
    KVX_HIP_RETURN_IF_ERROR(hipMalloc(&b.dev[k], bytes));
    void* h = nullptr;
    KVX_HIP_RETURN_IF_ERROR(hipHostMalloc(&h, bytes, hipHostMallocDefault));
    b.host[k] = static_cast<uint8_t*>(h);
    KVX_ASSIGN_OR_RETURN(b.sig[k], SdmaEngines::NewSignal());
  }
  // dev[0] -> host[0] (D2H), host[1] -> dev[1] (H2D). Set-up and read-back
  // run on a stream of their own (not waiting for the caller's work).
  KVX_HIP_RETURN_IF_ERROR(hipStreamCreateWithFlags(&b.stream, hipStreamNonBlocking));
  KVX_HIP_RETURN_IF_ERROR(hipMemsetAsync(b.dev[0], kDevicePattern, bytes, b.stream));
  KVX_HIP_RETURN_IF_ERROR(hipMemsetAsync(b.dev[1], 0, bytes, b.stream));
  std::memset(b.host[0], 0, bytes);
  std::memset(b.host[1], kHostPattern, bytes);
  KVX_HIP_RETURN_IF_ERROR(hipStreamSynchronize(b.stream));

  auto d2h = [&]() { return engines->Start(true, b.host[0], b.dev[0], bytes, b.sig[0]); };
  auto h2d = [&]() { return engines->Start(false, b.dev[1], b.host[1], bytes, b.sig[1]); };
  KVX_RETURN_IF_ERROR(d2h());
  KVX_RETURN_IF_ERROR(SdmaEngines::Wait(b.sig[0]));
  KVX_RETURN_IF_ERROR(h2d());
  KVX_RETURN_IF_ERROR(SdmaEngines::Wait(b.sig[1]));

  double t_d2h = 1e30, t_h2d = 1e30, t_bi = 1e30;
  for (int r = 0; r < kRounds; ++r) {
    auto t0 = std::chrono::steady_clock::now();
    for (int i = 0; i < reps; ++i) {
      KVX_RETURN_IF_ERROR(d2h());
      KVX_RETURN_IF_ERROR(SdmaEngines::Wait(b.sig[0]));
    }
    t_d2h = std::min(t_d2h, Seconds(t0) / reps);
    t0 = std::chrono::steady_clock::now();
    for (int i = 0; i < reps; ++i) {
      KVX_RETURN_IF_ERROR(h2d());
      KVX_RETURN_IF_ERROR(SdmaEngines::Wait(b.sig[1]));
    }
    t_h2d = std::min(t_h2d, Seconds(t0) / reps);
    t0 = std::chrono::steady_clock::now();
    for (int i = 0; i < reps; ++i) {
      KVX_RETURN_IF_ERROR(d2h());
      // Both copies are waited for on every path once started (a copy that
      // failed to start leaves its signal at 0).
      const Status s = h2d();
      const Status w0 = SdmaEngines::Wait(b.sig[0]);
      const Status w1 = SdmaEngines::Wait(b.sig[1]);
      KVX_RETURN_IF_ERROR(s);
      KVX_RETURN_IF_ERROR(w0);
      KVX_RETURN_IF_ERROR(w1);
    }
    t_bi = std::min(t_bi, Seconds(t0) / reps);
  }
  // The bytes landed: the host copy of the device pattern, and the device
  // copy of the host pattern (read back into host[0], already checked).
  if (!Sampled(b.host[0], bytes, kDevicePattern)) {
    return InternalError("link peaks: device-to-host bytes did not land");
  }
  KVX_HIP_RETURN_IF_ERROR(
      hipMemcpyAsync(b.host[0], b.dev[1], bytes, hipMemcpyDeviceToHost, b.stream));
  KVX_HIP_RETURN_IF_ERROR(hipStreamSynchronize(b.stream));
  if (!Sampled(b.host[0], bytes, kHostPattern)) {
    return InternalError("link peaks: host-to-device bytes did not land");
  }
  LinkPeaks out;
  out.d2h_gbps = static_cast<double>(bytes) / t_d2h / 1e9;
  out.h2d_gbps = static_cast<double>(bytes) / t_h2d / 1e9;
  out.bidir_gbps = 2.0 * static_cast<double>(bytes) / t_bi / 1e9;
  out.engines = engines->engine(true) << 16 | engines->engine(false);
  return out;
}

}  // namespace kvx
