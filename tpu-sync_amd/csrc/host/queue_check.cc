#include "queue_check.h"

#include <mutex>
#include <string>

#include "../kernels/queue_probe.h"
#include "hip_util.h"

namespace kvx {
namespace {

// Probe length: long enough that the host has enqueued every probe (a few
// microseconds apart) before the first one ends, short enough to go unseen
// at stream creation.
constexpr double kProbeSeconds = 200e-6;

// Stream sets created at most by the checked creation.
constexpr int kAttempts = 3;

// The probes' clock words: 2 per stream, one buffer per device, allocated on
// first use and kept for the process (freeing it would make the probe wait
// for all of the device's work).
constexpr int kMaxDevices = 64;
constexpr size_t kMaxStreams = 64;

StatusOr<uint64_t*> ProbeBuffer(int device) {
  static std::mutex mu;
  static uint64_t* bufs[kMaxDevices] = {};
  if (device < 0 || device >= kMaxDevices) return InvalidArgumentError("stream probe: bad device");
  std::lock_guard<std::mutex> lock(mu);
  if (bufs[device] == nullptr) {
    void* p = nullptr;
    KVX_HIP_RETURN_IF_ERROR(hipMalloc(&p, 2 * kMaxStreams * sizeof(uint64_t)));
    bufs[device] = static_cast<uint64_t*>(p);
  }
  return bufs[device];
}

// One probe of every stream: ser[i * n + j] is cleared for each pair (i, j)
// whose intervals overlapped.
Status ProbeOnce(const std::vector<hipStream_t>& streams, uint64_t* dev, uint64_t ticks,
                 std::vector<char>* ser) {
  const size_t n = streams.size();
  for (size_t i = 0; i < n; ++i) {
    KVX_HIP_RETURN_IF_ERROR(LaunchQueueProbe(dev + 2 * i, ticks, streams[i]));
  }
  for (size_t i = 0; i < n; ++i) {
    KVX_HIP_RETURN_IF_ERROR(hipStreamSynchronize(streams[i]));
  }
  // Read back on a probed stream (not the null stream, which would also wait
  // for the caller's work there).
  std::vector<uint64_t> h(2 * n);
  KVX_HIP_RETURN_IF_ERROR(hipMemcpyAsync(h.data(), dev, 2 * n * sizeof(uint64_t),
                                         hipMemcpyDeviceToHost, streams[0]));
  KVX_HIP_RETURN_IF_ERROR(hipStreamSynchronize(streams[0]));
  for (size_t i = 0; i < n; ++i) {
    if (h[2 * i + 1] < h[2 * i]) return InternalError("stream probe: clock went backwards");
  }
  for (size_t i = 0; i < n; ++i) {
    for (size_t j = i + 1; j < n; ++j) {
      const bool overlap = h[2 * j] < h[2 * i + 1] && h[2 * i] < h[2 * j + 1];
      if (overlap) (*ser)[i * n + j] = 0;
    }
  }
  return OkStatus();
}

}  // namespace

StatusOr<std::vector<std::pair<int, int>>> SerializedStreamPairs(
    const std::vector<hipStream_t>& streams) {
  const size_t n = streams.size();
  if (n > kMaxStreams) return InvalidArgumentError("stream probe: at most 64 streams");
  std::vector<std::pair<int, int>> pairs;
  if (n < 2) return pairs;
  int device = 0;
  KVX_HIP_RETURN_IF_ERROR(hipGetDevice(&device));
  // The probes write this device's buffer: every stream must belong to it.
  for (hipStream_t st : streams) {
    hipDevice_t sd = -1;
    if (hipStreamGetDevice(st, &sd) != hipSuccess) {
      (void)hipGetLastError();
      return InvalidArgumentError("stream probe: not a valid stream");
    }
    if (sd != device) {
      return InvalidArgumentError("stream probe: a stream of device " + std::to_string(sd) +
                                  ", not of the current device " + std::to_string(device));
    }
  }
  int khz = 0;
  if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, device) != hipSuccess ||
      khz <= 0) {
    (void)hipGetLastError();
    khz = 100000;  // gfx9's wall clock: 100 MHz
  }
  const uint64_t ticks = static_cast<uint64_t>(kProbeSeconds * khz * 1e3);
  KVX_ASSIGN_OR_RETURN(uint64_t* buf, ProbeBuffer(device));
  // Probes of concurrent callers on one device share the buffer.
  static std::mutex probe_mu;
  std::lock_guard<std::mutex> lock(probe_mu);
  std::vector<char> ser(n * n, 1);
  for (int round = 0; round < 2; ++round) {
    KVX_RETURN_IF_ERROR(ProbeOnce(streams, buf, ticks, &ser));
  }
  for (size_t i = 0; i < n; ++i) {
    for (size_t j = i + 1; j < n; ++j) {
      if (ser[i * n + j]) pairs.emplace_back(static_cast<int>(i), static_cast<int>(j));
    }
  }
  return pairs;
}

Status CreateStreamsOnDistinctQueuesChecked(std::initializer_list<hipStream_t*> out,
                                            StreamPlacement* placement) {
  const std::vector<hipStream_t*> outs(out);
  const int queues = HwQueuesPerProcess();
  // More streams than queues cannot all be apart: one set, probed once.
  const int attempts = static_cast<int>(outs.size()) <= queues ? kAttempts : 1;
  int spacers = queues;
  StreamPlacement pl;
  for (int a = 1; a <= attempts; ++a) {
    if (a > 1) {
      for (hipStream_t* s : outs) {
        (void)hipStreamDestroy(*s);
        *s = nullptr;
      }
    }
    KVX_RETURN_IF_ERROR(CreateStreamsOnDistinctQueues(outs, spacers));
    pl.attempts = a;
    std::vector<hipStream_t> ss;
    for (hipStream_t* s : outs) ss.push_back(*s);
    StatusOr<std::vector<std::pair<int, int>>> pairs = SerializedStreamPairs(ss);
    if (!pairs.ok()) {
      // The probe is a check, not a requirement: keep the streams.
      (void)hipGetLastError();
      pl.serialized_pairs = -1;
      break;
    }
    pl.serialized_pairs = static_cast<int>(pairs->size());
    if (pairs->empty()) break;
    spacers *= 2;
  }
  if (placement != nullptr) *placement = pl;
  return OkStatus();
}

}  // namespace kvx
