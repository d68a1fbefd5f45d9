// Stream placement probe for gfx950: one wavefront that spins on the wall
// clock (a constant-rate counter read by wall_clock64) for a bounded time and
// records when it started and stopped.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "queue_probe.h"

namespace kvx {
namespace {

// Clock reads per probe at most: with a 64-cycle sleep between reads this is
// far beyond any probe length the host asks for, and it bounds the loop even
// if the clock did not advance.
constexpr uint32_t kMaxReads = 1u << 20;

__global__ __launch_bounds__(64) void queue_probe_kernel(uint64_t* out, uint64_t ticks) {
  const uint64_t t0 = static_cast<uint64_t>(wall_clock64());
  uint64_t t = t0;
  for (uint32_t k = 0; k < kMaxReads && t - t0 < ticks; ++k) {
    __builtin_amdgcn_s_sleep(1);
    t = static_cast<uint64_t>(wall_clock64());
  }
  if (threadIdx.x == 0) {
    out[0] = t0;
    out[1] = t;
  }
}

}  // namespace

hipError_t LaunchQueueProbe(uint64_t* out, uint64_t ticks, hipStream_t stream) {
  if (out == nullptr) return hipErrorInvalidValue;
  hipLaunchKernelGGL(queue_probe_kernel, dim3(1), dim3(64), 0, stream, out, ticks);
  return hipGetLastError();
}

}  // namespace kvx
