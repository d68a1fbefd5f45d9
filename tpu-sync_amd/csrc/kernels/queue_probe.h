// Host-side interface of the stream placement probe kernel (gfx950).
//
// Work on one hardware queue runs in submission order; work on different
// queues can run at once. The probe kernel is one wavefront that spins on
// the GPU's constant-rate wall clock for a given number of ticks and records
// the clock when it started and when it stopped, so the intervals of probes
// launched on several streams at once show which streams ran one after the
// other.
#ifndef KVX_KERNELS_QUEUE_PROBE_H_
#define KVX_KERNELS_QUEUE_PROBE_H_

#include <hip/hip_runtime_api.h>

#include <cstdint>

namespace kvx {

// Launches one probe on `stream`: out[0] = wall clock at its start, out[1] =
// at its end, after about `ticks` ticks (and at most 2^20 clock reads, so it
// ends whatever the clock does). `out` is device memory of two words.
hipError_t LaunchQueueProbe(uint64_t* out, uint64_t ticks, hipStream_t stream);

}  // namespace kvx

#endif  // KVX_KERNELS_QUEUE_PROBE_H_
