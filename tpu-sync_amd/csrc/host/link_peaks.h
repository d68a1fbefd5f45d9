// Pinned-host <-> device copy rates on the SDMA engines the pageable lanes
// use, one direction at a time and both at once.
//
// hipMemcpyAsync leaves the engine to the runtime, which in some processes
// puts a host-to-device and a device-to-host copy issued together on one
// engine (they then run one after the other, at one direction's rate). The
// lanes choose an engine per direction (SdmaEngines), so their bound is the
// link's rate on those engines, measured here the same way.
#ifndef KVX_HOST_LINK_PEAKS_H_
#define KVX_HOST_LINK_PEAKS_H_

#include <cstddef>
#include <cstdint>

#include "status.h"

namespace kvx {

struct LinkPeaks {
  double d2h_gbps = 0;    // device -> pinned host, alone
  double h2d_gbps = 0;    // pinned host -> device, alone
  double bidir_gbps = 0;  // both at once (bytes of both / time)
  uint32_t engines = 0;   // device-to-host engine bit << 16 | host-to-device
};

// Copies of `bytes` between a device buffer and a pinned host buffer on the
// current device: per measure the best of 3 rounds of `reps` copies, after
// one warm-up copy per direction. Allocates 2 x `bytes` of device memory and
// 2 x `bytes` of pinned host memory for the call, and checks that the bytes
// landed. `bytes` 1..16 GiB, `reps` 1..1000. UNAVAILABLE when ROCr offers no
// SDMA engine for host copies.
StatusOr<LinkPeaks> MeasureLinkPeaks(size_t bytes, int reps);

}  // namespace kvx

#endif  // KVX_HOST_LINK_PEAKS_H_
