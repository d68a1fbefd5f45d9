// Checked placement of streams on hardware queues.
//
// The HIP runtime backs a process's streams with a few hardware queues and
// work on one queue runs in order, so two of the library's streams that share
// a queue serialize (an offload's DMA behind a reload's). Stream creation
// evens out the queues first (CreateStreamsOnDistinctQueues), which rests on
// the runtime's observed assignment policy; the probe here checks the result
// on the device: one short kernel per stream, all launched at once, and two
// streams whose kernels ran one after the other share a queue.
#ifndef KVX_HOST_QUEUE_CHECK_H_
#define KVX_HOST_QUEUE_CHECK_H_

#include <hip/hip_runtime_api.h>

#include <initializer_list>
#include <utility>
#include <vector>

#include "status.h"

namespace kvx {

// Pairs (i, j), i < j, of `streams` whose probes ran one after the other, in
// two probes in a row (a pair that overlapped in either is not counted: a
// GPU busy with other work can delay one probe past another once). At most
// 64 streams; the current device must be the streams' device.
StatusOr<std::vector<std::pair<int, int>>> SerializedStreamPairs(
    const std::vector<hipStream_t>& streams);

struct StreamPlacement {
  int attempts = 0;          // stream sets created (1: the first was kept)
  int serialized_pairs = 0;  // pairs still found on one queue after the last
};

// Creates the streams as CreateStreamsOnDistinctQueues does, then probes
// them. While a pair shares a queue, every stream is destroyed and created
// again behind twice as many spacer streams (which evens out queues whose
// stream counts differ by more), up to 3 sets. The last set is kept either
// way; *placement says how it went.
Status CreateStreamsOnDistinctQueuesChecked(std::initializer_list<hipStream_t*> out,
                                            StreamPlacement* placement);

}  // namespace kvx

#endif  // KVX_HOST_QUEUE_CHECK_H_
