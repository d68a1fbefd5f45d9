// Device <-> pinned-host DMA on chosen SDMA engines, for the pageable lanes.
//
// hipMemcpyAsync leaves the engine to the runtime, which picks one per copy:
// a lane's device-to-host copies then run as blit kernels or land on the
// engine already busy with the other lane's host-to-device copies, and a load
// and a save through the lanes at once reach about 75 of the 96 GB/s the
// link carries in both directions (measured on MI355X, 64 MiB chunks). ROCr's
// hsa_amd_memory_async_copy_on_engine takes the engine as an argument, so
// each direction keeps an engine of its own.
#ifndef KVX_HOST_SDMA_ENGINES_H_
#define KVX_HOST_SDMA_ENGINES_H_

#include <hsa/hsa.h>
#include <hsa/hsa_ext_amd.h>

#include <cstddef>
#include <cstdint>
#include <memory>

#include "status.h"

namespace kvx {

class SdmaEngines {
 public:
  // The ROCr agents of HIP device `device` (matched by PCI location) and of
  // host memory, and one SDMA engine per direction: distinct ones when the
  // device offers two. An error if ROCr cannot provide them; callers then
  // copy with hipMemcpyAsync.
  static StatusOr<std::unique_ptr<SdmaEngines>> Create(int device);
  // Gives back the ROCr reference Create took (HIP holds its own).
  ~SdmaEngines();
  SdmaEngines(const SdmaEngines&) = delete;
  SdmaEngines& operator=(const SdmaEngines&) = delete;

  // Starts a copy of `bytes` from `src` to `dst` on the direction's engine:
  // device memory to pinned host memory (d2h) or the reverse. `done` is set
  // to 1 here and drops to 0 when the bytes have landed (below 0 if the copy
  // failed).
  Status Start(bool d2h, void* dst, const void* src, size_t bytes, hsa_signal_t done) const;

  // Blocks until `done` drops below 1; an error if the copy failed.
  static Status Wait(hsa_signal_t done);

  static StatusOr<hsa_signal_t> NewSignal();
  static void DestroySignal(hsa_signal_t s);

  // Engine bit (hsa_amd_sdma_engine_id_t) of a direction.
  uint32_t engine(bool d2h) const { return d2h ? d2h_engine_ : h2d_engine_; }

 private:
  SdmaEngines() = default;
  bool hsa_ref_ = false;
  hsa_agent_t gpu_{};
  hsa_agent_t cpu_{};
  uint32_t h2d_engine_ = 0;
  uint32_t d2h_engine_ = 0;
};

}  // namespace kvx

#endif  // KVX_HOST_SDMA_ENGINES_H_
