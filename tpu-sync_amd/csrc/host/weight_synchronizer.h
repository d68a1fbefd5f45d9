// Weight sync on one GPU: the host-staging half of the reference's
// WeightSynchronizerBase (tpu_sync/weight_sync/weight_synchronizer_base.h:
// 78-240; D2h / D2hLayer / H2d / H2dLayer at
// weight_synchronizer_base.cc:307-539) for row-major GPU tensors.
//
// Each (layer, shard) is one device tensor ("layer" = one weight). Their host
// copies live in ONE pinned buffer at a per-tensor offset table (ascending,
// 256-byte aligned; bytes between tensors are unspecified), so the whole
// parameter set moves as a few large DMAs:
//   * D2h: the offset-table pack kernel gathers the scattered tensors chunk by
//     chunk into a device staging ring; each chunk then crosses PCIe as one
//     hipMemcpyAsync on the same stream;
//   * H2d: the mirror image (one H2D per chunk, then the unpack kernel);
//   * D2hLayer / H2dLayer: one direct copy per shard of that weight, as the
//     reference issues.
// Pack / Unpack run the same kernel against a caller device buffer laid out
// by the offset table (device-side contiguous staging), and CopyStrided runs
// arbitrary strided push entries (column-split resharding) on the device;
// StridedCopyPlan keeps such entries' device table for repeated runs.
//
// A tensor may be stored in a tiled layout (TiledPlan). Its host copy is
// then the row-major (linear) image, as the reference's D2hLayer / H2dLayer
// produce by detiling / tiling on the host around a raw DMA of the tiled
// bytes (weight_synchronizer_base.cc:357-389, 473-510). Here the tiled-copy
// kernel does it in HBM: D2h detiles into the staging chunk the DMA reads,
// H2d tiles out of the chunk the DMA wrote (padding cleared first). Chunk
// boundaries inside a tiled tensor fall on its tile rows.
#ifndef KVX_HOST_WEIGHT_SYNCHRONIZER_H_
#define KVX_HOST_WEIGHT_SYNCHRONIZER_H_

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <memory>
#include <mutex>
#include <utility>
#include <vector>

#include "../kernels/strided_copy.h"
#include "arg_ring.h"
#include "copy_future.h"
#include "host_allocator.h"
#include "status.h"
#include "tiled_layout.h"

namespace kvx {

struct WeightSyncConfig {
  int device = 0;
  int64_t num_layers = 0;
  int64_t num_shards = 1;
  std::vector<uint64_t> device_ptrs;  // [layer * num_shards + shard]
  std::vector<int64_t> device_bytes;
  // Per tensor (empty: none): a tiled layout, or null for row-major bytes.
  // A tiled tensor's device buffer holds at least plan->tiled_bytes and its
  // host copy plan->logical_bytes.
  std::vector<std::shared_ptr<const TiledPlan>> tiled;
  HostAllocKind host_alloc = HostAllocKind::kPinned;
  int64_t chunk_bytes = 256ll << 20;  // device staging chunk
  int staging_chunks = 2;
  bool profile_kernels = false;
  // The host image prefers the GPU's NUMA node (false: OS placement).
  bool numa_local = true;
};

class WeightSynchronizer {
 public:
  static StatusOr<std::unique_ptr<WeightSynchronizer>> Create(WeightSyncConfig cfg);
  ~WeightSynchronizer();

  // NUMA node of the host image, or -1.
  int numa_node() const { return numa_node_; }
  StatusOr<CopyFuture> D2h(hipStream_t dep = nullptr);
  StatusOr<CopyFuture> H2d(hipStream_t dep = nullptr);
  StatusOr<CopyFuture> D2hLayer(int64_t layer, hipStream_t dep = nullptr);
  StatusOr<CopyFuture> H2dLayer(int64_t layer, hipStream_t dep = nullptr);
  // Device-side pack of every tensor into `staging` at its offset (and the
  // reverse); staging must hold total_bytes().
  StatusOr<CopyFuture> Pack(uint64_t staging, int64_t staging_bytes, hipStream_t stream);
  StatusOr<CopyFuture> Unpack(uint64_t staging, int64_t staging_bytes, hipStream_t stream);

  int64_t num_layers() const { return cfg_.num_layers; }
  int64_t num_shards() const { return cfg_.num_shards; }
  int64_t total_bytes() const { return total_; }
  int device() const { return cfg_.device; }
  int64_t offset(int64_t layer, int64_t shard) const { return off_[layer * cfg_.num_shards + shard]; }
  // Bytes of one tensor's host copy (the linear image of a tiled tensor).
  int64_t size(int64_t layer, int64_t shard) const { return host_bytes_[layer * cfg_.num_shards + shard]; }
  uint8_t* host_base() const { return host_.ptr; }
  Status Synchronize();
  // Profiled pack (pack = true) or unpack kernel launches: count, summed
  // milliseconds (HIP events on the kernel stream), bytes moved.
  Status KernelTimes(bool pack, bool reset, int64_t* launches, double* ms, int64_t* bytes);

 private:
  explicit WeightSynchronizer(WeightSyncConfig cfg) : cfg_(std::move(cfg)) {}
  Status Init();
  StatusOr<CopyFuture> Chunked(bool d2h, hipStream_t dep);
  // Chunks [range_lo, range_hi) of the packed image through the ring on the
  // direction's stream (lock held, dependency already ordered).
  Status ChunkRange(bool d2h, int64_t range_lo, int64_t range_hi);
  // Largest cut point in (lo, x] of the packed image, or an error when a
  // tiled tensor's tile row does not fit between lo and x.
  StatusOr<int64_t> CutBelow(int64_t lo, int64_t x) const;
  StatusOr<CopyFuture> WholeCopy(bool pack, uint64_t staging, int64_t bytes,
                                 hipStream_t stream);
  // Entries for packed range [lo, hi) with the image placed at `image`
  // (pack: tensors -> image; unpack: image -> tensors).
  // Tiled tensors become tiled-copy jobs (*zero: padding cleared before
  // *tiled runs); the rest strided entries.
  Status RangeEntries(int64_t lo, int64_t hi, uint64_t image, bool pack,
                      std::vector<StridedCopy>* out, std::vector<TiledJob>* zero,
                      std::vector<TiledJob>* tiled) const;
  Status Launch(const std::vector<StridedCopy>& copies, const std::vector<TiledJob>& zero,
                const std::vector<TiledJob>& tiled, bool pack, hipStream_t stream);
  // Tiled layout of tensor k, or null for row-major bytes.
  const TiledPlan* plan(int64_t k) const {
    if (cfg_.tiled.empty() || cfg_.tiled[k] == nullptr || !cfg_.tiled[k]->tiled) return nullptr;
    return cfg_.tiled[k].get();
  }
  Status WaitDep(hipStream_t dep, hipStream_t on);

  struct Sample {
    hipEvent_t start = nullptr;
    hipEvent_t stop = nullptr;
    int64_t bytes = 0;
    bool pack = true;
  };

  WeightSyncConfig cfg_;
  std::vector<int64_t> off_;
  std::vector<int64_t> host_bytes_;
  int64_t total_ = 0;
  int numa_node_ = -1;
  HostBufferAllocation host_;
  std::mutex mu_;
  hipStream_t ks_ = nullptr;
  hipStream_t d2h_ = nullptr;
  hipStream_t h2d_ = nullptr;
  std::vector<uint64_t> ring_;
  std::vector<hipEvent_t> free_;           // recorded after each use of a slot
  std::vector<hipStream_t> slot_stream_;  // the stream of that use (null: none)
  size_t next_ = 0;
  ArgRing args_;
  std::vector<Sample> samples_;
};

// Runs arbitrary strided entries with device addresses in one launch on
// `stream` (no synchronizer needed); returns a future for the launch.
StatusOr<CopyFuture> CopyStridedOnDevice(int device, const std::vector<StridedCopy>& copies,
                                         hipStream_t stream);

// TileBuffer (tile = true: linear -> tiled, padding zero) or DetileBuffer
// (tiling_utils.h:30-36) of one tensor between device buffers, on `stream`.
// `tiled` holds plan.tiled_bytes, `linear` plan.logical_bytes.
StatusOr<CopyFuture> TileOnDevice(int device, const TiledPlan& plan, uint64_t linear,
                                  uint64_t tiled, bool tile, hipStream_t stream);

// Strided entries whose device image (entry table + tile map) is built and
// uploaded once, for callers that run the same entries again and again: a
// weight push repeats the same expansion every time
// (weight_synchronizer_base.cc:626-666). A run is one launch with no host
// table work and no upload. The addresses the entries name must stay valid
// while the plan is run. Runs may come from any thread.
class StridedCopyPlan {
 public:
  static StatusOr<std::unique_ptr<StridedCopyPlan>> Create(int device,
                                                           const std::vector<StridedCopy>& copies);
  // Waits for every run still in flight, then frees the image.
  ~StridedCopyPlan();
  StridedCopyPlan(const StridedCopyPlan&) = delete;
  StridedCopyPlan& operator=(const StridedCopyPlan&) = delete;

  StatusOr<CopyFuture> Run(hipStream_t stream);
  uint32_t workgroups() const { return grid_; }
  // With profiling on, each later run records a pair of timing events right
  // around its launch (and nothing else between them) on its stream.
  void SetProfiling(bool on);
  // Launches, summed duration and algorithmic HBM bytes (2 x bytes moved)
  // of the profiled runs so far; waits for them; reset drops them.
  Status KernelTimes(bool reset, int64_t* launches, double* ms, int64_t* bytes);

 private:
  StridedCopyPlan() = default;
  int device_ = 0;
  int vec_ = 16;
  uint32_t n_ = 0;
  uint32_t grid_ = 0;
  uint32_t long_tiles_ = 0;  // the first tiles of the grid, long rows (sliced)
  int64_t bytes_ = 0;  // bytes one run moves
  void* image_ = nullptr;
  std::mutex mu_;
  std::vector<hipEvent_t> runs_;  // one per run that may still read the image
  bool profile_ = false;
  std::vector<std::pair<hipEvent_t, hipEvent_t>> samples_;  // (start, stop) per profiled run
};

}  // namespace kvx

#endif  // KVX_HOST_WEIGHT_SYNCHRONIZER_H_
