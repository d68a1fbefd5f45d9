// Block transfer engine: moves whole blocks between paged device storages
// and host mirrors on one GPU.
//
// The reference issues one raw DMA per (layer, shard, run)
// (tpu_sync/kv_cache/kv_cache_manager_base.cc:1944-2124 ->
// tpu_sync/core/raw_transfer_core.h:638-692). Here a copy is planned as:
//   * direct: every run is large, so one hipMemcpyAsync per (storage, run)
//     between the device storage and the host mirror;
//   * staged (scattered device ids): the gather kernel packs the blocks of a
//     chunk of storages into a device staging buffer in host-id order, then a
//     few large hipMemcpyAsync move each host run; reload is the mirror image
//     (H2D into staging, then the scatter kernel).
// Staged copies are pipelined over a ring of staging buffers: the kernel
// stream and the copy stream hand chunks to each other with events, so the
// gather of chunk c+1 overlaps the DMA of chunk c and nothing blocks the
// host. D2H and H2D use separate stream pairs and rings, so an offload and a
// reload can run at the same time in both PCIe directions.
#ifndef KVX_HOST_TRANSFER_ENGINE_H_
#define KVX_HOST_TRANSFER_ENGINE_H_

#include <hip/hip_runtime_api.h>

#include <climits>
#include <cstdint>
#include <deque>
#include <functional>
#include <memory>
#include <mutex>
#include <vector>

#include "../kernels/block_copy.h"
#include "arg_ring.h"
#include "copy_future.h"
#include "queue_check.h"
#include "sdma_engines.h"
#include "status.h"

namespace kvx {

struct CopyLaunch;

// One storage as seen by one copy: a device buffer of pool blocks and the
// host region (a mirror or a staging-slot span) the copy reads or writes.
struct StorageView {
  uint64_t dev = 0;
  int64_t dev_bytes = 0;
  uint8_t* host = nullptr;
  int64_t host_bytes = 0;
  int64_t block_bytes = 0;
  // The host region is page-locked and mapped into the GPU's address space
  // (hipHostMalloc), so kernels may read and write it directly.
  bool host_kernel_access = false;
};

enum class Direction : int { kD2H = 0, kH2D = 1 };

// A byte range at the same offset in a storage's device buffer and in its
// host region (pool-block copies address both sides alike).
struct ByteExtent {
  int64_t offset = 0;
  int64_t bytes = 0;
};

// How a block copy with short runs crosses PCIe.
//   kStaged: gather kernel -> device staging ring -> hipMemcpyAsync (and the
//            mirror image for reload), pipelined chunk by chunk;
//   kZeroCopy: one kernel moves every block between the pool and the pinned
//            host mirror directly (GPU loads/stores over PCIe), no staging;
//   kAuto: staged when the host ids form long runs (average run of a
//          storage at least auto_staged_min_run_bytes); zero-copy otherwise;
//          a copy of more than auto_lanes_min_chunks staging chunks, or a
//          staged one that would leave more than that many staged chunks of
//          its direction in flight, goes through the lanes (as kLanes); so
//          does a short-run copy while the engine sees both directions at
//          work (auto_duplex_window_us). Host memory the GPU cannot map
//          always goes staged (through the pageable lanes).
//   kLanes: pinned host memory too goes through the pageable lanes (host
//          threads move the host side, whole chunks cross on SDMA): a load
//          and a save at once reach the link's duplex rate, where zero-copy
//          kernels in both directions interfere.
// Copies whose runs are all at least direct_min_bytes use one
// hipMemcpyAsync per (storage, run) in every mode, except that kAuto moves
// such runs of a pinned mirror zero-copy when they average under
// auto_direct_min_run_bytes and the other direction is idle.
enum class TransferMode : int { kAuto = 0, kStaged = 1, kZeroCopy = 2, kLanes = 3 };

struct EngineOptions {
  int device = 0;
  int64_t staging_chunk_bytes = 64ll << 20;
  int staging_chunks = 4;
  int64_t arg_ring_bytes = 8ll << 20;
  // A run moves directly (no staging) only when every run of the copy is at
  // least this many bytes.
  int64_t direct_min_bytes = 4ll << 20;
  // Bracket every kernel launch with timing events on its stream.
  bool profile_kernels = false;
  TransferMode mode = TransferMode::kAuto;
  // Workgroup caps of a zero-copy launch. A few dozen workgroups keep enough
  // 16-byte accesses in flight to fill the PCIe link in either direction;
  // more D2H writers crowd out the reads of a reload running at the same
  // time (measured on MI355X: 16 writers / 64 readers).
  int64_t zero_copy_d2h_workgroups = 16;
  int64_t zero_copy_h2d_workgroups = 64;
  // kAuto stages a copy whose host runs average at least this many bytes
  // per storage. Measured on MI355X (Llama-3-8B KV, 64 storages): alone in
  // its direction the zero-copy kernel is as fast or faster at every run
  // length; with an offload and a reload in flight together, staging (SDMA
  // for H2D) wins from 4 MiB runs (83 against 79 GB/s; 16 MiB: 93 against
  // 82) and loses at 2 MiB and below (71 against 73; 1 MiB: 51 against 64).
  int64_t auto_staged_min_run_bytes = 4ll << 20;
  // kAuto moves a pinned-mirror copy of more than this many staging chunks
  // through the lanes (when host_copy_threads > 0), and a staged copy too
  // when its chunks and those of the direction's staged copies still in
  // flight exceed it. The staged path enqueues every chunk of a copy at once
  // (kernels and copies chained over two streams by events), and chains far
  // deeper than the ring slow the runtime's copies: 1024 blocks of 5 MiB in
  // 32 MiB chunks (160 chunks) took 220-270 ms D2H alone against 97 ms with
  // the host issuing a chunk only once its ring slot was free; a load and a
  // save of that size at once fell to 25 GB/s; eight 640 MiB offloads issued
  // together took 148, 233, then 390 ms (the same copies one by one: 109 ms
  // each time). The same slowdown shows with torch's own copies chained
  // that way, and not on one stream. The lanes issue chunk by chunk from
  // their own threads: 96.7 ms alone and 113 ms both ways for the 1024
  // blocks; zero-copy 96.3 / 127.5 ms. Below the threshold the staged and
  // zero-copy paths are as fast or faster (a lone 64-block copy: zero-copy
  // 6.1 ms, lanes 6.5).
  int64_t auto_lanes_min_chunks = 32;
  // kAuto moves a short-run copy (one that would go zero-copy) through the
  // lanes, when host_copy_threads > 0, while a copy of the other direction
  // is in flight or was within this many microseconds of such an overlap
  // (0: never). Zero-copy kernels in both directions interfere (load + save
  // of 512 Llama-3-70B blocks each way on a pinned tier: 63-64 ms, against
  // 56.9 ms through the lanes), while a lone short copy is fastest
  // zero-copy (64 blocks: 6.05 against 6.5 ms). The window keeps both
  // directions of a load + save pattern on the same path: a zero-copy save
  // next to lane loads is the slowest mix of all (94 ms).
  int64_t auto_duplex_window_us = 250000;
  // kAuto moves a copy whose runs would go directly (all at least
  // direct_min_bytes, or blocks larger than a staging chunk) with one
  // zero-copy launch instead, when the mirror is pinned, the other direction
  // is idle (as for auto_duplex_window_us) and the runs average under this
  // many bytes per storage (0: never). A DMA per run pays a fixed cost per
  // run that one launch does not. Measured on MI355X (16 runs of one block
  // per storage, each direction alone, in one process alternating): 8 MiB
  // runs 53.2 / 53.4 GB/s D2H / H2D directly against 55.2 / 55.8 zero-copy,
  // 16 MiB 55.0 / 55.3 against 55.6 / 56.2, 32 MiB 56.0 / 56.3 against
  // 55.8 / 56.3. With both directions at work the DMAs stay: zero-copy
  // kernels in both directions interfere.
  int64_t auto_direct_min_run_bytes = 32ll << 20;
  // Host regions the GPU cannot map (malloc, /dev/shm) move through pinned
  // bounce buffers that this many host threads fill and drain, one lane per
  // direction with its own streams, staging ring and SDMA engine (0: leave
  // such copies to the runtime's pageable hipMemcpyAsync).
  int host_copy_threads = 8;
  // Workgroups of a one-block-per-workgroup gather that may share a CU
  // (CopyLaunch::gather_workgroups_per_cu; 0: no limit).
  int gather_workgroups_per_cu = kDefaultGatherWorkgroupsPerCu;
};

// Where DeviceCopy puts block k of storage s in its staging buffer:
// base[s] + k * stride_k[s]. Storages of equal block size form groups in
// first-appearance order; layer-major staging is, group after group,
// [member][n][block]; block-major staging needs one block size and is
// [n][storage][block].
struct StagingLayout {
  std::vector<int64_t> base;
  std::vector<int64_t> stride_k;
  int64_t total_bytes = 0;
};
StatusOr<StagingLayout> DeviceStagingLayout(const std::vector<int64_t>& block_bytes, int64_t n,
                                            bool block_major);

// Accumulated duration of the profiled launches of one kernel direction.
struct KernelTimes {
  int64_t launches = 0;
  double total_ms = 0;
  int64_t bytes = 0;  // algorithmic HBM bytes: 2 x bytes moved
};

// Counters of what the engine issued (for tests and the benchmark).
struct EngineStats {
  int64_t direct_copies = 0;
  int64_t staged_copies = 0;
  int64_t memcpy_calls = 0;
  int64_t kernel_launches = 0;
  int64_t chunks = 0;
  int64_t zero_copy_copies = 0;
  int64_t extent_kernel_copies = 0;
  int64_t bounce_copies = 0;  // copies through the pageable-host lanes
};

class TransferEngine {
 public:
  static StatusOr<std::unique_ptr<TransferEngine>> Create(
      const EngineOptions& opts);
  ~TransferEngine();

  // Copies runs of whole blocks for every storage in `storages`:
  // D2H: device block src[r]+k -> host block dst[r]+k;
  // H2D: host block src[r]+k -> device block dst[r]+k, for k < sizes[r].
  // Offsets are in blocks of each storage's own block size. The caller has
  // validated every range. If `dep` is non-null the copy is ordered after
  // the work already enqueued on it.
  StatusOr<CopyFuture> Copy(Direction dir,
                            const std::vector<StorageView>& storages,
                            const std::vector<int64_t>& src,
                            const std::vector<int64_t>& dst,
                            const std::vector<int64_t>& sizes,
                            hipStream_t dep);

  // Whole-buffer copy of `bytes` per storage (the reference's empty-spec
  // full-layer copy): one hipMemcpyAsync per storage, or through a bounce
  // lane for pageable host memory.
  StatusOr<CopyFuture> CopyFull(Direction dir,
                                const std::vector<StorageView>& storages,
                                const std::vector<int64_t>& bytes,
                                hipStream_t dep);

  // Copies `extents` of every storage between its device buffer and its
  // host region, the same offsets on both sides. With a page-locked host
  // region, extents shorter than direct_min_bytes go through one
  // strided-copy kernel that reads and writes it directly (no staging),
  // longer ones through one hipMemcpyAsync per (storage, extent). A pageable
  // host region (host_copy_threads > 0) goes through a bounce lane: the
  // strided kernel packs the live bytes into staging chunks, one DMA per
  // chunk, host threads place them. The caller has validated every range.
  StatusOr<CopyFuture> CopyExtents(Direction dir,
                                   const std::vector<StorageView>& storages,
                                   const std::vector<ByteExtent>& extents,
                                   hipStream_t dep);

  // Device-only gather/scatter between the storages and a caller buffer
  // laid out layer-major [storage][n][block] (block_major=false) or
  // block-major [n][storage][block]. Runs on `stream`.
  StatusOr<CopyFuture> DeviceCopy(bool gather,
                                  const std::vector<StorageView>& storages,
                                  const std::vector<int64_t>& ids,
                                  uint64_t staging, bool block_major,
                                  hipStream_t stream);

  int device() const { return opts_.device; }
  // The occupancy cap the engine's device gathers launch with.
  int gather_workgroups_per_cu() const { return opts_.gather_workgroups_per_cu; }
  EngineStats stats() const;
  // How the four streams landed on hardware queues at creation (probed: a
  // set with two streams on one queue is created again, up to 3 times).
  StreamPlacement placement() const { return placement_; }
  // SDMA engine bits of the pageable lanes' DMAs, (device-to-host << 16) |
  // host-to-device; 0 while no lane exists or when the lanes use
  // hipMemcpyAsync.
  uint32_t LaneDmaEngines();
  // Blocks until both pageable lanes have drained and everything enqueued on
  // the engine's streams has finished.
  Status Synchronize();
  // Sums the profiled launches of gather (or scatter) kernels recorded so
  // far; waits for them to finish. `reset` drops the samples.
  StatusOr<KernelTimes> ProfiledKernelTimes(bool gather, bool reset);

 private:
  struct Group {
    int64_t block_bytes = 0;
    int64_t pool_blocks = 0;
    std::vector<int> members;  // indices into the storages vector
    uint64_t table_dev = 0;    // device address of the base-address table
  };
  struct Ring {
    std::vector<uint64_t> bufs;
    std::vector<hipEvent_t> ready;
    std::vector<hipEvent_t> free;
    std::vector<bool> used;
    size_t next = 0;
  };
  struct ArgSlice {
    int64_t begin = 0;
    int64_t end = 0;
    hipEvent_t done = nullptr;
  };
  struct Bounce;        // pinned bounce buffers + host copier of one lane
  struct PageableLane;  // per direction: worker thread, streams, rings
  // Where a staged copy runs: the engine's own streams and ring (args ==
  // nullptr: the engine's argument ring, mu_ held; bounce == nullptr: the
  // host regions are pinned) or a pageable lane's.
  struct LaneView {
    hipStream_t ks = nullptr;
    hipStream_t cs = nullptr;
    Ring* ring = nullptr;
    ArgRing* args = nullptr;
    Bounce* bounce = nullptr;
  };

  explicit TransferEngine(const EngineOptions& opts);
  Status Init();
  // Reserves `bytes` of the pinned/device argument ring; waits on the host
  // only if the region is still read by an earlier, unfinished copy.
  StatusOr<int64_t> ArgAlloc(int64_t bytes);
  Status ArgCommit(int64_t begin, int64_t end, hipStream_t stream);
  Status GrowArgRing(int64_t bytes);
  static std::vector<Group> MakeGroups(const std::vector<StorageView>& s);
  Status WaitDep(hipStream_t dep, hipStream_t on);
  StatusOr<CopyFuture> CopyDirect(Direction dir,
                                  const std::vector<StorageView>& storages,
                                  const std::vector<int64_t>& src,
                                  const std::vector<int64_t>& dst,
                                  const std::vector<int64_t>& sizes,
                                  hipStream_t dep);
  // cdev / chost: compact (device id, host id) pairs from PlanPairs.
  StatusOr<CopyFuture> CopyStaged(Direction dir,
                                  const std::vector<StorageView>& storages,
                                  const std::vector<int64_t>& cdev,
                                  const std::vector<int64_t>& chost,
                                  hipStream_t dep);
  // The staged pipeline on `lane`; *done receives the completion event, or
  // nullptr for a D2H through bounce buffers, which completes when its last
  // bounce slot drains (the lane then fulfils its future).
  Status StagedOnLane(const LaneView& lane, Direction dir,
                      const std::vector<StorageView>& storages,
                      const std::vector<int64_t>& cdev, const std::vector<int64_t>& chost,
                      hipStream_t dep, hipEvent_t* done);
  // One staging chunk of a pipelined copy: its bytes in the chunk buffer,
  // the host side as segments, the device side as a kernel between the
  // storages and the chunk buffer (its address is the argument).
  struct HostSegment {
    uint8_t* host;
    int64_t off;  // in the chunk buffer
    int64_t bytes;
  };
  struct ChunkWork {
    int64_t bytes = 0;
    std::vector<HostSegment> segs;
    std::function<Status(uint64_t)> kernel;
  };
  // Runs `chunks` through the lane's staging ring (and bounce buffers). A D2H
  // through bounce buffers returns with its last slots still owed to host
  // memory; they drain when their slot comes round again or the lane idles.
  Status PipelineChunks(const LaneView& lane, Direction dir, const std::vector<ChunkWork>& chunks,
                        int64_t* memcpys);
  // PipelineChunks of a bounce lane whose DMAs run on fixed SDMA engines.
  Status PipelineBounceSdma(const LaneView& lane, Direction dir,
                            const std::vector<ChunkWork>& chunks, int64_t* memcpys);
  // Pool extents through a pageable lane (*done as StagedOnLane).
  Status ExtentsOnLane(const LaneView& lane, Direction dir,
                       const std::vector<StorageView>& storages,
                       const std::vector<ByteExtent>& extents, hipEvent_t* done);
  // Queues a block copy (cdev/chost) or a pool-extent copy (extents) on the
  // pageable lane of `dir`.
  StatusOr<CopyFuture> CopyPageable(Direction dir, const std::vector<StorageView>& storages,
                                    const std::vector<int64_t>& cdev,
                                    const std::vector<int64_t>& chost,
                                    const std::vector<ByteExtent>& extents, hipStream_t dep);
  StatusOr<PageableLane*> Lane(Direction dir);
  void LaneLoop(PageableLane* lane);
  StatusOr<CopyFuture> CopyZeroCopy(Direction dir,
                                    const std::vector<StorageView>& storages,
                                    const std::vector<int64_t>& cdev,
                                    const std::vector<int64_t>& chost,
                                    hipStream_t dep);
  // Expands runs to (device id, host id) pairs, keeps the last pair naming
  // each destination block and orders them by host id.
  static Status PlanPairs(Direction dir, const std::vector<int64_t>& src,
                          const std::vector<int64_t>& dst,
                          const std::vector<int64_t>& sizes,
                          std::vector<int64_t>* dev_ids,
                          std::vector<int64_t>* host_ids);
  StatusOr<hipEvent_t> NewEvent();
  Status EnsureRing(Ring* r);
  // Launches one block-copy kernel, bracketed by timing events when
  // profiling is on.
  Status LaunchCopy(const CopyLaunch& l, bool gather, int vec,
                    hipStream_t stream);

  struct KernelSample {
    hipEvent_t start = nullptr;
    hipEvent_t stop = nullptr;
    int64_t bytes = 0;
    bool gather = true;
  };

  EngineOptions opts_;
  std::vector<KernelSample> samples_;
  std::mutex mu_;
  hipStream_t gather_stream_ = nullptr;   // D2H: kernels
  hipStream_t d2h_stream_ = nullptr;      // D2H: DMA
  hipStream_t h2d_stream_ = nullptr;      // H2D: DMA
  hipStream_t scatter_stream_ = nullptr;  // H2D: kernels
  StreamPlacement placement_;
  Ring out_ring_;
  Ring in_ring_;
  uint8_t* arg_host_ = nullptr;
  uint64_t arg_dev_ = 0;
  int64_t arg_bytes_ = 0;
  int64_t arg_head_ = 0;
  std::deque<ArgSlice> arg_inflight_;
  std::unique_ptr<ArgRing> extent_args_;  // strided tables of CopyExtents
  std::mutex lanes_mu_;
  std::unique_ptr<PageableLane> lanes_[2];  // by Direction
  // Engines of the lanes' DMAs (null: hipMemcpyAsync), chosen with the
  // first lane; destroyed after the lanes.
  std::unique_ptr<SdmaEngines> sdma_;
  bool sdma_tried_ = false;
  EngineStats stats_;
  // Stream-ordered staged copies still in flight, per direction (under
  // mu_): an event recorded after each copy and the chunks it enqueued.
  struct StagedInFlight {
    hipEvent_t done;
    int64_t chunks;
  };
  std::deque<StagedInFlight> staged_inflight_[2];  // by Direction
  std::vector<hipEvent_t> spare_events_;           // finished ones, for reuse
  // Chunks of the direction's staged copies not yet finished (drops the
  // finished ones). Needs mu_.
  int64_t StagedChunksInFlightLocked(Direction dir);
  // Auto mode's view of both directions (under duplex_mu_): the futures of
  // its recent copies per direction, finished ones dropped from the front,
  // and when a copy last found the other direction in flight.
  std::mutex duplex_mu_;
  std::deque<CopyFuture> recent_[2];  // by Direction
  int64_t last_duplex_us_ = INT64_MIN / 2;
  // Copy() after auto mode's duplex check: picks the path and issues.
  StatusOr<CopyFuture> CopyPath(Direction dir, const std::vector<StorageView>& storages,
                                const std::vector<int64_t>& src,
                                const std::vector<int64_t>& dst,
                                const std::vector<int64_t>& sizes, hipStream_t dep,
                                bool duplex);
  // Whether a copy of `dir` issued now takes the duplex path (and records
  // an overlap when the other direction is in flight).
  bool DuplexNow(Direction dir);
  // Remembers an issued auto-mode copy of `dir`.
  void NoteIssued(Direction dir, const CopyFuture& f);
};

}  // namespace kvx

#endif  // KVX_HOST_TRANSFER_ENGINE_H_
