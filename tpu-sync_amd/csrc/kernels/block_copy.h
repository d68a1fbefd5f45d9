// Host-side interface of the paged-KV block copy kernels (gfx950).
//
// A "storage" is one device buffer laid out as [pool_blocks][block_bytes]
// (one K or V buffer of one layer and shard). A copy job moves the blocks
// ids[0..n) of W storages to or from a staging buffer. The flat index of
// block (w, i) is f = w * n + i. A launch covers up to kMaxPieces pieces;
// a piece is a run of flat indices over storages that share one block size,
// so one launch can move a KV payload together with a side table of a
// different block size (fp8 scales).
//
// The byte identity these kernels implement is the one of the reference's
// per-run raw DMA (tpu_sync/kv_cache/kv_cache_manager_base.cc:2035-2124,
// tpu_sync/core/raw_transfer_core.h:638-692): block id * block bytes within a
// storage, whole blocks, bytes copied opaquely.
#ifndef KVX_KERNELS_BLOCK_COPY_H_
#define KVX_KERNELS_BLOCK_COPY_H_

#include <hip/hip_runtime_api.h>

#include <cstdint>

namespace kvx {

constexpr int kMaxPieces = 4;
constexpr int kDefaultGatherWorkgroupsPerCu = 2;

struct CopyPiece {
  // Device address of a table of uint64 storage base addresses, indexed by w.
  uint64_t storages = 0;
  // Address of block (w, i) on the other side of the copy. When `others` is
  // 0 it is staging + w * stride_w + i * stride_i (a contiguous staging
  // buffer), computed in wrapping uint64 arithmetic, so a piece that starts
  // at f0 > 0 may pass a base that lies before its buffer. Otherwise it is
  // others[w] + ids2[i] * block_bytes: a second paged buffer (for example the
  // pinned host mirror, read and written by the kernel over PCIe).
  uint64_t staging = 0;
  uint64_t others = 0;
  int64_t stride_w = 0;
  int64_t stride_i = 0;
  int64_t f0 = 0;          // first flat block of the piece
  int64_t nblocks = 0;     // flat blocks in the piece
  int64_t block_bytes = 0; // bytes per block of every storage in the piece
  int64_t pool_blocks = 0; // valid block ids are [0, pool_blocks)
  int64_t other_blocks = 0; // valid ids2 are [0, other_blocks) when others != 0
};

struct CopyLaunch {
  CopyPiece pieces[kMaxPieces];
  int npieces = 0;
  const int64_t* ids = nullptr;   // device array of n block ids
  const int64_t* ids2 = nullptr;  // block ids on the `others` side (if used)
  int64_t n = 0;
  int32_t* error = nullptr;      // optional device word; set to 1 on a bad id
  // 0: one workgroup per large block (best for HBM-bound copies). Otherwise
  // at most about this many workgroups: each then moves a run of
  // consecutive blocks, which leaves CUs free for other work (a PCIe-bound
  // zero-copy kernel needs only a few hundred workgroups in flight).
  int64_t max_workgroups = 0;
  // Gathers (other than capped zero-copy grids) reserve LDS so that at most
  // this many of their workgroups share a CU (0: no limit). Fewer random
  // reads in flight per CU let the DRAM serve them more efficiently: 2
  // measured 74.5 -> 76.0 % of HBM peak for 512 x 64 blocks of 32 KiB (1 and
  // 3 the same, 4 and 6 no gain) and 67.2 -> 69.9 % for fp8 payload (16 KiB)
  // + scales; the scatter gains nothing. The LDS is not used, but while such
  // a gather runs it keeps LDS-hungry kernels of other streams off its CUs;
  // 0 leaves every CU's LDS to them.
  int32_t gather_workgroups_per_cu = kDefaultGatherWorkgroupsPerCu;
};

// kGather reads the `storages` side and writes the other side; kScatter the
// reverse.
enum class CopyDir : int { kGather = 0, kScatter = 1 };

// Largest vector width (16, 4 or 1 bytes) that every address of the launch
// is aligned to. `extra_align` folds in addresses the caller knows about.
int LaunchVectorBytes(const CopyLaunch& l, uint64_t extra_align);

// Enqueues the copy on `stream`. Returns hipErrorInvalidValue when the launch
// violates the kernel's index limits (checked here, before any launch).
hipError_t LaunchBlockCopy(const CopyLaunch& l, CopyDir dir, int vec_bytes,
                           hipStream_t stream);

// Workgroups a launch uses (for tests and profiling).
int64_t BlockCopyWorkgroups(const CopyLaunch& l, int vec_bytes);

}  // namespace kvx

#endif  // KVX_KERNELS_BLOCK_COPY_H_
