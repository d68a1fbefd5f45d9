// Tiled tensor layouts on one GPU: the reference's GetTiledBufferElements /
// TileBuffer / DetileBuffer (tpu_sync/weight_sync/tiling_utils.h:27-36,
// tiling_utils.cc:545-1036) as device jobs of the tiled-copy kernel.
//
// A layout is an XLA-style tiled layout written out as plain numbers:
// logical dimensions (row-major), their minor-to-major order, and up to four
// tiles applied in turn. TiledPlan checks a layout once and precomputes what
// the kernel needs; AppendTiledJobs turns a byte range of the tensor's
// linear image into jobs; LaunchTiledThroughRing uploads and launches them.
//
// Two forms, split where the reference splits (IsStandardRowMajorTiled,
// tiling_utils.cc:56-82):
//   * standard: row-major dimension order and one 2-D tile (tH, tW), or that
//     tile followed by a (P, 1) tile with P in {2, 4}, tH % P == 0 and
//     P * itemsize == 4 (16-bit elements packed in pairs, 8-bit in fours):
//     vectorised units of P rows;
//   * general: every other tiled layout, element by element through the
//     nested-tiling index map. The reference's specialised routine assumes
//     16-bit elements for P = 2 and 8-bit for P = 4 whatever the element type
//     is; here such layouts follow the general nested-tiling definition.
// A layout without tiles is a plain copy of its bytes (the reference
// memcpy's it whatever its dimension order, tiling_utils.cc:959-964).
#ifndef KVX_HOST_TILED_LAYOUT_H_
#define KVX_HOST_TILED_LAYOUT_H_

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <vector>

#include "../kernels/tiled_copy.h"
#include "arg_ring.h"
#include "status.h"

namespace kvx {

struct TiledLayout {
  int itemsize = 1;                       // 1, 2, 4 or 8 bytes
  std::vector<int64_t> dims;              // logical dimensions, row-major
  std::vector<int> minor_to_major;        // permutation of [0, rank)
  std::vector<std::vector<int64_t>> tiles;  // applied in order
};

// Checks ranks, sizes and the permutation; tile dimensions must be >= 1
// (XLA's combined-dimension marker is not supported).
Status ValidateTiledLayout(const TiledLayout& l);

// GetTiledBufferElements (tiling_utils.cc:905-957): elements of the tiled
// buffer, padding included. 1 for a rank-0 tensor.
StatusOr<int64_t> TiledBufferElements(const TiledLayout& l);
int64_t LogicalElements(const TiledLayout& l);

struct TiledPlan {
  TiledLayout layout;
  bool tiled = false;     // has tiles (else a plain copy)
  bool standard = false;  // standard form (else general)
  bool padded = false;    // tiled elements > logical elements
  int64_t logical_bytes = 0;
  int64_t tiled_bytes = 0;
  int vec = 16;       // widest vector the layout allows (standard form)
  int zero_vec = 16;  // vector width of the zero pass
  // Standard form: batch matrices [B][H][W], tiles (tH, tW), P rows per unit.
  uint32_t P = 1;
  uint64_t B = 1, H = 1, W = 1, tH = 1, tW = 1, nT0 = 1, nT1 = 1;
  // General form: the final tiled shape's dimensions.
  std::vector<TiledGenDim> gen;
  // Largest byte offset <= x (from the start of the linear image) at which
  // the linear image may be cut between two launches: whole tile rows (tH
  // rows, or the end of a batch matrix) in the standard form, whole elements
  // in the general form.
  int64_t CutAtOrBelow(int64_t x) const;
};

StatusOr<TiledPlan> PlanTiled(const TiledLayout& l);

// One job with the vector width its launch must use (0: any).
struct TiledJob {
  TiledJobDev dev{};
  int vec = 0;
  std::vector<TiledGenDim> gen;
};

// Jobs moving bytes [lo, hi) of the tensor's linear image (cut points from
// CutAtOrBelow, or 0 / logical_bytes) between its tiled buffer `tiled` and
// a linear image whose byte 0 is at `linear` (only [lo, hi) of it is
// touched). tile = true: linear -> tiled. Standard-form tiling writes the
// padding of the tile rows it covers; otherwise, with zero_pass, the whole
// tiled buffer is first cleared when the layout has padding (the caller
// passes zero_pass for the range that starts the tensor, and launches *zero
// before *jobs).
// Untiled layouts yield no jobs (callers copy their bytes).
Status AppendTiledJobs(const TiledPlan& p, uint64_t tiled, uint64_t linear, int64_t lo,
                       int64_t hi, bool tile, bool zero_pass, std::vector<TiledJob>* zero,
                       std::vector<TiledJob>* jobs);

// Uploads `jobs` through `ring` and launches them on `stream`, one launch
// per vector width; a non-null kernel_start is recorded before the first.
Status LaunchTiledThroughRing(ArgRing& ring, const std::vector<TiledJob>& jobs,
                              hipStream_t stream, hipEvent_t kernel_start = nullptr);

}  // namespace kvx

#endif  // KVX_HOST_TILED_LAYOUT_H_
