// Host-side interface of the tiled-layout copy kernel (gfx950).
//
// A tiled layout stores a tensor the way XLA's tiled layouts do (the layouts
// the reference's TileBuffer / DetileBuffer convert,
// tpu_sync/weight_sync/tiling_utils.h:27-36): the logical dimensions are put
// in physical (major-to-minor) order, then each tile in turn splits the
// minor-most dimensions into (outer = ceil(d / t), inner = t) and the result
// is stored row-major; positions past a dimension's end are padding.
//
// "Detile" copies a tiled buffer into the row-major (linear) byte image of
// the tensor, "tile" the reverse. One launch runs any number of jobs; a job
// is a range of one tensor in one of five modes:
//   * kDetileStd / kTileStd: the standard form (row-major dimension order and
//     one 2-D tile (tH, tW), optionally followed by a (P, 1) tile that packs
//     P consecutive rows element by element, P in {2, 4} with P * itemsize =
//     4). A unit is P rows x V bytes: V contiguous bytes of each of P linear
//     rows and P * V contiguous bytes of the tiled buffer.
//   * kDetileGen / kTileGen: any other layout, element by element through the
//     index map of the nested tiling.
//   * kZero: clears a tiled buffer (V-byte vectors), launched before a tile
//     job writes its data so that padding reads as zero.
#ifndef KVX_KERNELS_TILED_COPY_H_
#define KVX_KERNELS_TILED_COPY_H_

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <vector>

namespace kvx {

// Division of a 32-bit unsigned n by a fixed d >= 1 with a multiply-high:
// q = (umulhi(n, m) + n) >> s, with s = ceil(log2 d) and
// m = floor(2^32 (2^s - d) / d) + 1 (Granlund and Montgomery, "Division by
// invariant integers using multiplication", PLDI 1994). Exact for every
// n < 2^32 and 1 <= d <= 2^31.
struct FastDivU32 {
  uint32_t d;
  uint32_t m;
  uint32_t s;
  uint32_t pad;
};

inline FastDivU32 MakeFastDivU32(uint32_t d) {
  FastDivU32 f{};
  f.d = d;
  uint32_t s = 0;
  while ((uint64_t{1} << s) < d) ++s;
  f.s = s;
  f.m = static_cast<uint32_t>(((uint64_t{1} << 32) * ((uint64_t{1} << s) - d)) / d + 1);
  return f;
}

// Host twin of the device division (same arithmetic), for checks.
inline uint32_t FastDivHost(const FastDivU32& f, uint32_t n) {
  const uint64_t hi = (static_cast<uint64_t>(n) * f.m) >> 32;
  return static_cast<uint32_t>((hi + n) >> f.s);
}

enum TiledMode : uint32_t {
  kDetileStd = 0,
  kTileStd = 1,
  kZero = 2,
  kDetileGen = 3,
  kTileGen = 4,
};

constexpr int kTiledMaxRank = 8;     // logical dimensions (general path)
constexpr int kTiledMaxGenDims = 16; // dimensions of the final tiled shape
constexpr int kTiledMaxOps = 4;      // tiles applied to one dimension

// One dimension of the final tiled shape (general path): its index is the
// index of logical dimension `src` (0 if src < 0, a padded leading 1) passed
// through `nops` divisions or modulos (bit k of is_mod) in order; it
// contributes index * stride elements to the physical position.
struct TiledGenDim {
  int32_t src;
  uint32_t nops;
  uint32_t is_mod;
  uint32_t pad;
  FastDivU32 op[kTiledMaxOps];
  uint64_t stride;
  uint64_t pad2;
};
static_assert(sizeof(TiledGenDim) == 96, "device layout");

// One job of a launch (built on the host, read with scalar loads).
struct TiledJobDev {
  uint64_t tiled;   // tiled buffer of the tensor
  uint64_t linear;  // linear image of the tensor (byte 0 = element 0)
  uint64_t lo;      // first unit (std), element (gen) or vector (zero)
  uint64_t count;   // units / elements / vectors
  uint32_t mode;    // TiledMode
  uint32_t wg_begin;
  uint32_t P;        // std: rows per unit (1, 2 or 4)
  uint32_t itemsize; // bytes per element
  // Standard form: unit u = ((b * NG + g) * NCV + cv).
  FastDivU32 ncv;  // column vectors per row
  FastDivU32 ng;   // row groups per batch matrix = ceil(H / P)
  FastDivU32 th;   // tile rows
  FastDivU32 tw;   // tile columns
  uint64_t H;
  uint64_t W;
  uint64_t nT0;  // tile rows per matrix = ceil(H / tH)
  uint64_t nT1;  // tile columns per matrix = ceil(W / tW)
  // General form.
  uint32_t rank;        // logical dimensions
  uint32_t ngen;        // dimensions of the final tiled shape
  uint32_t gen_offset;  // byte offset of this job's TiledGenDim array in the image
  uint32_t pad;
  FastDivU32 dims[kTiledMaxRank];  // logical dimensions (row-major)
};
static_assert(sizeof(TiledJobDev) % 16 == 0, "device layout");

// Units (std), elements (gen) or vectors (zero) one workgroup moves.
uint32_t TiledJobPerWorkgroup(const TiledJobDev& j);

// Launches the jobs of a device-resident image: `n` TiledJobDev, then the
// general-path dimension arrays, then a workgroup -> job map of `grid`
// uint32 at byte offset `map_offset`. Every standard and zero job of one
// launch uses vector width `vec_bytes` (16, 8, 4, 2 or 1; P > 1 needs >= 4).
hipError_t LaunchTiledCopy(const void* image_dev, uint32_t n, uint32_t map_offset,
                           uint32_t grid, int vec_bytes, hipStream_t stream);

}  // namespace kvx

#endif  // KVX_KERNELS_TILED_COPY_H_
