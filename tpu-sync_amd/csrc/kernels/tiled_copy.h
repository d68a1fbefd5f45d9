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
//     rows and P * V contiguous bytes of the tiled buffer, moved by one lane
//     or, for P = 2 at V = 16, by two lanes that exchange halves. Units are
//     enumerated in linear order (row groups of the linear image, then column
//     vectors) or in tiled order (unit u is bytes [u P V, (u + 1) P V) of the
//     tiled buffer, padding included: rows past H and columns past W read as
//     zero when tiling and are skipped when detiling).
//   * kDetileGen / kTileGen: any other layout, element by element through the
//     index map of the nested tiling.
//   * kZero: clears a tiled buffer (V-byte vectors), launched before a
//     general-form tile job writes its data so that padding reads as zero
//     (standard-form tiling writes its padding itself).
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
  // Tiled order: u = ((T * GT + gi) * NCVT + cvt), T = (b * nT0 + tr) * nT1 + tc.
  FastDivU32 t_ncv;  // column vectors per tile row group (NCVT = tW * itemsize / V)
  FastDivU32 t_gpt;  // row groups per tile (GT = tH / P)
  FastDivU32 t_nt1;  // tile columns per matrix (nT1)
  FastDivU32 t_nt0;  // tile rows per matrix (nT0)
  uint32_t torder;   // 0: linear order, 1: tiled order
  uint32_t lanes_per_unit;  // packed units: 1, or 2 (P = 2) / 4 (P = 4) detiling at 16-byte rows
  uint32_t sliced;  // detiling with 2 or 4 lanes per unit: slots in whole groups go sliced
  uint32_t pad0;
  uint32_t h32;         // H (rows per batch matrix)
  uint32_t w32;         // W (columns)
  uint32_t nt0;         // tile rows per matrix = ceil(H / tH)
  uint32_t nt1;         // tile columns per matrix = ceil(W / tW)
  uint32_t tile_elems;  // tH * tW
  uint32_t log2s;       // log2(itemsize)
  uint32_t pad1[2];
  // General form.
  uint32_t rank;        // logical dimensions
  uint32_t ngen;        // dimensions of the final tiled shape
  uint32_t gen_offset;  // byte offset of this job's TiledGenDim array in the image
  uint32_t pad;
  FastDivU32 dims[kTiledMaxRank];  // logical dimensions (row-major)
};
static_assert(sizeof(TiledJobDev) % 16 == 0, "device layout");

// What selects a kernel: every job of one launch shares it.
struct TiledLaunchKey {
  uint32_t mode;
  uint32_t vec;       // standard and zero jobs: vector width
  uint32_t P;         // standard jobs
  uint32_t torder;    // standard jobs
  uint32_t lanes;     // standard packed jobs: lanes per unit
  uint32_t itemsize;  // general jobs
  bool operator==(const TiledLaunchKey& o) const {
    return mode == o.mode && vec == o.vec && P == o.P && torder == o.torder &&
           lanes == o.lanes && itemsize == o.itemsize;
  }
};

// The key of a job whose launch uses vector width vec_bytes.
TiledLaunchKey LaunchKeyOf(const TiledJobDev& j, int vec_bytes);

// Units (std), elements (gen) or vectors (zero) one workgroup moves.
uint32_t TiledPerWorkgroup(const TiledLaunchKey& k);

// Launches the jobs of a device-resident image: the TiledJobDev array, the
// general-path dimension arrays, then a workgroup -> job map of `grid`
// uint32 at byte offset `map_offset`. Every job of the image has `key`.
hipError_t LaunchTiledCopy(const void* image_dev, uint32_t map_offset, uint32_t grid,
                           const TiledLaunchKey& key, hipStream_t stream);

}  // namespace kvx

#endif  // KVX_KERNELS_TILED_COPY_H_
