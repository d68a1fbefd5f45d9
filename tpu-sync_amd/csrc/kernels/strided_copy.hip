// Strided-entry copy for gfx950 (MI355X): per-tensor offset-table pack /
// unpack and column splits of row-major weights, any number of entries per
// launch.
//
// Pure data movement, bound by HBM bandwidth. Work is cut into tiles of
// kTileVecs vectors (32 KiB at 16-byte vectors); a workgroup of 256 lanes
// moves one tile with kUnroll independent loads in flight per lane before
// its stores, the pattern that keeps HBM busy. A tile is either a run of
// whole rows of one entry (short rows, e.g. the 1-3.5 KiB row chunks of a
// column split) or a slice of one long row (a whole tensor is one row).
// The tile -> entry map and the entry table are read with workgroup-uniform
// scalar loads; lanes find their row with a multiply-shift instead of a
// division. Loads and stores are non-temporal (every byte is touched once).
//
// At 16-byte vectors with one workgroup per tile, tiles go sliced: in a
// group of 32 consecutive tiles (of one long row, or of one entry's runs of
// short rows) the workgroup holding tile j moves the j-th 1 KiB of each of
// the group's tiles instead of one contiguous tile. Long-row tiles are
// numbered first and taken in plain workgroup order, short-row tiles after
// them in XCD order. Measured on MI355X in one process against contiguous
// tiles in XCD order: a 1 GiB copy 77.6 -> 83.3 % of HBM peak, a 16 GiB copy
// 80.6 -> 84.4 %, the 291-tensor Llama-3-8B pack 80.4 -> 84.9 %, its 8-way
// column split 78.4 -> 80.9 %. (Plain order cost the column split 12 points
// with contiguous tiles and gained it nothing sliced.)
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "strided_copy.h"

namespace kvx {
namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 8;
constexpr uint32_t kTileVecs = kThreads * kUnroll;
// MI355X has 8 XCDs; consecutive workgroups are dispatched round-robin over
// them.
constexpr uint32_t kXcds = 8;
// LDS of one CU on gfx950.
constexpr uint32_t kLdsPerCu = 160u << 10;
// A launch with one workgroup per tile reserves LDS it does not use, so that
// at most this many of its workgroups share a CU: fewer streams of reads and
// writes per CU keep the DRAM closer to sequential. The 16 GB pack of 291
// tensors measured 73.3 -> 79.7 % of HBM peak and the 8-way column split
// 71.0 -> 78.3 % (3 the same; 1 and 4 lower; 16 or 4 loads per lane instead
// of 8 lower at 2). While such a launch runs, its CUs' LDS is taken.
constexpr uint32_t kWorkgroupsPerCu = 2;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define KVX_GLOBAL __attribute__((address_space(1)))
#define KVX_CONST __attribute__((address_space(4)))

struct KArgs {
  const StridedEntryDev* table;
  const uint32_t* tile_entry;  // tile -> entry index
  uint32_t tiles;
  uint32_t sliced;        // tiles in whole groups of kSliceTiles go sliced
  uint32_t sliced_tiles;  // tiles [0, sliced_tiles): long rows, in plain order
};

// Tiles taken as groups of kSliceTiles: the workgroup that holds tile j of a
// group moves the j-th wave-sized slice (64 vectors) of every tile of the
// group, so each workgroup's bytes are 32 pieces spread over the group (1 MiB
// of a long row at 16-byte vectors) instead of one contiguous tile.
constexpr uint32_t kSliceVecs = 64;
constexpr uint32_t kSliceTiles = kTileVecs / kSliceVecs;
static_assert(kSliceTiles == kUnroll * (kThreads / 64), "one slice per wave and step");

template <typename V>
__device__ __forceinline__ void copy_sliced(uint64_t src, uint64_t dst, uint32_t vecs,
                                            uint32_t ct) {
  const uint32_t j = ct & (kSliceTiles - 1);
  const uint64_t first = static_cast<uint64_t>(ct - j) * kTileVecs + j * kSliceVecs;
  const uint32_t wave = threadIdx.x / 64;
  const uint32_t lane = threadIdx.x % 64;
  V r[kUnroll];
  uint64_t vi[kUnroll];
  // As in copy_tile: every load goes out (lanes past the row re-read its
  // last vector); only the stores are predicated.
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const uint32_t c = u * (kThreads / 64) + wave;  // tile of the group
    vi[u] = first + static_cast<uint64_t>(c) * kTileVecs + lane;
    const uint64_t vl = vi[u] < vecs ? vi[u] : vecs - 1;
    r[u] = __builtin_nontemporal_load((const KVX_GLOBAL V*)(src + vl * sizeof(V)));
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    if (vi[u] < vecs) {
      __builtin_nontemporal_store(r[u], (KVX_GLOBAL V*)(dst + vi[u] * sizeof(V)));
    }
  }
}

// Slice j of each tile of the group of kSliceTiles tiles from tile tb of an
// entry of short rows (rows_per_tile rows per tile; only the entry's last
// tile may hold fewer).
template <typename V>
__device__ __forceinline__ void copy_sliced_rows(const KVX_CONST StridedEntryDev& ent,
                                                 uint32_t tb, uint32_t j) {
  const uint32_t wave = threadIdx.x / 64;
  const uint32_t lane = threadIdx.x % 64;
  const uint32_t rpt = ent.rows_per_tile;
  const uint32_t vecs = ent.vecs;
  const uint64_t magic = ent.div_magic;
  V r[kUnroll];
  uint64_t doff[kUnroll];
  bool valid[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const uint32_t c = u * (kThreads / 64) + wave;  // tile of the group
    const uint32_t row0 = (tb + c) * rpt;
    const uint32_t left = ent.count - row0;
    const uint32_t total = (left < rpt ? left : rpt) * vecs;
    const uint32_t k = j * kSliceVecs + lane;
    valid[u] = k < total;
    // Lanes past the tile re-read its last vector; only stores are predicated.
    const uint32_t kk = valid[u] ? k : total - 1;
    const uint32_t row = static_cast<uint32_t>((kk * magic) >> 32);
    const uint64_t r_abs = row0 + row;
    const uint64_t col = static_cast<uint64_t>(kk - row * vecs) * sizeof(V);
    r[u] = __builtin_nontemporal_load(
        (const KVX_GLOBAL V*)(ent.src + r_abs * ent.src_stride + col));
    doff[u] = r_abs * ent.dst_stride + col;
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    if (valid[u]) __builtin_nontemporal_store(r[u], (KVX_GLOBAL V*)(ent.dst + doff[u]));
  }
}

// Moves tile `wg` (one entry's rows, or one slice of a long row).
template <typename V>
__device__ __forceinline__ void copy_tile(const KArgs& a, uint32_t wg) {
  const uint32_t e = ((const KVX_CONST uint32_t*)a.tile_entry)[wg];
  const KVX_CONST StridedEntryDev* ent = (const KVX_CONST StridedEntryDev*)a.table + e;
  const uint64_t src = ent->src;
  const uint64_t dst = ent->dst;
  const uint64_t sstride = ent->src_stride;
  const uint64_t dstride = ent->dst_stride;
  const uint32_t vecs = ent->vecs;
  const uint32_t t = wg - ent->tile_begin;
  if (a.sliced && ent->rows_per_tile == 0) {
    const uint32_t tpr = ent->tiles_per_row;
    const uint32_t row = t / tpr;
    const uint32_t ct = t - row * tpr;
    // Tiles in whole groups go sliced; a row's last tiles (fewer than a
    // group) stay contiguous.
    if (ct < (tpr & ~(kSliceTiles - 1))) {
      copy_sliced<V>(src + row * sstride, dst + row * dstride, vecs, ct);
      return;
    }
  } else if (a.sliced) {
    const uint32_t rpt = ent->rows_per_tile;
    const uint32_t ntiles = (ent->count + rpt - 1) / rpt;
    const uint32_t tb = t & ~(kSliceTiles - 1);
    // Runs of short rows: tiles in whole groups of the entry go sliced, the
    // entry's last tiles (fewer than a group) contiguous.
    if (tb + kSliceTiles <= ntiles) {
      copy_sliced_rows<V>(*ent, tb, t - tb);
      return;
    }
  }
  uint32_t row0, nrows, v0, nv;
  if (ent->rows_per_tile > 0) {
    const uint32_t rpt = ent->rows_per_tile;
    row0 = t * rpt;
    const uint32_t left = ent->count - row0;
    nrows = left < rpt ? left : rpt;
    v0 = 0;
    nv = vecs;
  } else {
    const uint32_t tpr = ent->tiles_per_row;
    row0 = t / tpr;
    v0 = (t - row0 * tpr) * kTileVecs;
    const uint32_t left = vecs - v0;
    nv = left < kTileVecs ? left : kTileVecs;
    nrows = 1;
  }
  const uint32_t total = nrows * nv;
  const uint32_t last = total - 1;
  const uint64_t magic = ent->div_magic;
  V r[kUnroll];
  uint64_t doff[kUnroll];
  // Every lane issues all kUnroll loads unconditionally (lanes past the end
  // of the tile re-read its last vector), so the loads go out back to back;
  // only the stores are predicated.
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    uint32_t k = threadIdx.x + u * kThreads;
    k = k < total ? k : last;
    // nrows == 1 whenever nv != vecs, so the row is 0 there.
    const uint32_t row = nrows == 1 ? 0u : static_cast<uint32_t>((k * magic) >> 32);
    const uint32_t v = k - row * nv;
    const uint64_t r_abs = row0 + row;
    const uint64_t col = static_cast<uint64_t>(v0 + v) * sizeof(V);
    r[u] = __builtin_nontemporal_load((const KVX_GLOBAL V*)(src + r_abs * sstride + col));
    doff[u] = r_abs * dstride + col;
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    if (threadIdx.x + u * kThreads < total) {
      __builtin_nontemporal_store(r[u], (KVX_GLOBAL V*)(dst + doff[u]));
    }
  }
}

// Workgroup g runs on XCD g % kXcds; it takes tile (g % kXcds) * per +
// g / kXcds, so each XCD streams one contiguous eighth of the tiles and its
// address translations are not repeated on the other seven XCDs (a 16 GiB
// copy: 63.6 % -> 72.8 % of HBM peak). Tiles past kXcds * per map to
// themselves; the map is a bijection on [0, tiles).
__device__ __forceinline__ uint32_t xcd_tile(uint32_t g, uint32_t tiles) {
  const uint32_t per = tiles / kXcds;
  if (g >= per * kXcds) return g;
  return (g % kXcds) * per + g / kXcds;
}

// One tile per workgroup, or (capped grid) tiles blockIdx.x, + gridDim.x, ...
// The loop bound is uniform, so every wave leaves it together. With a full
// grid the sliced tiles go in plain order (a group's workgroups on
// consecutive ids) and the others in XCD order after them.
template <typename V>
__global__ __launch_bounds__(kThreads) void strided_copy_kernel(KArgs a) {
  if (gridDim.x == a.tiles) {
    const uint32_t g = blockIdx.x;
    const uint32_t L = a.sliced_tiles;
    copy_tile<V>(a, g < L ? g : L + xcd_tile(g - L, a.tiles - L));
    return;
  }
  for (uint32_t t = blockIdx.x; t < a.tiles; t += gridDim.x) copy_tile<V>(a, t);
}

}  // namespace

int StridedVectorBytes(const std::vector<StridedCopy>& copies) {
  uint64_t acc = 0;
  for (const StridedCopy& c : copies) {
    acc |= c.src | c.dst | static_cast<uint64_t>(c.size);
    if (c.count > 1) {
      acc |= static_cast<uint64_t>(c.src_stride) | static_cast<uint64_t>(c.dst_stride);
    }
  }
  for (int v : {16, 8, 4, 2}) {
    if ((acc & static_cast<uint64_t>(v - 1)) == 0) return v;
  }
  return 1;
}

bool BuildStridedTable(const std::vector<StridedCopy>& copies, int vec_bytes,
                       std::vector<StridedEntryDev>* table, uint32_t* grid,
                       uint32_t* long_tiles) {
  table->clear();
  uint64_t tiles = 0;
  uint64_t long_end = 0;
  // Entries of long rows (more than one tile) first, then the others; each
  // entry keeps the copies' relative order within its pass.
  for (int pass = 0; pass < 2; ++pass) {
    for (const StridedCopy& c : copies) {
      const int64_t count = c.count > 0 ? c.count : 1;
      if (c.size <= 0 || c.size % vec_bytes != 0 || c.src == 0 || c.dst == 0 ||
          c.src_stride < 0 || c.dst_stride < 0 || count > UINT32_MAX) {
        return false;
      }
      const uint64_t vecs = static_cast<uint64_t>(c.size) / vec_bytes;
      if (vecs > UINT32_MAX) return false;
      const bool long_row = vecs > kTileVecs;
      if (long_row != (pass == 0)) continue;
      StridedEntryDev d{};
      d.src = c.src;
      d.dst = c.dst;
      d.src_stride = static_cast<uint64_t>(c.src_stride);
      d.dst_stride = static_cast<uint64_t>(c.dst_stride);
      d.count = static_cast<uint32_t>(count);
      d.vecs = static_cast<uint32_t>(vecs);
      d.div_magic = (uint64_t{1} << 32) / vecs + 1;
      d.tile_begin = static_cast<uint32_t>(tiles);
      uint64_t t;
      if (!long_row) {
        d.rows_per_tile = static_cast<uint32_t>(kTileVecs / vecs);
        t = (static_cast<uint64_t>(count) + d.rows_per_tile - 1) / d.rows_per_tile;
      } else {
        d.tiles_per_row = static_cast<uint32_t>((vecs + kTileVecs - 1) / kTileVecs);
        t = static_cast<uint64_t>(count) * d.tiles_per_row;
      }
      tiles += t;
      if (tiles > INT32_MAX) return false;
      table->push_back(d);
    }
    if (pass == 0) long_end = tiles;
  }
  *grid = static_cast<uint32_t>(tiles);
  if (long_tiles != nullptr) *long_tiles = static_cast<uint32_t>(long_end);
  return true;
}

hipError_t LaunchStridedCopy(const StridedEntryDev* table_dev, uint32_t n,
                             uint32_t tiles, int vec_bytes, hipStream_t stream,
                             uint32_t max_workgroups, uint32_t long_tiles) {
  if (tiles == 0) return hipSuccess;
  KArgs a;
  a.table = table_dev;
  // The tile -> entry map follows the table in the same device allocation.
  a.tile_entry = reinterpret_cast<const uint32_t*>(table_dev + n);
  a.tiles = tiles;
  const uint32_t grid = max_workgroups > 0 && max_workgroups < tiles ? max_workgroups : tiles;
  // Slicing is measured at 16-byte vectors with one workgroup per tile.
  a.sliced = vec_bytes == 16 && grid == tiles ? 1u : 0u;
  a.sliced_tiles = a.sliced && long_tiles <= tiles ? long_tiles : 0;
  // HBM-bound launches take the occupancy cap; PCIe-bound ones (a capped
  // grid) keep their few workgroups spread without it.
  const uint32_t lds = max_workgroups == 0 ? kLdsPerCu / kWorkgroupsPerCu : 0;
  switch (vec_bytes) {
    case 16:
      hipLaunchKernelGGL(strided_copy_kernel<u32x4>, dim3(grid), dim3(kThreads), lds, stream, a);
      break;
    case 8:
      hipLaunchKernelGGL(strided_copy_kernel<u32x2>, dim3(grid), dim3(kThreads), lds, stream, a);
      break;
    case 4:
      hipLaunchKernelGGL(strided_copy_kernel<uint32_t>, dim3(grid), dim3(kThreads), lds, stream, a);
      break;
    case 2:
      hipLaunchKernelGGL(strided_copy_kernel<uint16_t>, dim3(grid), dim3(kThreads), lds, stream, a);
      break;
    case 1:
      hipLaunchKernelGGL(strided_copy_kernel<uint8_t>, dim3(grid), dim3(kThreads), lds, stream, a);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace kvx
