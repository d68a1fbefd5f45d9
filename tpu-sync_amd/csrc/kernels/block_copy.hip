// Paged-KV block gather/scatter for gfx950 (MI355X).
//
// Pure data movement, bound by HBM bandwidth: no MFMA, no LDS on the data
// itself. Blocks of >= 8 KiB get one 256-lane workgroup each (four wave64s);
// every lane keeps kUnroll independent 16-byte loads in flight before it
// stores, which is what saturates HBM on a streaming copy. The block id and
// the storage base are workgroup-uniform, so the compiler reads them with
// scalar loads into SGPRs: the id table is read once per block, broadcast
// through SGPRs instead of an LDS round trip and barrier. Small blocks (side
// tables such as per-head fp8 scales) are packed many to a workgroup so that
// every lane still moves one vector.
//
// Loads and stores are non-temporal: a gathered block is read once and the
// staging copy is next read by the DMA engine, so neither should displace
// L2/MALL lines.
//
// Bad block ids (outside [0, pool_blocks)) are skipped and reported through
// an optional device flag; no lane ever forms an address from one.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "block_copy.h"

namespace kvx {
namespace {

constexpr int kThreads = 256;
// Blocks per workgroup on the small-block path: the LDS address table holds
// 16 bytes per block (4 KiB, which leaves the occupancy of 8 workgroups per
// CU untouched).
constexpr uint32_t kSmallMaxBlocks = 256;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Explicit address spaces: data goes through global_load/global_store (not
// flat), and workgroup-uniform table reads through the constant address
// space so they become scalar loads.
#define KVX_GLOBAL __attribute__((address_space(1)))
#define KVX_CONST __attribute__((address_space(4)))

template <typename T>
__device__ __forceinline__ KVX_GLOBAL T* gptr(uint64_t addr) {
  return (KVX_GLOBAL T*)addr;
}

template <typename T>
__device__ __forceinline__ T uniform_load(uint64_t table, uint32_t idx) {
  return ((const KVX_CONST T*)table)[idx];
}

struct KPiece {
  uint64_t storages;
  uint64_t staging;
  uint64_t others;
  int64_t stride_w;
  int64_t stride_i;
  int64_t pool_blocks;
  int64_t other_blocks;
  uint32_t f0;
  uint32_t nblocks;
  uint32_t elems;     // vectors per block
  uint32_t bpw;       // blocks per workgroup
  uint32_t wg_begin;  // first workgroup of the piece
  uint32_t whole;     // 1: every lane works on one block at a time
};

struct KParams {
  KPiece p[kMaxPieces];
  const int64_t* ids;
  const int64_t* ids2;
  int32_t* error;
  uint32_t n;
  int32_t npieces;
};

template <typename V>
__device__ __forceinline__ V ld_nt(const KVX_GLOBAL V* p) {
  return __builtin_nontemporal_load(p);
}

template <typename V>
__device__ __forceinline__ void st_nt(V v, KVX_GLOBAL V* p) {
  __builtin_nontemporal_store(v, p);
}

// Whole-block copy by all lanes of the workgroup.
template <typename V, int kUnroll>
__device__ __forceinline__ void copy_whole_block(const KVX_GLOBAL V* __restrict__ src,
                                                 KVX_GLOBAL V* __restrict__ dst,
                                                 uint32_t elems) {
  uint32_t k = threadIdx.x;
  for (; k + (kUnroll - 1) * kThreads < elems; k += kUnroll * kThreads) {
    V r[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) r[u] = ld_nt(src + k + u * kThreads);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) st_nt(r[u], dst + k + u * kThreads);
  }
  // The tail (all of a 16 KiB block) still keeps 4, then 2 loads in flight.
  if (k + 3 * kThreads < elems) {
    V r[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) r[u] = ld_nt(src + k + u * kThreads);
#pragma unroll
    for (int u = 0; u < 4; ++u) st_nt(r[u], dst + k + u * kThreads);
    k += 4 * kThreads;
  }
  if (k + kThreads < elems) {
    const V r0 = ld_nt(src + k);
    const V r1 = ld_nt(src + k + kThreads);
    st_nt(r0, dst + k);
    st_nt(r1, dst + k + kThreads);
    k += 2 * kThreads;
  }
  if (k < elems) st_nt(ld_nt(src + k), dst + k);
}

__device__ __forceinline__ KPiece select_piece(const KParams& P, uint32_t wg) {
  // Pieces are sorted by wg_begin; the choice is workgroup-uniform. Each
  // candidate is copied by a constant index so the kernel argument block is
  // read in place rather than spilled to scratch.
  KPiece p = P.p[0];
  if (P.npieces > 1 && wg >= P.p[1].wg_begin) p = P.p[1];
  if (P.npieces > 2 && wg >= P.p[2].wg_begin) p = P.p[2];
  if (P.npieces > 3 && wg >= P.p[3].wg_begin) p = P.p[3];
  return p;
}

__device__ __forceinline__ bool bad_id(int64_t id, int64_t limit) {
  return static_cast<uint64_t>(id) >= static_cast<uint64_t>(limit);
}

// Many small blocks per workgroup (side tables such as fp8 scales). The
// workgroup first resolves its blocks -- id, table entries, bounds check --
// with one pass of independent, coalesced loads, one block per lane, and
// stages each block's source and destination address in LDS (0 for a bad
// id). Then lane e moves vector (e % elems) of block (e / elems) with both
// addresses read from LDS, so no lane waits on a chain of dependent table
// loads before its data load. b0: the workgroup's first block of the piece.
template <typename V, bool kGather>
__device__ __forceinline__ void copy_small_blocks(const KPiece& p, const int64_t* ids,
                                                  const int64_t* ids2, int32_t* error,
                                                  uint32_t n, uint32_t b0) {
  __shared__ uint64_t s_src[kSmallMaxBlocks];
  __shared__ uint64_t s_dst[kSmallMaxBlocks];
  const uint32_t left = p.nblocks - b0;
  const uint32_t nb = left < p.bpw ? left : p.bpw;
  const uint64_t block_bytes = static_cast<uint64_t>(p.elems) * sizeof(V);
  for (uint32_t b = threadIdx.x; b < nb; b += kThreads) {
    const uint32_t f = p.f0 + b0 + b;
    const uint32_t w = f / n;
    const uint32_t i = f - w * n;
    const int64_t id = gptr<const int64_t>(reinterpret_cast<uint64_t>(ids))[i];
    const uint64_t base = gptr<const uint64_t>(p.storages)[w];
    bool bad = bad_id(id, p.pool_blocks);
    uint64_t other;
    if (p.others != 0) {
      const int64_t id2 = gptr<const int64_t>(reinterpret_cast<uint64_t>(ids2))[i];
      const uint64_t obase = gptr<const uint64_t>(p.others)[w];
      bad = bad || bad_id(id2, p.other_blocks);
      other = obase + static_cast<uint64_t>(id2) * block_bytes;
    } else {
      other = p.staging + w * static_cast<uint64_t>(p.stride_w) +
              i * static_cast<uint64_t>(p.stride_i);
    }
    const uint64_t pool = base + static_cast<uint64_t>(id) * block_bytes;
    if (bad && error != nullptr) atomicOr(error, 1);
    s_src[b] = bad ? 0 : (kGather ? pool : other);
    s_dst[b] = bad ? 0 : (kGather ? other : pool);
  }
  __syncthreads();
  const uint32_t total = nb * p.elems;
  for (uint32_t e = threadIdx.x; e < total; e += kThreads) {
    const uint32_t b = e / p.elems;
    const uint32_t sub = e - b * p.elems;
    const uint64_t src = s_src[b];
    if (src == 0) continue;
    st_nt(ld_nt(gptr<const V>(src) + sub), gptr<V>(s_dst[b]) + sub);
  }
}

template <typename V, bool kGather, int kUnroll>
__global__ __launch_bounds__(kThreads) void block_copy_kernel(KParams P) {
  const uint32_t wg = blockIdx.x;
  const KPiece p = select_piece(P, wg);
  const uint32_t b0 = (wg - p.wg_begin) * p.bpw;
  const uint32_t n = P.n;

  if (p.whole) {
    // All lanes move one block at a time; the workgroup walks a run of
    // consecutive flat blocks (one block unless the grid is capped).
    const uint32_t left = p.nblocks - b0;
    const uint32_t nb = left < p.bpw ? left : p.bpw;
    for (uint32_t b = 0; b < nb; ++b) {
      const uint32_t f = p.f0 + b0 + b;
      const uint32_t w = f / n;
      const uint32_t i = f - w * n;
      const int64_t id = uniform_load<int64_t>(reinterpret_cast<uint64_t>(P.ids), i);
      uint64_t other;
      bool bad = bad_id(id, p.pool_blocks);
      if (p.others != 0) {
        const int64_t id2 = uniform_load<int64_t>(reinterpret_cast<uint64_t>(P.ids2), i);
        bad = bad || bad_id(id2, p.other_blocks);
        other = uniform_load<uint64_t>(p.others, w) +
                static_cast<uint64_t>(id2) * p.elems * sizeof(V);
      } else {
        other = p.staging + w * static_cast<uint64_t>(p.stride_w) +
                i * static_cast<uint64_t>(p.stride_i);
      }
      if (bad) {
        if (threadIdx.x == 0 && P.error != nullptr) atomicOr(P.error, 1);
        continue;
      }
      const uint64_t base = uniform_load<uint64_t>(p.storages, w);
      KVX_GLOBAL V* pool = gptr<V>(base) + static_cast<uint64_t>(id) * p.elems;
      KVX_GLOBAL V* stg = gptr<V>(other);
      if (kGather) {
        copy_whole_block<V, kUnroll>(pool, stg, p.elems);
      } else {
        copy_whole_block<V, kUnroll>(stg, pool, p.elems);
      }
    }
    return;
  }

  copy_small_blocks<V, kGather>(p, P.ids, P.ids2, P.error, n, b0);
}

// The common launch (one piece of large blocks, no second paged side, one
// block per workgroup) without the piece selection: the workgroup reads the
// block id and the storage base with two independent scalar loads and starts
// its vector loads after one wait. Over whole storages the workgroup order
// is chosen by measurement (random ids, 64 storages of 512 MiB):
//   kAllStorages (scatter): consecutive workgroups take the same block index
//     of consecutive storages, so the writes in flight spread over every
//     storage instead of crowding one (+1 to +3 points of HBM bandwidth);
//   kStoragePairs (gather): the same block index of storages 2q and 2q + 1,
//     then the next index (+1.5 points against storage-major order; wider
//     groups measured slower).
struct FastParams {
  uint64_t storages;
  uint64_t staging;
  const int64_t* ids;
  int32_t* error;
  int64_t stride_w;
  int64_t stride_i;
  int64_t pool_blocks;
  uint32_t f0;
  uint32_t n;
  uint32_t elems;
  uint32_t wstorages;  // whole-storage orders: storages in the launch
  uint32_t w0;         // whole-storage orders: first storage (f0 = w0 * n)
  uint32_t pieces;     // workgroups per block (1, or blocks above kUnroll * kThreads vectors)
  uint32_t piece_elems;  // vectors per workgroup when pieces > 1
};

enum FastOrder : int { kStorageMajor = 0, kStoragePairs = 1, kAllStorages = 2 };

// Workgroup g of a fast launch: one whole block, or with pieces > 1 one
// piece of piece_elems vectors of a block, the pieces of a block on
// consecutive workgroups (so a large block's writes are in flight together).
template <typename V, bool kGather, int kUnroll, int kOrder>
__device__ __forceinline__ void fast_block(const FastParams& P, uint32_t g) {
  uint32_t piece = 0;
  if (P.pieces > 1) {
    const uint32_t b = g / P.pieces;
    piece = g - b * P.pieces;
    g = b;
  }
  uint32_t w, i;
  if (kOrder == kAllStorages) {
    i = g / P.wstorages;
    w = P.w0 + (g - i * P.wstorages);
  } else if (kOrder == kStoragePairs) {
    const uint32_t q = g / (2 * P.n);
    const uint32_t r = g - q * 2 * P.n;
    i = r >> 1;
    w = P.w0 + 2 * q + (r & 1);
  } else {
    const uint32_t f = P.f0 + g;
    w = f / P.n;
    i = f - w * P.n;
  }
  // Both table loads go out together (the base first: issued in the other
  // order, the compiler waits for the id before loading the base) and nothing
  // branches on the id before the copy: a workgroup waits for one scalar
  // round trip before its first vector load. A bad id turns the copy into no
  // work. (Measured against the branching form in one process on the same
  // allocations: equal, within 0.3 %.)
  const uint64_t base = uniform_load<uint64_t>(P.storages, w);
  const int64_t id = uniform_load<int64_t>(reinterpret_cast<uint64_t>(P.ids), i);
  const bool bad = bad_id(id, P.pool_blocks);
  const uint32_t first = piece * P.piece_elems;  // 0 unless the block is split
  const uint32_t left = P.elems - first;
  const uint32_t span = P.pieces > 1 && left > P.piece_elems ? P.piece_elems : left;
  const uint32_t elems = bad ? 0u : span;
  KVX_GLOBAL V* pool =
      gptr<V>(base) + static_cast<uint64_t>(bad ? 0 : id) * P.elems + first;
  KVX_GLOBAL V* stg = gptr<V>(P.staging + w * static_cast<uint64_t>(P.stride_w) +
                              i * static_cast<uint64_t>(P.stride_i)) + first;
  if (kGather) {
    copy_whole_block<V, kUnroll>(pool, stg, elems);
  } else {
    copy_whole_block<V, kUnroll>(stg, pool, elems);
  }
  if (bad && threadIdx.x == 0 && P.error != nullptr) atomicOr(P.error, 1);
}

template <typename V, bool kGather, int kUnroll, int kOrder>
__global__ __launch_bounds__(kThreads) void block_copy_fast_kernel(FastParams P) {
  fast_block<V, kGather, kUnroll, kOrder>(P, blockIdx.x);
}

// Sliced form of the fast gather, for blocks of exactly one pass (kUnroll *
// kThreads vectors: 32 KiB at 16-byte vectors) over an even number of whole
// storages: workgroup g moves slice g mod 2^kLog2H of each of 2^kLog2H
// consecutive ids of one storage, the slices of those blocks on consecutive
// workgroups, and storages in the fast gather's pairs order with id groups
// in place of ids. The bytes and where they land are those of the fast
// kernel; only the set a workgroup moves at once differs. Measured on MI355X
// (512 random ids over 64 storages of 16384 blocks, 2 GiB per launch, in one
// process alternating with the fast kernel, four machines): 4 slices +0.9 to
// +2.2 points of HBM bandwidth (e.g. 75.2 against 73.9 %). The same form for
// the scatter (8 slices, all-storages order) measured -1.5 to +1.7 points
// and is not used.
template <typename V, int kUnroll, int kLog2H>
__global__ __launch_bounds__(kThreads) void block_copy_sliced_gather_kernel(FastParams P) {
  constexpr uint32_t kH = 1u << kLog2H;
  constexpr uint32_t kSlice = kUnroll * kThreads / kH;  // vectors per slice
  // Each unrolled step's kThreads vectors lie in one slice of one block, so
  // a step's block (and its id) is the same for the whole workgroup.
  static_assert(kSlice % kThreads == 0, "a step must stay in one slice");
  constexpr uint32_t kSteps = kSlice / kThreads;  // steps per block
  uint32_t g = blockIdx.x;
  const uint32_t cc = g & (kH - 1);
  g >>= kLog2H;
  const uint32_t groups = (P.n + kH - 1) >> kLog2H;
  const uint32_t q = g / (2 * groups);
  const uint32_t r2 = g - q * 2 * groups;
  const uint32_t ig = r2 >> 1;
  const uint32_t w = P.w0 + 2 * q + (r2 & 1);
  const uint64_t base = uniform_load<uint64_t>(P.storages, w);
  const uint64_t stg0 = P.staging + w * static_cast<uint64_t>(P.stride_w);
  // The group's ids (the last group of a launch may hold fewer than kH); a
  // missing or bad id moves nothing, and a bad one sets the error flag.
  uint64_t pool_at[kH], stg_at[kH];
  bool ok[kH];
  bool bad_any = false;
#pragma unroll
  for (uint32_t r = 0; r < kH; ++r) {
    const uint32_t i = (ig << kLog2H) + r;
    const bool in = i < P.n;
    const int64_t id = in ? uniform_load<int64_t>(reinterpret_cast<uint64_t>(P.ids), i) : 0;
    const bool bad = in && bad_id(id, P.pool_blocks);
    ok[r] = in && !bad;
    bad_any |= bad;
    pool_at[r] = base + static_cast<uint64_t>(ok[r] ? id : 0) * P.elems * sizeof(V);
    stg_at[r] = stg0 + i * static_cast<uint64_t>(P.stride_i);
  }
  bool all_ok = true;
#pragma unroll
  for (uint32_t r = 0; r < kH; ++r) all_ok = all_ok && ok[r];
  const uint32_t lane0 = cc * kSlice + threadIdx.x;
  if (all_ok) {
    // Every step's load issued before the first store, as in the fast kernel.
    V v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const uint32_t r = u / kSteps;
      const uint32_t k = lane0 + (u % kSteps) * kThreads;
      v[u] = ld_nt(gptr<V>(pool_at[r]) + k);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const uint32_t r = u / kSteps;
      const uint32_t k = lane0 + (u % kSteps) * kThreads;
      st_nt(v[u], gptr<V>(stg_at[r]) + k);
    }
    return;
  }
  // The last group of a launch, or a group with a bad id: block by block.
  for (uint32_t r = 0; r < kH; ++r) {
    if (!ok[r]) continue;
    for (uint32_t t = 0; t < kSteps; ++t) {
      const uint32_t k = lane0 + t * kThreads;
      st_nt(ld_nt(gptr<V>(pool_at[r]) + k), gptr<V>(stg_at[r]) + k);
    }
  }
  if (bad_any && threadIdx.x == 0 && P.error != nullptr) atomicOr(P.error, 1);
}

// Slices per block (log2) of a sliced gather, 0 when the launch goes to the
// fast kernel: 16-byte vectors, blocks of exactly one pass, an even number of
// whole storages (the pairs order), an uncapped grid that fits.
constexpr int kGatherLog2Slices = 2;
int SlicedGatherLog2(const FastParams& F, CopyDir dir, int order, int vec_bytes, int unroll,
                     bool capped_grid) {
  if (dir != CopyDir::kGather || order != kStoragePairs) return 0;
  if (vec_bytes != 16 || capped_grid || F.pieces != 1) return 0;
  if (F.elems != static_cast<uint32_t>(unroll * kThreads)) return 0;
  const uint64_t groups =
      (static_cast<uint64_t>(F.n) + (1u << kGatherLog2Slices) - 1) >> kGatherLog2Slices;
  if ((groups << kGatherLog2Slices) * F.wstorages > INT32_MAX) return 0;
  return kGatherLog2Slices;
}

// The fast launch behind one leading small-block piece: the fp8 payload and
// its scale side table in one launch. The first side_wgs workgroups move the
// side piece (many blocks each, as in the general kernel), the rest take the
// payload blocks in the fast kernel's order.
template <typename V, bool kGather, int kUnroll, int kOrder>
__global__ __launch_bounds__(kThreads) void block_copy_fast_side_kernel(FastParams P, KPiece side,
                                                                        uint32_t side_wgs) {
  if (blockIdx.x < side_wgs) {
    copy_small_blocks<V, kGather>(side, P.ids, nullptr, P.error, P.n, blockIdx.x * side.bpw);
    return;
  }
  fast_block<V, kGather, kUnroll, kOrder>(P, blockIdx.x - side_wgs);
}

// Blocks per workgroup: one for blocks of >= 2 vectors per lane, otherwise
// enough blocks to give each lane up to 8 vectors, at most kSmallMaxBlocks.
uint32_t BlocksPerWorkgroup(uint64_t elems) {
  if (elems >= 2 * kThreads) return 1;
  uint64_t bpw = (8 * kThreads) / (elems == 0 ? 1 : elems);
  if (bpw > kSmallMaxBlocks) bpw = kSmallMaxBlocks;
  return static_cast<uint32_t>(bpw < 1 ? 1 : bpw);
}

bool BuildParams(const CopyLaunch& l, int vec_bytes, KParams* P,
                 uint32_t* grid) {
  if (l.npieces < 1 || l.npieces > kMaxPieces || l.ids == nullptr ||
      l.n <= 0 || l.n > INT32_MAX || vec_bytes <= 0) {
    return false;
  }
  *P = KParams{};
  P->ids = l.ids;
  P->ids2 = l.ids2;
  P->error = l.error;
  P->n = static_cast<uint32_t>(l.n);
  P->npieces = l.npieces;
  uint64_t total_blocks = 0;
  for (int k = 0; k < l.npieces; ++k) {
    total_blocks += static_cast<uint64_t>(l.pieces[k].nblocks > 0 ? l.pieces[k].nblocks : 0);
  }
  // Small-block pieces (side tables) take the first workgroups, so their
  // few workgroups run alongside the large blocks instead of after them.
  int order[kMaxPieces];
  int norder = 0;
  for (int pass = 0; pass < 2; ++pass) {
    for (int k = 0; k < l.npieces; ++k) {
      const int64_t bb = l.pieces[k].block_bytes;
      if (bb <= 0) return false;
      const bool whole = static_cast<uint64_t>(bb) / vec_bytes >= 2 * kThreads;
      if (whole == (pass == 1)) order[norder++] = k;
    }
  }
  uint64_t wg = 0;
  for (int slot = 0; slot < l.npieces; ++slot) {
    const CopyPiece& c = l.pieces[order[slot]];
    if (c.storages == 0 || c.nblocks <= 0 || c.f0 < 0 || c.block_bytes <= 0 ||
        c.block_bytes % vec_bytes != 0 || c.pool_blocks <= 0) {
      return false;
    }
    if (c.others != 0 && (l.ids2 == nullptr || c.other_blocks <= 0)) return false;
    if (static_cast<uint64_t>(c.f0) + static_cast<uint64_t>(c.nblocks) >
        UINT32_MAX) {
      return false;
    }
    const uint64_t elems = static_cast<uint64_t>(c.block_bytes) / vec_bytes;
    if (elems > UINT32_MAX) return false;
    const bool whole = elems >= 2 * kThreads;
    uint64_t bpw = BlocksPerWorkgroup(elems);
    if (whole && l.max_workgroups > 0) {
      // This piece's share of the workgroup cap, at least one.
      uint64_t share = static_cast<uint64_t>(l.max_workgroups) *
                       static_cast<uint64_t>(c.nblocks) / total_blocks;
      if (share < 1) share = 1;
      const uint64_t need = (static_cast<uint64_t>(c.nblocks) + share - 1) / share;
      if (need > bpw) bpw = need;
    }
    if (bpw > UINT32_MAX || (!whole && bpw * elems > UINT32_MAX)) return false;
    KPiece& kp = P->p[slot];
    kp.storages = c.storages;
    kp.staging = c.staging;
    kp.others = c.others;
    kp.other_blocks = c.other_blocks;
    kp.stride_w = c.stride_w;
    kp.stride_i = c.stride_i;
    kp.pool_blocks = c.pool_blocks;
    kp.f0 = static_cast<uint32_t>(c.f0);
    kp.nblocks = static_cast<uint32_t>(c.nblocks);
    kp.elems = static_cast<uint32_t>(elems);
    kp.bpw = static_cast<uint32_t>(bpw);
    kp.whole = whole ? 1u : 0u;
    kp.wg_begin = static_cast<uint32_t>(wg);
    wg += (static_cast<uint64_t>(c.nblocks) + bpw - 1) / bpw;
    if (wg > INT32_MAX) return false;
  }
  *grid = static_cast<uint32_t>(wg);
  return true;
}

// The fast kernel's parameters when the launch qualifies (one whole-block
// piece, bpw 1, no second paged side).
bool BuildFastParams(const KParams& K, CopyDir dir, FastParams* F, int* order) {
  const KPiece& p = K.p[0];
  if (K.npieces != 1 || !p.whole || p.bpw != 1 || p.others != 0) return false;
  *F = FastParams{};
  F->storages = p.storages;
  F->staging = p.staging;
  F->ids = K.ids;
  F->error = K.error;
  F->stride_w = p.stride_w;
  F->stride_i = p.stride_i;
  F->pool_blocks = p.pool_blocks;
  F->f0 = p.f0;
  F->n = K.n;
  F->elems = p.elems;
  const bool whole_storages = p.f0 % K.n == 0 && p.nblocks % K.n == 0;
  const uint32_t W = p.nblocks / K.n;
  *order = kStorageMajor;
  if (whole_storages && W >= 2) {
    if (dir == CopyDir::kScatter) {
      *order = kAllStorages;
    } else if (W % 2 == 0) {
      *order = kStoragePairs;
    }
  }
  F->wstorages = W;
  F->w0 = p.f0 / K.n;
  F->pieces = 1;
  F->piece_elems = p.elems;
  return true;
}

// The fast-with-side-piece parameters when the launch is one small-block
// piece (no second paged side; BuildParams puts it first) followed by one
// whole-block piece that qualifies for the fast kernel.
bool BuildFastSideParams(const KParams& K, CopyDir dir, FastParams* F, KPiece* side,
                         uint32_t* side_wgs, int* order) {
  if (K.npieces != 2 || K.p[0].whole || K.p[0].others != 0) return false;
  KParams one = K;
  one.npieces = 1;
  one.p[0] = K.p[1];
  if (!BuildFastParams(one, dir, F, order)) return false;
  *side = K.p[0];
  *side_wgs = K.p[1].wg_begin;
  return true;
}

// LDS of one CU on gfx950.
constexpr uint32_t kLdsPerCu = 160u << 10;

// LDS the general kernel declares (the small-block path's address tables).
constexpr uint32_t kStaticLds = 2 * kSmallMaxBlocks * sizeof(uint64_t);

template <typename V, int kUnroll>
hipError_t Launch(const KParams& P, uint32_t grid, CopyDir dir, int wg_per_cu,
                  bool capped_grid, hipStream_t stream) {
  FastParams F;
  int order = kStorageMajor;
  // Blocks above one workgroup's pass (kUnroll * kThreads vectors, 32 KiB at
  // 16-byte vectors) go to consecutive workgroups a pass each, unless the
  // launch's grid is capped (zero-copy copies keep their few workgroups).
  auto split = [&](FastParams* f, uint32_t blocks, uint32_t* g) {
    const uint32_t pass = kUnroll * kThreads;
    if (capped_grid || f->elems <= pass) return;
    const uint64_t pieces = (static_cast<uint64_t>(f->elems) + pass - 1) / pass;
    if (static_cast<uint64_t>(blocks) * pieces + (*g - blocks) > INT32_MAX) return;
    f->pieces = static_cast<uint32_t>(pieces);
    f->piece_elems = pass;
    *g = *g - blocks + blocks * f->pieces;
  };
  if (BuildFastParams(P, dir, &F, &order)) {
    if constexpr (sizeof(V) == 16) {
      const int s = SlicedGatherLog2(F, dir, order, 16, kUnroll, capped_grid);
      if (s > 0) {
        const uint32_t sgrid = (((F.n + (1u << s) - 1) >> s) << s) * F.wstorages;
        // The same cap on workgroups per CU as the fast gather.
        const uint32_t lds = wg_per_cu > 0 ? kLdsPerCu / static_cast<uint32_t>(wg_per_cu) : 0;
        hipLaunchKernelGGL((block_copy_sliced_gather_kernel<V, kUnroll, kGatherLog2Slices>),
                           dim3(sgrid), dim3(kThreads), lds, stream, F);
        return hipGetLastError();
      }
    }
    split(&F, grid, &grid);
    // Gathers reserve (unused) LDS to cap their workgroups per CU.
    const uint32_t lds = wg_per_cu > 0 ? kLdsPerCu / static_cast<uint32_t>(wg_per_cu) : 0;
    if (dir == CopyDir::kGather && order == kStoragePairs) {
      hipLaunchKernelGGL((block_copy_fast_kernel<V, true, kUnroll, kStoragePairs>), dim3(grid),
                         dim3(kThreads), lds, stream, F);
    } else if (dir == CopyDir::kGather) {
      hipLaunchKernelGGL((block_copy_fast_kernel<V, true, kUnroll, kStorageMajor>), dim3(grid),
                         dim3(kThreads), lds, stream, F);
    } else if (order == kAllStorages) {
      hipLaunchKernelGGL((block_copy_fast_kernel<V, false, kUnroll, kAllStorages>), dim3(grid),
                         dim3(kThreads), 0, stream, F);
    } else {
      hipLaunchKernelGGL((block_copy_fast_kernel<V, false, kUnroll, kStorageMajor>), dim3(grid),
                         dim3(kThreads), 0, stream, F);
    }
    return hipGetLastError();
  }
  // HBM-bound gathers (not the capped grids of zero-copy copies) on the
  // kernels with the small-block path take the same cap, minus that path's
  // own 4 KiB of address tables.
  const uint32_t glds = wg_per_cu > 0 && !capped_grid
                            ? kLdsPerCu / static_cast<uint32_t>(wg_per_cu) - kStaticLds
                            : 0;
  KPiece side;
  uint32_t side_wgs = 0;
  if (BuildFastSideParams(P, dir, &F, &side, &side_wgs, &order)) {
    split(&F, grid - side_wgs, &grid);
    if (dir == CopyDir::kGather && order == kStoragePairs) {
      hipLaunchKernelGGL((block_copy_fast_side_kernel<V, true, kUnroll, kStoragePairs>),
                         dim3(grid), dim3(kThreads), glds, stream, F, side, side_wgs);
    } else if (dir == CopyDir::kGather) {
      hipLaunchKernelGGL((block_copy_fast_side_kernel<V, true, kUnroll, kStorageMajor>),
                         dim3(grid), dim3(kThreads), glds, stream, F, side, side_wgs);
    } else if (order == kAllStorages) {
      hipLaunchKernelGGL((block_copy_fast_side_kernel<V, false, kUnroll, kAllStorages>),
                         dim3(grid), dim3(kThreads), 0, stream, F, side, side_wgs);
    } else {
      hipLaunchKernelGGL((block_copy_fast_side_kernel<V, false, kUnroll, kStorageMajor>),
                         dim3(grid), dim3(kThreads), 0, stream, F, side, side_wgs);
    }
    return hipGetLastError();
  }
  if (dir == CopyDir::kGather) {
    hipLaunchKernelGGL((block_copy_kernel<V, true, kUnroll>), dim3(grid),
                       dim3(kThreads), glds, stream, P);
  } else {
    hipLaunchKernelGGL((block_copy_kernel<V, false, kUnroll>), dim3(grid),
                       dim3(kThreads), 0, stream, P);
  }
  return hipGetLastError();
}

}  // namespace

int LaunchVectorBytes(const CopyLaunch& l, uint64_t extra_align) {
  uint64_t acc = extra_align;
  for (int k = 0; k < l.npieces && k < kMaxPieces; ++k) {
    const CopyPiece& c = l.pieces[k];
    acc |= static_cast<uint64_t>(c.block_bytes) | c.staging |
           static_cast<uint64_t>(c.stride_w) | static_cast<uint64_t>(c.stride_i);
  }
  if ((acc & 15) == 0) return 16;
  if ((acc & 3) == 0) return 4;
  return 1;
}

int64_t BlockCopyWorkgroups(const CopyLaunch& l, int vec_bytes) {
  KParams P;
  uint32_t grid = 0;
  if (!BuildParams(l, vec_bytes, &P, &grid)) return -1;
  return grid;
}

hipError_t LaunchBlockCopy(const CopyLaunch& l, CopyDir dir, int vec_bytes,
                           hipStream_t stream) {
  KParams P;
  uint32_t grid = 0;
  if (!BuildParams(l, vec_bytes, &P, &grid)) return hipErrorInvalidValue;
  if (l.gather_workgroups_per_cu < 0 || l.gather_workgroups_per_cu > 32) {
    return hipErrorInvalidValue;
  }
  const int cap = l.gather_workgroups_per_cu;
  switch (vec_bytes) {
    case 16:
      return Launch<u32x4, 8>(P, grid, dir, cap, l.max_workgroups > 0, stream);
    case 4:
      return Launch<uint32_t, 8>(P, grid, dir, cap, l.max_workgroups > 0, stream);
    case 1:
      return Launch<uint8_t, 8>(P, grid, dir, cap, l.max_workgroups > 0, stream);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace kvx
