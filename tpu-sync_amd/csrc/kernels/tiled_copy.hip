// Tiled-layout copy for gfx950 (MI355X): tile / detile of XLA-style tiled
// tensor layouts on the device, the work the reference's TileBuffer /
// DetileBuffer do on the host CPU (tpu_sync/weight_sync/tiling_utils.cc:
// 545-1036) before or after a raw DMA of the tiled bytes.
//
// Pure data movement, bound by HBM bandwidth. Every (vector width, rows per
// unit, direction, unit order) combination is a kernel of its own, so the
// hot loop carries no mode branches; the host groups a launch's jobs by that
// key. Standard-form jobs move units of P rows x V bytes; a lane issues all
// loads of its units (128 bytes in flight) before its stores, so a workgroup
// keeps 32 KiB in flight like the other copy kernels. Consecutive lanes take
// consecutive units, which are consecutive column vectors of the same rows
// in linear order and consecutive pieces of the tiled buffer in tiled order.
// Packed layouts (P = 2 for 16-bit, P = 4 for 8-bit elements) interleave the
// P rows in registers with 32-bit shifts, masks and byte permutes. Divisions
// by layout constants use multiply-high (FastDivU32). Loads and stores are
// non-temporal (every byte is touched once).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "tiled_copy.h"

namespace kvx {
namespace {

constexpr int kThreads = 256;
constexpr int kVecsPerLane = 8;
// A launch reserves LDS it does not use so that at most 2 of its workgroups
// share a CU, as the strided and block copies do (fewer concurrent streams
// per CU keep the DRAM access pattern closer to sequential).
constexpr uint32_t kLdsPerCu = 160u << 10;
constexpr uint32_t kWorkgroupsPerCu = 2;
constexpr uint32_t kXcds = 8;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define KVX_GLOBAL __attribute__((address_space(1)))
#define KVX_CONST __attribute__((address_space(4)))

__device__ __forceinline__ uint32_t fdiv(const KVX_CONST FastDivU32* f, uint32_t n) {
  const uint32_t hi = __umulhi(n, f->m);
  return static_cast<uint32_t>((static_cast<uint64_t>(hi) + n) >> f->s);
}

// V-byte vector type.
template <int V> struct VecT;
template <> struct VecT<16> { typedef u32x4 T; };
template <> struct VecT<8> { typedef u32x2 T; };
template <> struct VecT<4> { typedef uint32_t T; };
template <> struct VecT<2> { typedef uint16_t T; };
template <> struct VecT<1> { typedef uint8_t T; };

template <int V>
__device__ __forceinline__ typename VecT<V>::T ld(uint64_t a) {
  return __builtin_nontemporal_load((const KVX_GLOBAL typename VecT<V>::T*)a);
}
template <int V>
__device__ __forceinline__ void st(uint64_t a, typename VecT<V>::T v) {
  __builtin_nontemporal_store(v, (KVX_GLOBAL typename VecT<V>::T*)a);
}

// 32-bit words of a V-byte vector (V >= 4).
template <int V>
__device__ __forceinline__ void to_words(typename VecT<V>::T v, uint32_t* w) {
  if constexpr (V == 16) {
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
  } else if constexpr (V == 8) {
    w[0] = v.x; w[1] = v.y;
  } else {
    w[0] = v;
  }
}
template <int V>
__device__ __forceinline__ typename VecT<V>::T from_words(const uint32_t* w) {
  typename VecT<V>::T v;
  if constexpr (V == 16) {
    v.x = w[0]; v.y = w[1]; v.z = w[2]; v.w = w[3];
  } else if constexpr (V == 8) {
    v.x = w[0]; v.y = w[1];
  } else {
    v = w[0];
  }
  return v;
}

// Tiled order of P rows of n words each: element c of row k lands at
// position c * P + k. P = 2: 16-bit elements; P = 4: 8-bit elements.
template <int P, int n>
__device__ __forceinline__ void interleave(const uint32_t (&rows)[P][n], uint32_t (&out)[P * n]) {
#pragma unroll
  for (int i = 0; i < n; ++i) {
    if constexpr (P == 2) {
      const uint32_t a = rows[0][i], b = rows[1][i];
      out[2 * i] = (a & 0xffffu) | (b << 16);
      out[2 * i + 1] = (a >> 16) | (b & 0xffff0000u);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        out[4 * i + j] = ((rows[0][i] >> (8 * j)) & 0xffu) |
                         (((rows[1][i] >> (8 * j)) & 0xffu) << 8) |
                         (((rows[2][i] >> (8 * j)) & 0xffu) << 16) |
                         (((rows[3][i] >> (8 * j)) & 0xffu) << 24);
      }
    }
  }
}

template <int P, int n>
__device__ __forceinline__ void deinterleave(const uint32_t (&in)[P * n], uint32_t (&rows)[P][n]) {
#pragma unroll
  for (int i = 0; i < n; ++i) {
    if constexpr (P == 2) {
      const uint32_t x = in[2 * i], y = in[2 * i + 1];
      rows[0][i] = (x & 0xffffu) | (y << 16);
      rows[1][i] = (x >> 16) | (y & 0xffff0000u);
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        rows[k][i] = ((in[4 * i] >> (8 * k)) & 0xffu) |
                     (((in[4 * i + 1] >> (8 * k)) & 0xffu) << 8) |
                     (((in[4 * i + 2] >> (8 * k)) & 0xffu) << 16) |
                     (((in[4 * i + 3] >> (8 * k)) & 0xffu) << 24);
      }
    }
  }
}

// Addresses of a standard-form unit: the tiled piece, the linear address of
// its first row (row k is k * W * itemsize further), its first row h within
// the batch matrix and first column c. In tiled order the unit may lie in
// padding (h >= H or c >= W): the linear address is then clamped to the last
// row / last column vector of the matrix (the same tile row, so inside the
// job's range) for callers that load before they test.
template <int P, bool TORDER>
__device__ __forceinline__ void unit_addr(const KVX_CONST TiledJobDev* j, uint32_t u,
                                          uint32_t E, uint32_t unit_bytes, uint64_t* tiled,
                                          uint64_t* lin, uint32_t* h, uint32_t* c_out) {
  const uint32_t H = j->h32, W = j->w32, sh = j->log2s;
  uint32_t b, row, c, T, within;
  if constexpr (TORDER) {
    const uint32_t q = fdiv(&j->t_ncv, u);
    const uint32_t cvt = u - q * j->t_ncv.d;
    T = fdiv(&j->t_gpt, q);
    const uint32_t gi = q - T * j->t_gpt.d;
    const uint32_t btr = fdiv(&j->t_nt1, T);
    const uint32_t tc = T - btr * j->t_nt1.d;
    b = fdiv(&j->t_nt0, btr);
    const uint32_t tr = btr - b * j->t_nt0.d;
    row = tr * j->th.d + gi * P;
    c = tc * j->tw.d + cvt * E;
    *tiled = j->tiled + static_cast<uint64_t>(u) * unit_bytes;
    const uint32_t rc = row < H ? row : H - 1;
    const uint32_t cc = c < W ? c : W - E;
    *lin = j->linear + ((static_cast<uint64_t>(b * H + rc) * W + cc) << sh);
  } else {
    const uint32_t q = fdiv(&j->ncv, u);
    const uint32_t cv = u - q * j->ncv.d;
    b = fdiv(&j->ng, q);
    const uint32_t g = q - b * j->ng.d;
    row = g * P;
    const uint32_t tr = fdiv(&j->th, row);
    const uint32_t r0 = row - tr * j->th.d;
    c = cv * E;
    const uint32_t tc = fdiv(&j->tw, c);
    const uint32_t cc = c - tc * j->tw.d;
    T = (b * j->nt0 + tr) * j->nt1 + tc;
    within = r0 * j->tw.d + cc * P;
    *tiled = j->tiled + ((static_cast<uint64_t>(T) * j->tile_elems + within) << sh);
    *lin = j->linear + ((static_cast<uint64_t>(b * H + row) * W + c) << sh);
  }
  *h = row;
  *c_out = c;
}

// Standard form, P = 1: each unit is one V-byte vector on both sides.
template <int V, bool TILE, bool TORDER>
__device__ __forceinline__ void std_p1(const KVX_CONST TiledJobDev* j, uint32_t local) {
  constexpr int U = kVecsPerLane;
  const uint32_t E = V >> j->log2s;
  const uint64_t first = j->lo + static_cast<uint64_t>(local) * (kThreads * U);
  const uint64_t end = j->lo + j->count;
  const uint32_t H = j->h32, W = j->w32;
  typename VecT<V>::T r[U];
  uint64_t dst[U];
  bool valid[U];
#pragma unroll
  for (int i = 0; i < U; ++i) {
    uint64_t u = first + threadIdx.x + i * kThreads;
    u = u < end ? u : end - 1;
    uint64_t ta, la;
    uint32_t h, c;
    unit_addr<1, TORDER>(j, static_cast<uint32_t>(u), E, V, &ta, &la, &h, &c);
    valid[i] = !TORDER || (h < H && c < W);
    r[i] = ld<V>(TILE ? la : ta);
    dst[i] = TILE ? ta : la;
  }
#pragma unroll
  for (int i = 0; i < U; ++i) {
    if (first + threadIdx.x + i * kThreads >= end) continue;
    if (TILE) {
      st<V>(dst[i], valid[i] ? r[i] : typename VecT<V>::T{});
    } else if (valid[i]) {
      st<V>(dst[i], r[i]);
    }
  }
}

// Standard form, P = 2 or 4, one lane per unit: P rows x V bytes, P * V
// bytes of the tiled buffer.
template <int V, int P, bool TILE, bool TORDER>
__device__ __forceinline__ void std_packed(const KVX_CONST TiledJobDev* j, uint32_t local) {
  constexpr int U = 128 / (P * V);
  constexpr int n = V / 4;
  constexpr uint32_t E = V * P / 4;  // elements per row vector (P * itemsize = 4)
  const uint64_t first = j->lo + static_cast<uint64_t>(local) * (kThreads * U);
  const uint64_t end = j->lo + j->count;
  const uint64_t row_bytes = static_cast<uint64_t>(j->w32) << j->log2s;
  const uint32_t H = j->h32, W = j->w32;
  uint32_t words[U][P * n];
  uint64_t ta[U], la[U];
  uint32_t h[U], c[U];
#pragma unroll
  for (int i = 0; i < U; ++i) {
    uint64_t u = first + threadIdx.x + i * kThreads;
    u = u < end ? u : end - 1;
    unit_addr<P, TORDER>(j, static_cast<uint32_t>(u), E, P * V, &ta[i], &la[i], &h[i], &c[i]);
    if (TILE) {
      // Rows past the matrix's end read a valid row and are zeroed below.
#pragma unroll
      for (int k = 0; k < P; ++k) {
        const uint32_t kk = h[i] + k < H ? k : 0;
        to_words<V>(ld<V>(la[i] + kk * row_bytes), &words[i][k * n]);
      }
    } else {
#pragma unroll
      for (int k = 0; k < P; ++k) to_words<V>(ld<V>(ta[i] + k * V), &words[i][k * n]);
    }
  }
#pragma unroll
  for (int i = 0; i < U; ++i) {
    if (first + threadIdx.x + i * kThreads >= end) continue;
    const bool col_ok = c[i] < W;
    if (TILE) {
      uint32_t rows[P][n];
#pragma unroll
      for (int k = 0; k < P; ++k) {
        const bool valid = col_ok && h[i] + k < H;
#pragma unroll
        for (int w = 0; w < n; ++w) rows[k][w] = valid ? words[i][k * n + w] : 0u;
      }
      uint32_t out[P * n];
      interleave<P, n>(rows, out);
#pragma unroll
      for (int k = 0; k < P; ++k) st<V>(ta[i] + k * V, from_words<V>(&out[k * n]));
    } else {
      uint32_t in[P * n];
#pragma unroll
      for (int w = 0; w < P * n; ++w) in[w] = words[i][w];
      uint32_t rows[P][n];
      deinterleave<P, n>(in, rows);
#pragma unroll
      for (int k = 0; k < P; ++k) {
        if (col_ok && h[i] + k < H) st<V>(la[i] + k * row_bytes, from_words<V>(rows[k]));
      }
    }
  }
}

// Detiling, standard form, P = 2 (16-bit elements in pairs) with 16-byte row
// vectors, linear order, two lanes per unit: 2 rows x 16 bytes of the linear
// image, 32 contiguous bytes of the tiled buffer (8 columns of 4 bytes, one
// per row). A workgroup's lane slot i covers 128 consecutive units, exchanged
// through LDS so that every store of a wave is one contiguous 1 KiB span:
//   loads: lane t loads 16 tiled bytes (columns 4 (t % 2) .. + 3 of both
//     rows) of unit t / 2, so a wave reads 1 KiB of the tiled buffer;
//   stores: lane t stores 16 bytes (one column vector) of unit t % 128 in
//     row t / 128, so each wave writes 1 KiB of one row.
// Measured on the Llama-3-8B parameter set in T(8,128)(2,1) (16.06 GB), one
// process, two builds side by side: 79.6 % of HBM peak against 78.4 % with
// the exchange inside each lane pair (__shfl_xor; each store instruction then
// 2 rows x 512 bytes). A lane keeps 8 vectors in flight. Slots taken sliced
// over groups of 8 workgroups (below): 77.3 -> 79.2 % in one process.
constexpr uint32_t kPairLdsBytes = kVecsPerLane * 2 * (kThreads / 2) * 4 * 4;

__device__ __forceinline__ void std_pair_detile(const KVX_CONST TiledJobDev* j, uint32_t local) {
  constexpr int P = 2;
  constexpr int U = kVecsPerLane;
  constexpr uint32_t E = 8;                      // 16-bit elements per 16-byte row vector
  constexpr uint32_t kSlotUnits = kThreads / P;  // 128 units per slot
  __shared__ __attribute__((aligned(16))) uint32_t lds[U][P][kSlotUnits * 4];
  const uint64_t first = j->lo + static_cast<uint64_t>(local) * (U * kSlotUnits);
  // Slots in whole groups of U consecutive workgroups of the job go sliced:
  // slot i of the workgroup at place jj of its group takes the jj-th slot of
  // the group's chunk i, so a workgroup's bytes are U pieces spread over the
  // group instead of one contiguous chunk. The job's last workgroups (fewer
  // than a group) keep their own chunk.
  constexpr uint32_t kChunk = U * kSlotUnits;
  const uint64_t nwg = (j->count + kChunk - 1) / kChunk;
  const uint32_t gb = local & ~static_cast<uint32_t>(U - 1);
  const uint32_t jj = local & static_cast<uint32_t>(U - 1);
  const bool sliced = j->sliced != 0 && gb + static_cast<uint64_t>(U) <= nwg;
  const uint64_t end = j->lo + j->count;
  const uint64_t last_unit = end - 1;
  const uint64_t row_bytes = static_cast<uint64_t>(j->w32) << j->log2s;
  const uint32_t H = j->h32;
  const uint32_t t = threadIdx.x;
  // Loads: piece k of unit ut; stores: row r of unit ul.
  const uint32_t ut = t / P, k = t % P;
  const uint32_t ul = t % kSlotUnits, r = t / kSlotUnits;
  uint32_t v[U][4];
#pragma unroll
  for (int i = 0; i < U; ++i) {
    const uint64_t base = sliced ? j->lo + static_cast<uint64_t>(gb + i) * kChunk +
                                       static_cast<uint64_t>(jj) * kSlotUnits
                                 : first + static_cast<uint64_t>(i) * kSlotUnits;
    const uint64_t u0 = base + ut;
    const uint64_t u = u0 < last_unit ? u0 : last_unit;
    uint64_t ta, la;
    uint32_t h, c;
    unit_addr<P, false>(j, static_cast<uint32_t>(u), E, P * 16, &ta, &la, &h, &c);
    to_words<16>(ld<16>(ta + 16 * k), v[i]);
  }
#pragma unroll
  for (int i = 0; i < U; ++i) {
    uint32_t rows[P][2];
    deinterleave<P, 2>(v[i], rows);  // columns 4k..4k+3 of each row
#pragma unroll
    for (int q = 0; q < P; ++q) {
      lds[i][q][ut * 4 + 2 * k] = rows[q][0];
      lds[i][q][ut * 4 + 2 * k + 1] = rows[q][1];
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < U; ++i) {
    const u32x4 x = *reinterpret_cast<const u32x4*>(&lds[i][r][ul * 4]);
    v[i][0] = x.x; v[i][1] = x.y; v[i][2] = x.z; v[i][3] = x.w;
  }
#pragma unroll
  for (int i = 0; i < U; ++i) {
    const uint64_t base = sliced ? j->lo + static_cast<uint64_t>(gb + i) * kChunk +
                                       static_cast<uint64_t>(jj) * kSlotUnits
                                 : first + static_cast<uint64_t>(i) * kSlotUnits;
    const uint64_t u0 = base + ul;
    const uint64_t u = u0 < last_unit ? u0 : last_unit;
    uint64_t ta, la;
    uint32_t h, c;
    unit_addr<P, false>(j, static_cast<uint32_t>(u), E, P * 16, &ta, &la, &h, &c);
    if (u0 < end && h + r < H) st<16>(la + r * row_bytes, from_words<16>(v[i]));
  }
}

// Detiling, standard form, P = 4 (8-bit elements in fours) with 16-byte row
// vectors, linear order, four lanes per unit: 4 rows x 16 bytes of the
// linear image, 64 contiguous bytes of the tiled buffer (16 columns of 4
// bytes, one per row). A workgroup's lane slot i covers 64 consecutive
// units, exchanged through LDS so that every global access of a wave is one
// contiguous 1 KiB span:
//   loads: lane t loads 16 tiled bytes (columns 4 (t % 4) .. + 3, all four
//     rows) of unit t / 4, so a wave covers 16 whole units;
//   stores: lane t stores 16 bytes (one column vector) of unit t % 64 in row
//     t / 64, so wave w writes 1 KiB of row w.
// Each tiled vector is unpacked into one word per row; the words go to LDS
// (row r of the slot's 64 units is one 1 KiB LDS row) and, after a workgroup
// barrier, come back 16 bytes of one row per lane. Measured on 8 int8
// [14336, 8192] matrices in T(8,128)(4,1) (0.94 GB), one process, two builds
// side by side: 71.6 % of HBM peak against 61.8 % with one lane per 16-byte
// tiled vector (4-byte row stores) and 65.3 % with the exchange inside each
// wave (each store instruction then 4 rows x 256 bytes). Tiling the same
// way measured 67.0 % against 72.3 % for one lane per tiled vector, so
// tiling keeps that form. A lane keeps 8 vectors in flight. Slots taken
// sliced over groups of 8 workgroups: 74.1 -> 76.8 % in one process.
constexpr uint32_t kQuadLdsBytes = kVecsPerLane * 4 * kThreads * 4;

__device__ __forceinline__ void std_quad_detile(const KVX_CONST TiledJobDev* j, uint32_t local) {
  constexpr int P = 4;
  constexpr int U = kVecsPerLane;
  constexpr uint32_t E = 16;  // 8-bit elements per 16-byte row vector
  constexpr uint32_t kSlotUnits = kThreads / P;  // 64 units per slot
  __shared__ uint32_t lds[U][P][kThreads];       // [slot][row][unit * 4 + word]
  const uint64_t first = j->lo + static_cast<uint64_t>(local) * (U * kSlotUnits);
  // Slots in whole groups of U consecutive workgroups of the job go sliced:
  // slot i of the workgroup at place jj of its group takes the jj-th slot of
  // the group's chunk i, so a workgroup's bytes are U pieces spread over the
  // group instead of one contiguous chunk. The job's last workgroups (fewer
  // than a group) keep their own chunk.
  constexpr uint32_t kChunk = U * kSlotUnits;
  const uint64_t nwg = (j->count + kChunk - 1) / kChunk;
  const uint32_t gb = local & ~static_cast<uint32_t>(U - 1);
  const uint32_t jj = local & static_cast<uint32_t>(U - 1);
  const bool sliced = j->sliced != 0 && gb + static_cast<uint64_t>(U) <= nwg;
  const uint64_t end = j->lo + j->count;
  const uint64_t last_unit = end - 1;
  const uint64_t row_bytes = static_cast<uint64_t>(j->w32) << j->log2s;
  const uint32_t H = j->h32;
  const uint32_t t = threadIdx.x;
  // Loads: piece k of unit ut; stores: row r of unit ul.
  const uint32_t ut = t / P, k = t % P;
  const uint32_t ul = t % kSlotUnits, r = t / kSlotUnits;
  // Every slot's load first, so that a lane has 8 vectors in flight.
  uint32_t v[U][4];
#pragma unroll
  for (int i = 0; i < U; ++i) {
    const uint64_t base = sliced ? j->lo + static_cast<uint64_t>(gb + i) * kChunk +
                                       static_cast<uint64_t>(jj) * kSlotUnits
                                 : first + static_cast<uint64_t>(i) * kSlotUnits;
    const uint64_t u0 = base + ut;
    const uint64_t u = u0 < last_unit ? u0 : last_unit;
    uint64_t ta, la;
    uint32_t h, c;
    unit_addr<P, false>(j, static_cast<uint32_t>(u), E, P * 16, &ta, &la, &h, &c);
    to_words<16>(ld<16>(ta + 16 * k), v[i]);
  }
#pragma unroll
  for (int i = 0; i < U; ++i) {
    uint32_t rows[4][1];
    deinterleave<4, 1>(v[i], rows);  // columns 4k..4k+3 of each row
#pragma unroll
    for (int q = 0; q < 4; ++q) lds[i][q][t] = rows[q][0];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < U; ++i) {
    const u32x4 x = *reinterpret_cast<const u32x4*>(&lds[i][r][ul * 4]);
    v[i][0] = x.x; v[i][1] = x.y; v[i][2] = x.z; v[i][3] = x.w;
  }
#pragma unroll
  for (int i = 0; i < U; ++i) {
    const uint64_t base = sliced ? j->lo + static_cast<uint64_t>(gb + i) * kChunk +
                                       static_cast<uint64_t>(jj) * kSlotUnits
                                 : first + static_cast<uint64_t>(i) * kSlotUnits;
    const uint64_t u0 = base + ul;
    const uint64_t u = u0 < last_unit ? u0 : last_unit;
    uint64_t ta, la;
    uint32_t h, c;
    unit_addr<P, false>(j, static_cast<uint32_t>(u), E, P * 16, &ta, &la, &h, &c);
    if (u0 < end && h + r < H) st<16>(la + r * row_bytes, from_words<16>(v[i]));
  }
}

// General form: physical element of logical element e.
__device__ __forceinline__ uint64_t gen_phys(const KVX_CONST TiledJobDev* j,
                                             const KVX_CONST TiledGenDim* gd, uint32_t e) {
  uint32_t idx[kTiledMaxRank];
  uint32_t rest = e;
#pragma unroll
  for (int r = kTiledMaxRank - 1; r >= 0; --r) {
    if (r < static_cast<int>(j->rank)) {
      const uint32_t q = fdiv(&j->dims[r], rest);
      idx[r] = rest - q * j->dims[r].d;
      rest = q;
    } else {
      idx[r] = 0;
    }
  }
  uint64_t phys = 0;
  for (uint32_t k = 0; k < j->ngen; ++k) {
    const int32_t src = gd[k].src;
    uint32_t x = 0;
#pragma unroll
    for (int r = 0; r < kTiledMaxRank; ++r) x = src == r ? idx[r] : x;
    for (uint32_t o = 0; o < gd[k].nops; ++o) {
      const uint32_t q = fdiv(&gd[k].op[o], x);
      x = (gd[k].is_mod >> o) & 1u ? x - q * gd[k].op[o].d : q;
    }
    phys += static_cast<uint64_t>(x) * gd[k].stride;
  }
  return phys;
}

template <typename T, bool TILE>
__device__ __forceinline__ void gen_job(const KVX_CONST TiledJobDev* j,
                                        const KVX_CONST TiledGenDim* gd, uint32_t local) {
  constexpr int U = kVecsPerLane;
  const uint64_t first = j->lo + static_cast<uint64_t>(local) * (kThreads * U);
  const uint64_t end = j->lo + j->count;
  T v[U];
  uint64_t dst[U];
#pragma unroll
  for (int i = 0; i < U; ++i) {
    uint64_t e = first + threadIdx.x + i * kThreads;
    e = e < end ? e : end - 1;
    const uint64_t p = gen_phys(j, gd, static_cast<uint32_t>(e));
    const uint64_t ta = j->tiled + p * sizeof(T);
    const uint64_t la = j->linear + e * sizeof(T);
    v[i] = *(const KVX_GLOBAL T*)(TILE ? la : ta);
    dst[i] = TILE ? ta : la;
  }
#pragma unroll
  for (int i = 0; i < U; ++i) {
    if (first + threadIdx.x + i * kThreads < end) *(KVX_GLOBAL T*)dst[i] = v[i];
  }
}

// Workgroup g runs on XCD g % 8 (MI355X dispatches workgroups round-robin
// over its 8 XCDs); it takes work item (g % 8) * per + g / 8, so each XCD
// streams one contiguous eighth of the launch, as the strided copy does.
// Items past 8 * per map to themselves; the map is a bijection.
__device__ __forceinline__ uint32_t xcd_item(uint32_t g, uint32_t n) {
  const uint32_t per = n / kXcds;
  if (g >= per * kXcds) return g;
  return (g % kXcds) * per + g / kXcds;
}

__device__ __forceinline__ const KVX_CONST TiledJobDev* job_of(const uint8_t* image,
                                                               uint32_t map_offset,
                                                               uint32_t* local) {
  const uint32_t wg = xcd_item(blockIdx.x, gridDim.x);
  const uint32_t ji = ((const KVX_CONST uint32_t*)(image + map_offset))[wg];
  const KVX_CONST TiledJobDev* j = (const KVX_CONST TiledJobDev*)image + ji;
  *local = wg - j->wg_begin;
  return j;
}

// LANES: lanes per unit; 2 for P = 2 and 4 for P = 4 when detiling at 16-byte
// rows (through LDS), else 1.
template <int V, int P, bool TILE, bool TORDER, int LANES>
__global__ __launch_bounds__(kThreads) void tiled_std_kernel(const uint8_t* image,
                                                             uint32_t map_offset) {
  uint32_t local;
  const KVX_CONST TiledJobDev* j = job_of(image, map_offset, &local);
  if constexpr (P == 1) {
    std_p1<V, TILE, TORDER>(j, local);
  } else if constexpr (LANES == 2) {
    static_assert(!TILE && !TORDER, "two lanes per unit: detiling in linear order only");
    std_pair_detile(j, local);
  } else if constexpr (LANES == 4) {
    static_assert(!TILE && !TORDER, "four lanes per unit: detiling in linear order only");
    std_quad_detile(j, local);
  } else {
    std_packed<V, P, TILE, TORDER>(j, local);
  }
}

template <typename T, bool TILE>
__global__ __launch_bounds__(kThreads) void tiled_gen_kernel(const uint8_t* image,
                                                             uint32_t map_offset) {
  uint32_t local;
  const KVX_CONST TiledJobDev* j = job_of(image, map_offset, &local);
  gen_job<T, TILE>(j, (const KVX_CONST TiledGenDim*)(image + j->gen_offset), local);
}

template <int V>
__global__ __launch_bounds__(kThreads) void tiled_zero_kernel(const uint8_t* image,
                                                              uint32_t map_offset) {
  uint32_t local;
  const KVX_CONST TiledJobDev* j = job_of(image, map_offset, &local);
  const uint64_t first = j->lo + static_cast<uint64_t>(local) * (kThreads * kVecsPerLane);
  const uint64_t end = j->lo + j->count;
  typename VecT<V>::T z{};
#pragma unroll
  for (int i = 0; i < kVecsPerLane; ++i) {
    const uint64_t x = first + threadIdx.x + i * kThreads;
    if (x < end) st<V>(j->tiled + x * V, z);
  }
}

typedef void (*KernelFn)(const uint8_t*, uint32_t);

template <int V, int P, int LANES>
KernelFn StdKernel(bool tile, bool torder) {
  if (tile) {
    return torder ? tiled_std_kernel<V, P, true, true, LANES>
                  : tiled_std_kernel<V, P, true, false, LANES>;
  }
  return torder ? tiled_std_kernel<V, P, false, true, LANES>
                : tiled_std_kernel<V, P, false, false, LANES>;
}

template <int V>
KernelFn StdKernelP(int P, bool tile, bool torder, int lanes) {
  if (P == 1) return StdKernel<V, 1, 1>(tile, torder);
  if constexpr (V >= 4) {
    if constexpr (V == 16) {
      if (lanes == 2 && P == 2 && !tile && !torder) {
        return tiled_std_kernel<16, 2, false, false, 2>;
      }
      if (lanes == 4 && P == 4 && !tile && !torder) {
        return tiled_std_kernel<16, 4, false, false, 4>;
      }
    }
    if (P == 2) return StdKernel<V, 2, 1>(tile, torder);
    if (P == 4) return StdKernel<V, 4, 1>(tile, torder);
  }
  return nullptr;
}

KernelFn PickKernel(const TiledLaunchKey& k) {
  if (k.mode == kZero) {
    switch (k.vec) {
      case 16: return tiled_zero_kernel<16>;
      case 8: return tiled_zero_kernel<8>;
      case 4: return tiled_zero_kernel<4>;
      case 2: return tiled_zero_kernel<2>;
      case 1: return tiled_zero_kernel<1>;
      default: return nullptr;
    }
  }
  if (k.mode == kDetileGen || k.mode == kTileGen) {
    const bool t = k.mode == kTileGen;
    switch (k.itemsize) {
      case 1: return t ? tiled_gen_kernel<uint8_t, true> : tiled_gen_kernel<uint8_t, false>;
      case 2: return t ? tiled_gen_kernel<uint16_t, true> : tiled_gen_kernel<uint16_t, false>;
      case 4: return t ? tiled_gen_kernel<uint32_t, true> : tiled_gen_kernel<uint32_t, false>;
      case 8: return t ? tiled_gen_kernel<uint64_t, true> : tiled_gen_kernel<uint64_t, false>;
      default: return nullptr;
    }
  }
  const bool tile = k.mode == kTileStd;
  const int lanes = static_cast<int>(k.lanes);
  switch (k.vec) {
    case 16: return StdKernelP<16>(k.P, tile, k.torder != 0, lanes);
    case 8: return StdKernelP<8>(k.P, tile, k.torder != 0, lanes);
    case 4: return StdKernelP<4>(k.P, tile, k.torder != 0, lanes);
    case 2: return StdKernelP<2>(k.P, tile, k.torder != 0, lanes);
    case 1: return StdKernelP<1>(k.P, tile, k.torder != 0, lanes);
    default: return nullptr;
  }
}

}  // namespace

TiledLaunchKey LaunchKeyOf(const TiledJobDev& j, int vec_bytes) {
  TiledLaunchKey k{};
  k.mode = j.mode;
  k.itemsize = j.itemsize;
  if (j.mode == kDetileStd || j.mode == kTileStd) {
    k.vec = static_cast<uint32_t>(vec_bytes);
    k.P = j.P;
    k.torder = j.torder;
    k.lanes = j.P == 2 && vec_bytes == 16 && j.lanes_per_unit == 2   ? 2
              : j.P == 4 && vec_bytes == 16 && j.lanes_per_unit == 4 ? 4
                                                                     : 1;
  } else if (j.mode == kZero) {
    k.vec = static_cast<uint32_t>(vec_bytes);
    k.itemsize = 0;
  }
  return k;
}

uint32_t TiledPerWorkgroup(const TiledLaunchKey& k) {
  if ((k.mode == kDetileStd || k.mode == kTileStd) && k.P > 1) {
    if (k.lanes == 2) return kThreads * kVecsPerLane / 2;  // two lanes per unit
    if (k.lanes == 4) return kThreads * kVecsPerLane / 4;  // four lanes per unit
    return kThreads * (128 / (k.P * k.vec));
  }
  return kThreads * kVecsPerLane;
}

hipError_t LaunchTiledCopy(const void* image_dev, uint32_t map_offset, uint32_t grid,
                           const TiledLaunchKey& key, hipStream_t stream) {
  if (grid == 0) return hipSuccess;
  const KernelFn fn = PickKernel(key);
  if (fn == nullptr) return hipErrorInvalidValue;
  const uint8_t* img = static_cast<const uint8_t*>(image_dev);
  // The bf16 Llama-3-8B set and a set of f32 matrices measured 1.3-3.4
  // points of HBM peak above no cap. The four-lane kernels' own LDS counts
  // towards the reservation.
  const bool quad = (key.mode == kDetileStd || key.mode == kTileStd) && key.lanes == 4;
  const bool pair = key.mode == kDetileStd && key.lanes == 2 && key.torder == 0;
  const uint32_t lds = kLdsPerCu / kWorkgroupsPerCu - (quad ? kQuadLdsBytes : 0) -
                       (pair ? kPairLdsBytes : 0);
  hipLaunchKernelGGL(fn, dim3(grid), dim3(kThreads), lds, stream, img, map_offset);
  return hipGetLastError();
}

}  // namespace kvx
