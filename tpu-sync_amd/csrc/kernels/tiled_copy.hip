// Tiled-layout copy for gfx950 (MI355X): tile / detile of XLA-style tiled
// tensor layouts on the device, the work the reference's TileBuffer /
// DetileBuffer do on the host CPU (tpu_sync/weight_sync/tiling_utils.cc:
// 545-1036) before or after a raw DMA of the tiled bytes.
//
// Pure data movement, bound by HBM bandwidth. Standard-form jobs move units
// of P rows x V bytes: a lane issues all loads of its units (8 / P units,
// 8 V-byte vectors in flight) before its stores, so a workgroup keeps 32 KiB
// in flight at V = 16 like the other copy kernels. Reads and writes are both
// contiguous across the lanes of a wave: consecutive lanes take consecutive
// column vectors of the same rows, which are consecutive in the linear image
// and consecutive P * V-byte pieces of one tile row group in the tiled
// buffer. Packed layouts (P = 2 for 16-bit, P = 4 for 8-bit elements)
// interleave the P rows in registers with 32-bit shifts and masks.
// Divisions by layout constants use multiply-high (FastDivU32). Loads and
// stores are non-temporal (every byte is touched once).
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

// Addresses of a standard-form unit: the tiled piece and the linear row of
// its first row (row k is k * W * itemsize further); *h = its first row.
__device__ __forceinline__ void unit_addr(const KVX_CONST TiledJobDev* j, uint32_t u,
                                          uint32_t P, uint32_t E, uint64_t* tiled,
                                          uint64_t* lin, uint32_t* h, uint32_t* b_out) {
  const uint32_t q = fdiv(&j->ncv, u);
  const uint32_t cv = u - q * j->ncv.d;
  const uint32_t b = fdiv(&j->ng, q);
  const uint32_t g = q - b * j->ng.d;
  const uint32_t row = g * P;
  const uint32_t tr = fdiv(&j->th, row);
  const uint32_t r0 = row - tr * j->th.d;
  const uint32_t c = cv * E;
  const uint32_t tc = fdiv(&j->tw, c);
  const uint32_t cc = c - tc * j->tw.d;
  const uint64_t s = j->itemsize;
  const uint64_t tile = (static_cast<uint64_t>(b) * j->nT0 + tr) * j->nT1 + tc;
  *tiled = j->tiled + ((tile * j->th.d + r0) * j->tw.d + static_cast<uint64_t>(cc) * P) * s;
  *lin = j->linear + ((static_cast<uint64_t>(b) * j->H + row) * j->W + c) * s;
  *h = row;
  *b_out = b;
}

// Standard form, P = 1: each unit is one V-byte vector on both sides.
template <int V>
__device__ __forceinline__ void std_p1(const KVX_CONST TiledJobDev* j, uint32_t local, bool tile) {
  constexpr int U = kVecsPerLane;
  const uint32_t E = V / j->itemsize;
  const uint64_t first = j->lo + static_cast<uint64_t>(local) * (kThreads * U);
  const uint64_t end = j->lo + j->count;
  typename VecT<V>::T r[U];
  uint64_t dst[U];
#pragma unroll
  for (int i = 0; i < U; ++i) {
    uint64_t u = first + threadIdx.x + i * kThreads;
    u = u < end ? u : end - 1;
    uint64_t ta, la;
    uint32_t h, b;
    unit_addr(j, static_cast<uint32_t>(u), 1, E, &ta, &la, &h, &b);
    r[i] = ld<V>(tile ? la : ta);
    dst[i] = tile ? ta : la;
  }
#pragma unroll
  for (int i = 0; i < U; ++i) {
    if (first + threadIdx.x + i * kThreads < end) st<V>(dst[i], r[i]);
  }
}

// Standard form, P = 2 or 4: a unit is P rows x V bytes.
template <int V, int P>
__device__ __forceinline__ void std_packed(const KVX_CONST TiledJobDev* j, uint32_t local,
                                           bool tile) {
  constexpr int U = kVecsPerLane / P;
  constexpr int n = V / 4;
  constexpr uint32_t E = V * P / 4;  // elements per row vector (P * itemsize = 4)
  const uint64_t first = j->lo + static_cast<uint64_t>(local) * (kThreads * U);
  const uint64_t end = j->lo + j->count;
  const uint64_t row_bytes = j->W * j->itemsize;
  const uint32_t H = static_cast<uint32_t>(j->H);
  uint32_t words[U][P * n];
  uint64_t ta[U], la[U];
  uint32_t h[U];
#pragma unroll
  for (int i = 0; i < U; ++i) {
    uint64_t u = first + threadIdx.x + i * kThreads;
    u = u < end ? u : end - 1;
    uint32_t b;
    unit_addr(j, static_cast<uint32_t>(u), P, E, &ta[i], &la[i], &h[i], &b);
    if (tile) {
      // Rows past the matrix's end are padding: read a valid row, store 0.
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
    if (tile) {
      uint32_t rows[P][n];
#pragma unroll
      for (int k = 0; k < P; ++k) {
        const bool valid = h[i] + k < H;
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
        if (h[i] + k < H) st<V>(la[i] + k * row_bytes, from_words<V>(rows[k]));
      }
    }
  }
}

template <int V>
__device__ __forceinline__ void zero_job(const KVX_CONST TiledJobDev* j, uint32_t local) {
  const uint64_t first = j->lo + static_cast<uint64_t>(local) * (kThreads * kVecsPerLane);
  const uint64_t end = j->lo + j->count;
  typename VecT<V>::T z{};
#pragma unroll
  for (int i = 0; i < kVecsPerLane; ++i) {
    const uint64_t x = first + threadIdx.x + i * kThreads;
    if (x < end) st<V>(j->tiled + x * V, z);
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
#pragma unroll
  for (int k = 0; k < kTiledMaxGenDims; ++k) {
    if (k >= static_cast<int>(j->ngen)) break;
    const int32_t src = gd[k].src;
    uint32_t x = 0;
#pragma unroll
    for (int r = 0; r < kTiledMaxRank; ++r) x = src == r ? idx[r] : x;
#pragma unroll
    for (int o = 0; o < kTiledMaxOps; ++o) {
      if (o >= static_cast<int>(gd[k].nops)) break;
      const uint32_t q = fdiv(&gd[k].op[o], x);
      x = (gd[k].is_mod >> o) & 1u ? x - q * gd[k].op[o].d : q;
    }
    phys += static_cast<uint64_t>(x) * gd[k].stride;
  }
  return phys;
}

template <typename T>
__device__ __forceinline__ void gen_job(const KVX_CONST TiledJobDev* j,
                                        const KVX_CONST TiledGenDim* gd, uint32_t local,
                                        bool tile) {
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
    v[i] = *(const KVX_GLOBAL T*)(tile ? la : ta);
    dst[i] = tile ? ta : la;
  }
#pragma unroll
  for (int i = 0; i < U; ++i) {
    if (first + threadIdx.x + i * kThreads < end) *(KVX_GLOBAL T*)dst[i] = v[i];
  }
}

template <int V>
__global__ __launch_bounds__(kThreads) void tiled_copy_kernel(const uint8_t* image,
                                                              uint32_t map_offset) {
  const uint32_t wg = blockIdx.x;
  const uint32_t ji = ((const KVX_CONST uint32_t*)(image + map_offset))[wg];
  const KVX_CONST TiledJobDev* j = (const KVX_CONST TiledJobDev*)image + ji;
  const uint32_t local = wg - j->wg_begin;
  const uint32_t mode = j->mode;
  if (mode == kZero) {
    zero_job<V>(j, local);
  } else if (mode == kDetileStd || mode == kTileStd) {
    const bool tile = mode == kTileStd;
    if constexpr (V >= 4) {
      if (j->P == 2) {
        std_packed<V, 2>(j, local, tile);
        return;
      }
      if (j->P == 4) {
        std_packed<V, 4>(j, local, tile);
        return;
      }
    }
    std_p1<V>(j, local, tile);
  } else {
    const bool tile = mode == kTileGen;
    const KVX_CONST TiledGenDim* gd = (const KVX_CONST TiledGenDim*)(image + j->gen_offset);
    switch (j->itemsize) {
      case 1: gen_job<uint8_t>(j, gd, local, tile); break;
      case 2: gen_job<uint16_t>(j, gd, local, tile); break;
      case 4: gen_job<uint32_t>(j, gd, local, tile); break;
      default: gen_job<uint64_t>(j, gd, local, tile); break;
    }
  }
}

}  // namespace

uint32_t TiledJobPerWorkgroup(const TiledJobDev& j) {
  if (j.mode == kDetileStd || j.mode == kTileStd) {
    return kThreads * (kVecsPerLane / (j.P == 0 ? 1 : j.P));
  }
  return kThreads * kVecsPerLane;
}

hipError_t LaunchTiledCopy(const void* image_dev, uint32_t n, uint32_t map_offset,
                           uint32_t grid, int vec_bytes, hipStream_t stream) {
  (void)n;
  if (grid == 0) return hipSuccess;
  const uint8_t* img = static_cast<const uint8_t*>(image_dev);
  const uint32_t lds = kLdsPerCu / kWorkgroupsPerCu;
  switch (vec_bytes) {
    case 16:
      hipLaunchKernelGGL(tiled_copy_kernel<16>, dim3(grid), dim3(kThreads), lds, stream, img, map_offset);
      break;
    case 8:
      hipLaunchKernelGGL(tiled_copy_kernel<8>, dim3(grid), dim3(kThreads), lds, stream, img, map_offset);
      break;
    case 4:
      hipLaunchKernelGGL(tiled_copy_kernel<4>, dim3(grid), dim3(kThreads), lds, stream, img, map_offset);
      break;
    case 2:
      hipLaunchKernelGGL(tiled_copy_kernel<2>, dim3(grid), dim3(kThreads), lds, stream, img, map_offset);
      break;
    case 1:
      hipLaunchKernelGGL(tiled_copy_kernel<1>, dim3(grid), dim3(kThreads), lds, stream, img, map_offset);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace kvx
