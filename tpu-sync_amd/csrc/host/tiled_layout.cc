#include "tiled_layout.h"

#include <algorithm>
#include <cstring>

#include "hip_util.h"

namespace kvx {
namespace {

constexpr int kMaxTiles = 4;
constexpr int64_t kU32Limit = int64_t{1} << 32;
constexpr int64_t kDivLimit = int64_t{1} << 31;  // FastDivU32 divisors

bool MulOk(int64_t a, int64_t b, int64_t* out) { return !__builtin_mul_overflow(a, b, out); }

int64_t CeilDiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// One dimension of a shape while the tiles are applied: the logical
// dimension it indexes (-1: a padded leading 1), the divisions / modulos
// applied to that index so far, and its size.
struct WorkDim {
  int src = -1;
  std::vector<std::pair<bool, int64_t>> ops;  // (is_mod, divisor)
  int64_t size = 1;
};

// The physical-order shape the tiles apply to (tiling_utils.cc:911-921):
// rank 1 becomes (1, d0); higher ranks are permuted major-to-minor.
std::vector<WorkDim> PhysicalOrder(const TiledLayout& l) {
  const int r = static_cast<int>(l.dims.size());
  std::vector<WorkDim> cur;
  if (r == 1) {
    cur.push_back(WorkDim{});
    WorkDim d;
    d.src = 0;
    d.size = l.dims[0];
    cur.push_back(d);
  } else {
    for (int i = r - 1; i >= 0; --i) {
      WorkDim d;
      d.src = l.minor_to_major[i];
      d.size = l.dims[d.src];
      cur.push_back(d);
    }
  }
  return cur;
}

// Applies every tile (tiling_utils.cc:923-950): a tile of rank k splits the
// k minor-most dimensions into (ceil(d / t)) and (t) parts; a tile of larger
// rank than the shape first pads it with leading 1s.
std::vector<WorkDim> ApplyTiles(const TiledLayout& l) {
  std::vector<WorkDim> cur = PhysicalOrder(l);
  for (const std::vector<int64_t>& tile : l.tiles) {
    const size_t k = tile.size();
    if (k > cur.size()) cur.insert(cur.begin(), k - cur.size(), WorkDim{});
    const size_t start = cur.size() - k;
    std::vector<WorkDim> next(cur.begin(), cur.begin() + start);
    for (size_t i = 0; i < k; ++i) {
      WorkDim d = cur[start + i];
      d.ops.push_back({false, tile[i]});
      d.size = CeilDiv(d.size, tile[i]);
      next.push_back(d);
    }
    for (size_t i = 0; i < k; ++i) {
      WorkDim d = cur[start + i];
      d.ops.push_back({true, tile[i]});
      d.size = tile[i];
      next.push_back(d);
    }
    cur.swap(next);
  }
  return cur;
}

// Standard-form units run in tiled order when tiling (each workgroup writes
// one contiguous span of the tiled buffer, padding included) and in linear
// order when detiling (each workgroup writes whole rows of the linear
// image). On the Llama-3-8B set in T(8,128)(2,1), one process, one launch
// each: tiling 79.2 % of HBM peak in tiled order against 78.2 % in linear
// order, detiling 77.0 % in linear order against 75.4 %.

int WidestVector(uint64_t acc, int cap) {
  for (int v = cap; v > 1; v /= 2) {
    if ((acc & static_cast<uint64_t>(v - 1)) == 0) return v;
  }
  return 1;
}

}  // namespace

Status ValidateTiledLayout(const TiledLayout& l) {
  if (l.itemsize != 1 && l.itemsize != 2 && l.itemsize != 4 && l.itemsize != 8) {
    return InvalidArgumentError("tiled layout: itemsize must be 1, 2, 4 or 8");
  }
  const size_t r = l.dims.size();
  if (r > static_cast<size_t>(kTiledMaxRank)) {
    return InvalidArgumentError("tiled layout: at most 8 dimensions");
  }
  if (l.minor_to_major.size() != r) {
    return InvalidArgumentError("tiled layout: minor_to_major needs one entry per dimension");
  }
  std::vector<bool> seen(r, false);
  for (int m : l.minor_to_major) {
    if (m < 0 || static_cast<size_t>(m) >= r || seen[m]) {
      return InvalidArgumentError("tiled layout: minor_to_major is not a permutation");
    }
    seen[m] = true;
  }
  for (int64_t d : l.dims) {
    if (d < 0) return InvalidArgumentError("tiled layout: negative dimension");
  }
  if (l.tiles.size() > static_cast<size_t>(kMaxTiles)) {
    return InvalidArgumentError("tiled layout: at most 4 tiles");
  }
  for (const std::vector<int64_t>& t : l.tiles) {
    if (t.empty() || t.size() > static_cast<size_t>(kTiledMaxRank)) {
      return InvalidArgumentError("tiled layout: a tile has 1 to 8 dimensions");
    }
    for (int64_t d : t) {
      if (d < 1) {
        return InvalidArgumentError(
            "tiled layout: tile dimensions must be >= 1 (combined dimensions are not supported)");
      }
    }
  }
  return OkStatus();
}

int64_t LogicalElements(const TiledLayout& l) {
  int64_t n = 1;
  for (int64_t d : l.dims) {
    if (!MulOk(n, d, &n)) return -1;
  }
  return n;
}

StatusOr<int64_t> TiledBufferElements(const TiledLayout& l) {
  KVX_RETURN_IF_ERROR(ValidateTiledLayout(l));
  if (l.dims.empty()) return int64_t{1};
  int64_t n = 1;
  for (const WorkDim& d : ApplyTiles(l)) {
    if (!MulOk(n, d.size, &n)) return InvalidArgumentError("tiled layout: size overflows");
  }
  return n;
}

int64_t TiledPlan::CutAtOrBelow(int64_t x) const {
  if (x <= 0) return 0;
  if (x >= logical_bytes) return logical_bytes;
  const int64_t s = layout.itemsize;
  if (!tiled) return x;
  if (!standard) return x / s * s;
  const int64_t row_bytes = static_cast<int64_t>(W) * s;
  const int64_t row = x / row_bytes;
  const int64_t b = row / static_cast<int64_t>(H);
  const int64_t h = row % static_cast<int64_t>(H);
  const int64_t th = static_cast<int64_t>(tH);
  return (b * static_cast<int64_t>(H) + h / th * th) * row_bytes;
}

StatusOr<TiledPlan> PlanTiled(const TiledLayout& l) {
  KVX_RETURN_IF_ERROR(ValidateTiledLayout(l));
  TiledPlan p;
  p.layout = l;
  const int64_t s = l.itemsize;
  const int64_t logical = LogicalElements(l);
  if (logical < 0 || !MulOk(logical, s, &p.logical_bytes)) {
    return InvalidArgumentError("tiled layout: size overflows");
  }
  KVX_ASSIGN_OR_RETURN(int64_t phys, TiledBufferElements(l));
  const int r = static_cast<int>(l.dims.size());
  p.tiled = !l.tiles.empty() && r > 0;
  if (!p.tiled) {
    p.tiled_bytes = p.logical_bytes;
    return p;
  }
  if (!MulOk(phys, s, &p.tiled_bytes)) return InvalidArgumentError("tiled layout: size overflows");
  p.padded = phys > logical;
  p.zero_vec = WidestVector(static_cast<uint64_t>(p.tiled_bytes), 16);
  if (logical == 0) return p;

  // Standard form: the reference's IsStandardRowMajorTiled
  // (tiling_utils.cc:56-82) plus this kernel's own limits.
  bool standard = true;
  for (int i = 0; i < r; ++i) standard = standard && l.minor_to_major[i] == r - 1 - i;
  uint32_t P = 1;
  if (l.tiles.size() == 1) {
    standard = standard && l.tiles[0].size() == 2;
  } else if (l.tiles.size() == 2) {
    standard = standard && l.tiles[0].size() == 2 && l.tiles[1].size() == 2 &&
               l.tiles[1][1] == 1 && (l.tiles[1][0] == 2 || l.tiles[1][0] == 4) &&
               l.tiles[0][0] % l.tiles[1][0] == 0;
    if (standard) {
      P = static_cast<uint32_t>(l.tiles[1][0]);
      standard = P * s == 4;
    }
  } else {
    standard = false;
  }
  if (standard) {
    const uint64_t W = static_cast<uint64_t>(l.dims[r - 1]);
    const uint64_t H = r == 1 ? 1 : static_cast<uint64_t>(l.dims[r - 2]);
    const uint64_t B = static_cast<uint64_t>(logical) / (W * H);
    const int64_t tH = l.tiles[0][0], tW = l.tiles[0][1];
    const int vec = WidestVector(static_cast<uint64_t>(W * s) | static_cast<uint64_t>(tW * s), 16);
    const uint64_t ng = (H + P - 1) / P;
    const uint64_t ncv = W * s / vec;
    int64_t units = 0;
    standard = H < static_cast<uint64_t>(kDivLimit) && W < static_cast<uint64_t>(kDivLimit) &&
               tH <= kDivLimit && tW <= kDivLimit && (P == 1 || vec >= 4) &&
               MulOk(static_cast<int64_t>(B * ng), static_cast<int64_t>(ncv), &units) &&
               units < kU32Limit && B * ng < static_cast<uint64_t>(kU32Limit) &&
               B * H < static_cast<uint64_t>(kU32Limit) && tH * tW < kDivLimit &&
               p.tiled_bytes / (static_cast<int64_t>(P) * vec) < kU32Limit;
    if (standard) {
      p.standard = true;
      p.P = P;
      p.B = B;
      p.H = H;
      p.W = W;
      p.tH = static_cast<uint64_t>(tH);
      p.tW = static_cast<uint64_t>(tW);
      p.nT0 = (H + p.tH - 1) / p.tH;
      p.nT1 = (W + p.tW - 1) / p.tW;
      p.vec = vec;
    }
  }

  // General form (also the fallback of a standard layout whose buffers are
  // too poorly aligned for its vectors): the final shape's dimensions.
  std::vector<WorkDim> fin = ApplyTiles(l);
  bool gen_ok = logical < kU32Limit && fin.size() <= static_cast<size_t>(kTiledMaxGenDims);
  for (int64_t d : l.dims) gen_ok = gen_ok && d <= kDivLimit;
  for (const auto& t : l.tiles) {
    for (int64_t d : t) gen_ok = gen_ok && d <= kDivLimit;
  }
  if (gen_ok) {
    int64_t stride = 1;
    p.gen.resize(fin.size());
    for (int k = static_cast<int>(fin.size()) - 1; k >= 0; --k) {
      TiledGenDim g{};
      g.src = fin[k].src;
      g.nops = static_cast<uint32_t>(fin[k].ops.size());
      for (size_t o = 0; o < fin[k].ops.size(); ++o) {
        if (fin[k].ops[o].first) g.is_mod |= 1u << o;
        g.op[o] = MakeFastDivU32(static_cast<uint32_t>(fin[k].ops[o].second));
      }
      g.stride = static_cast<uint64_t>(stride);
      p.gen[k] = g;
      stride *= fin[k].size;
    }
  } else if (!p.standard) {
    return UnimplementedError(
        "tiled layout: general layouts need fewer than 2^32 elements, dimensions and tiles "
        "of at most 2^31 and at most 16 tiled dimensions");
  }
  return p;
}

// Whether the standard form's units at vector width v stay within the
// kernels' 32-bit unit indices and FastDivU32 divisors: linear order counts
// B * ceil(H / P) * (W * s / v) units, tiled order tiled_bytes / (P * v).
static bool StdUnitsFit(const TiledPlan& p, int v, bool tile) {
  if (v <= 0) return false;
  const uint64_t s = static_cast<uint64_t>(p.layout.itemsize);
  const uint64_t ng = (p.H + p.P - 1) / p.P;
  const uint64_t ncv = p.W * s / static_cast<uint64_t>(v);
  uint64_t units = 0;
  if (ncv >= static_cast<uint64_t>(kDivLimit) || ng >= static_cast<uint64_t>(kDivLimit) ||
      __builtin_mul_overflow(p.B * ng, ncv, &units) ||
      units >= static_cast<uint64_t>(kU32Limit)) {
    return false;
  }
  if (tile) {
    const uint64_t ncvt = p.tW * s / static_cast<uint64_t>(v);
    const uint64_t tunits = static_cast<uint64_t>(p.tiled_bytes) / (p.P * static_cast<uint64_t>(v));
    if (ncvt >= static_cast<uint64_t>(kDivLimit) || tunits >= static_cast<uint64_t>(kU32Limit)) {
      return false;
    }
  }
  return true;
}

Status AppendTiledJobs(const TiledPlan& p, uint64_t tiled, uint64_t linear, int64_t lo,
                       int64_t hi, bool tile, bool zero_pass, std::vector<TiledJob>* zero,
                       std::vector<TiledJob>* jobs) {
  if (!p.tiled || lo >= hi) return OkStatus();
  if (lo < 0 || hi > p.logical_bytes || p.CutAtOrBelow(lo) != lo ||
      p.CutAtOrBelow(hi) != hi) {
    return InvalidArgumentError("tiled copy range does not start and end on a tile row");
  }
  if (tiled == 0) return InvalidArgumentError("tiled copy: null tiled buffer");
  const int64_t s = p.layout.itemsize;
  // Both forms address whole elements: a buffer that is not aligned to the
  // element size would give the vector form fewer bytes per vector than one
  // element (no element per vector at all).
  if (((tiled | linear) & static_cast<uint64_t>(s - 1)) != 0) {
    return InvalidArgumentError("tiled copy: buffers not aligned to the element size");
  }
  // Units need vectors aligned on both buffers; a packed layout whose
  // buffers allow less than 4 bytes goes element by element.
  int v = WidestVector(tiled | linear, p.vec);
  // Packed units: one lane per unit with units of one 16-byte tiled vector
  // (v = 16 / P), except that detiling at 16-byte rows goes two lanes per
  // unit for pairs (P = 2) and four for quads (P = 4), exchanging through
  // LDS so that each wave writes 1 KiB of one row per store. Measured on the
  // Llama-3-8B set (bf16, P = 2), one process, one launch each: tiling
  // 79.2 % of HBM peak at v = 8 against 76.7 % with two lanes per 16-byte
  // unit and 67.8 % with one lane per 16-byte unit (each 16-byte tiled store
  // of a wave then leaves 16-byte holes); detiling 77.0 % with two lanes
  // (exchanging within the lane pair) against 75.7 % at v = 8, and 79.6
  // against 78.4 % for the LDS exchange over the lane-pair one. For int8
  // (P = 4) at 16-byte rows, detiling: 71.6 % through LDS against 61.8 % for
  // one lane per 16-byte tiled vector; tiling keeps one lane per tiled
  // vector (72.3 % against 67.0 % through LDS).
  bool two_lanes = false, four_lanes = false;
  if (p.P == 2 && !tile && v == 16) {
    two_lanes = true;
  } else if (p.P == 4 && !tile && v == 16) {
    four_lanes = true;
  } else if (p.P > 1) {
    v = std::min(v, 16 / static_cast<int>(p.P));
  }
  // PlanTiled checked the 32-bit unit and divisor limits at the plan's widest
  // vector; narrower buffers multiply the unit counts, so they are checked
  // again at the width chosen here (the kernels index units in 32 bits).
  bool use_std = p.standard && (p.P == 1 || v >= 4);
  if (use_std && !StdUnitsFit(p, v, tile)) use_std = false;
  if (!use_std && p.standard && p.gen.empty()) {
    return UnimplementedError(
        "tiled copy: this layout has more 32-bit-indexed units than one launch can address "
        "at the buffers' alignment");
  }
  const bool tiled_order = use_std && tile;
  // Tiled-order units write the padding themselves; otherwise it is cleared
  // first.
  if (tile && zero_pass && p.padded && !tiled_order) {
    const int v = WidestVector(tiled, p.zero_vec);
    TiledJob z;
    z.vec = v;
    z.dev.mode = kZero;
    z.dev.tiled = tiled;
    z.dev.lo = 0;
    z.dev.count = static_cast<uint64_t>(p.tiled_bytes / v);
    z.dev.itemsize = static_cast<uint32_t>(s);
    z.dev.P = 1;
    zero->push_back(z);
  }
  TiledJob j;
  j.dev.tiled = tiled;
  j.dev.linear = linear;
  j.dev.itemsize = static_cast<uint32_t>(s);
  if (use_std) {
    const uint64_t row_bytes = p.W * s;
    const uint64_t ng = (p.H + p.P - 1) / p.P;
    const uint64_t ncv = row_bytes / v;
    auto group = [&](int64_t x) -> uint64_t {
      if (x >= p.logical_bytes) return p.B * ng;
      const uint64_t row = static_cast<uint64_t>(x) / row_bytes;
      return row / p.H * ng + row % p.H / p.P;
    };
    j.vec = v;
    j.dev.mode = tile ? kTileStd : kDetileStd;
    j.dev.lanes_per_unit = two_lanes ? 2 : four_lanes ? 4 : 1;
    j.dev.sliced = two_lanes || four_lanes ? 1u : 0u;
    if (tiled_order) {
      // Whole tile rows (cuts fall on them): units of tile rows [t_lo, t_hi).
      auto tile_row = [&](int64_t x) -> uint64_t {
        if (x >= p.logical_bytes) return p.B * p.nT0;
        const uint64_t row = static_cast<uint64_t>(x) / row_bytes;
        return row / p.H * p.nT0 + row % p.H / p.tH;
      };
      const uint64_t gpt = p.tH / p.P;
      const uint64_t ncvt = p.tW * s / v;
      const uint64_t per_tile_row = p.nT1 * gpt * ncvt;
      const uint64_t t_lo = tile_row(lo), t_hi = tile_row(hi);
      j.dev.torder = 1;
      j.dev.lo = t_lo * per_tile_row;
      j.dev.count = (t_hi - t_lo) * per_tile_row;
      j.dev.t_ncv = MakeFastDivU32(static_cast<uint32_t>(ncvt));
      j.dev.t_gpt = MakeFastDivU32(static_cast<uint32_t>(gpt));
      j.dev.t_nt1 = MakeFastDivU32(static_cast<uint32_t>(p.nT1));
      j.dev.t_nt0 = MakeFastDivU32(static_cast<uint32_t>(p.nT0));
    } else {
      const uint64_t g_lo = group(lo), g_hi = group(hi);
      j.dev.lo = g_lo * ncv;
      j.dev.count = (g_hi - g_lo) * ncv;
    }
    j.dev.P = p.P;
    j.dev.ncv = MakeFastDivU32(static_cast<uint32_t>(ncv));
    j.dev.ng = MakeFastDivU32(static_cast<uint32_t>(ng));
    j.dev.th = MakeFastDivU32(static_cast<uint32_t>(p.tH));
    j.dev.tw = MakeFastDivU32(static_cast<uint32_t>(p.tW));
    j.dev.h32 = static_cast<uint32_t>(p.H);
    j.dev.w32 = static_cast<uint32_t>(p.W);
    j.dev.nt0 = static_cast<uint32_t>(p.nT0);
    j.dev.nt1 = static_cast<uint32_t>(p.nT1);
    j.dev.tile_elems = static_cast<uint32_t>(p.tH * p.tW);
    j.dev.log2s = static_cast<uint32_t>(__builtin_ctz(static_cast<unsigned>(s)));
  } else {
    if (p.gen.empty()) {
      return UnimplementedError("tiled copy: buffers not aligned for this layout's vectors");
    }
    if (((tiled | linear) & static_cast<uint64_t>(s - 1)) != 0) {
      return InvalidArgumentError("tiled copy: buffers not aligned to the element size");
    }
    j.vec = 0;
    j.dev.mode = tile ? kTileGen : kDetileGen;
    j.dev.lo = static_cast<uint64_t>(lo / s);
    j.dev.count = static_cast<uint64_t>((hi - lo) / s);
    j.dev.P = 1;
    j.dev.rank = static_cast<uint32_t>(p.layout.dims.size());
    for (size_t r = 0; r < p.layout.dims.size(); ++r) {
      j.dev.dims[r] = MakeFastDivU32(static_cast<uint32_t>(p.layout.dims[r]));
    }
    j.dev.ngen = static_cast<uint32_t>(p.gen.size());
    j.gen = p.gen;
  }
  if (j.dev.count > 0) jobs->push_back(std::move(j));
  return OkStatus();
}

Status LaunchTiledThroughRing(ArgRing& ring, const std::vector<TiledJob>& jobs,
                              hipStream_t stream, hipEvent_t kernel_start) {
  if (jobs.empty()) return OkStatus();
  // One launch per kernel (vector width, rows per unit, direction, unit
  // order; element size for the general form), in order of first
  // appearance. General jobs take any vector width.
  std::vector<TiledLaunchKey> keys;
  std::vector<TiledLaunchKey> job_key(jobs.size());
  for (size_t i = 0; i < jobs.size(); ++i) {
    job_key[i] = LaunchKeyOf(jobs[i].dev, jobs[i].vec);
    if (std::find(keys.begin(), keys.end(), job_key[i]) == keys.end()) {
      keys.push_back(job_key[i]);
    }
  }
  bool started = false;
  for (const TiledLaunchKey& key : keys) {
    std::vector<const TiledJob*> mine;
    for (size_t i = 0; i < jobs.size(); ++i) {
      if (job_key[i] == key) mine.push_back(&jobs[i]);
    }
    const uint64_t per = TiledPerWorkgroup(key);
    const int64_t head = static_cast<int64_t>(mine.size() * sizeof(TiledJobDev));
    int64_t gen_bytes = 0;
    uint64_t grid = 0;
    for (const TiledJob* j : mine) {
      gen_bytes += static_cast<int64_t>(j->gen.size() * sizeof(TiledGenDim));
      grid += (j->dev.count + per - 1) / per;
    }
    if (grid >= (uint64_t{1} << 31)) return InvalidArgumentError("tiled copy too large for one launch");
    const int64_t map_off = head + gen_bytes;
    const int64_t bytes = map_off + static_cast<int64_t>(grid) * 4;
    KVX_ASSIGN_OR_RETURN(int64_t off, ring.Alloc(bytes));
    ArgSliceGuard keep([&ring, off, bytes, stream] { return ring.Commit(off, bytes, stream); },
                       stream);
    uint8_t* img = ring.host(off);
    uint32_t* map = reinterpret_cast<uint32_t*>(img + map_off);
    int64_t gen_at = head;
    uint32_t wg = 0;
    for (size_t i = 0; i < mine.size(); ++i) {
      TiledJobDev d = mine[i]->dev;
      d.wg_begin = wg;
      if (!mine[i]->gen.empty()) {
        d.gen_offset = static_cast<uint32_t>(gen_at);
        const size_t gb = mine[i]->gen.size() * sizeof(TiledGenDim);
        std::memcpy(img + gen_at, mine[i]->gen.data(), gb);
        gen_at += static_cast<int64_t>(gb);
      }
      std::memcpy(img + i * sizeof(TiledJobDev), &d, sizeof(d));
      const uint32_t n = static_cast<uint32_t>((d.count + per - 1) / per);
      for (uint32_t k = 0; k < n; ++k) map[wg + k] = static_cast<uint32_t>(i);
      wg += n;
    }
    KVX_RETURN_IF_ERROR(ring.Upload(off, bytes, stream));
    if (kernel_start != nullptr && !started) {
      KVX_HIP_RETURN_IF_ERROR(hipEventRecord(kernel_start, stream));
    }
    started = true;
    KVX_HIP_RETURN_IF_ERROR(LaunchTiledCopy(reinterpret_cast<const void*>(ring.dev(off)),
                                            static_cast<uint32_t>(map_off),
                                            static_cast<uint32_t>(grid), key, stream));
    KVX_RETURN_IF_ERROR(keep.Commit());
  }
  return OkStatus();
}

}  // namespace kvx
