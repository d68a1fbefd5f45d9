#include "pool_layout.h"

#include <algorithm>
#include <limits>

namespace kvx {
namespace {

constexpr int64_t kMax = std::numeric_limits<int64_t>::max();
constexpr int64_t kMaxLiveSegments = int64_t{1} << 20;

// a * b and a + b for non-negative operands; false on overflow or a
// negative operand.
bool Mul(int64_t a, int64_t b, int64_t* out) {
  return a >= 0 && b >= 0 && !__builtin_mul_overflow(a, b, out);
}
bool Add(int64_t a, int64_t b, int64_t* out) {
  return a >= 0 && b >= 0 && !__builtin_add_overflow(a, b, out);
}

Status Overflow(const std::string& what) {
  return InvalidArgumentError(what + " overflows int64");
}

}  // namespace

int64_t RegionSpec::live_bytes() const {
  int64_t a = 0, b = 0;
  if (!Mul(unit_bytes, num_units, &a) || !Mul(a, units_per_stride, &b)) return kMax;
  return b;
}

int64_t RegionSpec::extent_end_bytes() const {
  if (num_units == 0) return offset_bytes;
  int64_t strided = 0, packed = 0, start = 0, end = 0;
  if (num_units < 0 || !Mul(num_units - 1, stride_bytes, &strided) ||
      !Mul(units_per_stride, unit_bytes, &packed) || !Add(offset_bytes, strided, &start) ||
      !Add(start, packed, &end)) {
    return kMax;
  }
  return end;
}

Status RegionSpec::Validate(int64_t slot_bytes) const {
  if (name.empty()) return InvalidArgumentError("region name must be non-empty");
  if (slot_bytes <= 0) return InvalidArgumentError("slot_bytes must be positive");
  const std::string r = "region " + name;
  if (offset_bytes < 0) return InvalidArgumentError(r + " offset_bytes must be >= 0");
  if (stride_bytes < 0) return InvalidArgumentError(r + " stride_bytes must be >= 0");
  if (unit_bytes < 0) return InvalidArgumentError(r + " unit_bytes must be >= 0");
  if (num_units < 0) return InvalidArgumentError(r + " num_units must be >= 0");
  if (units_per_stride <= 0) {
    return InvalidArgumentError(r + " units_per_stride must be positive");
  }
  if (num_units > 0 && unit_bytes <= 0) {
    return InvalidArgumentError(r + " unit_bytes must be positive");
  }
  if (num_units > 1 && stride_bytes <= 0) {
    return InvalidArgumentError(r + " stride_bytes must be positive");
  }
  int64_t packed = 0, span = 0, start = 0, end = 0;
  if (!Mul(units_per_stride, unit_bytes, &packed)) return Overflow(r + " packed unit bytes");
  if (num_units > 0 && stride_bytes < packed) {
    return InvalidArgumentError(r + " stride_bytes is smaller than packed units");
  }
  if (!Mul(num_units > 0 ? num_units - 1 : 0, stride_bytes, &span)) {
    return Overflow(r + " stride extent");
  }
  if (!Add(offset_bytes, span, &start)) return Overflow(r + " extent start");
  if (!Add(start, packed, &end)) return Overflow(r + " extent end");
  if (end > slot_bytes) {
    return InvalidArgumentError(r + " exceeds slot bytes: end=" + std::to_string(end) +
                                " slot=" + std::to_string(slot_bytes));
  }
  return OkStatus();
}

int64_t PoolSpec::storage_extent_end_bytes() const {
  if (base_offset_bytes < 0 || block_stride_bytes < 0 || num_blocks <= 0) return kMax;
  int64_t block_off = 0, last = 0, end = 0;
  if (!Mul(num_blocks - 1, block_stride_bytes, &block_off)) return kMax;
  int64_t live_end = 0;
  for (const RegionSpec& r : regions) live_end = std::max(live_end, r.extent_end_bytes());
  if (!Add(base_offset_bytes, block_off, &last) || !Add(last, live_end, &end)) return kMax;
  return end;
}

Status PoolSpec::Validate(int64_t storage_bytes) const {
  if (tag.empty()) return InvalidArgumentError("pool tag must be non-empty");
  const std::string p = "pool " + tag;
  if (block_stride_bytes <= 0) {
    return InvalidArgumentError(p + " block_stride_bytes must be positive");
  }
  if (num_blocks <= 0) return InvalidArgumentError(p + " num_blocks must be positive");
  if (base_offset_bytes < 0) {
    return InvalidArgumentError(p + " base_offset_bytes must be >= 0");
  }
  if (regions.empty()) return InvalidArgumentError(p + " must contain at least one region");
  for (const RegionSpec& r : regions) {
    Status st = r.Validate(block_stride_bytes);
    if (!st.ok()) return InvalidArgumentError(p + ": " + st.message());
  }
  if (storage_bytes >= 0) {
    const int64_t end = storage_extent_end_bytes();
    if (end == kMax) return InvalidArgumentError(p + " live storage extent overflows int64");
    if (end > storage_bytes) {
      return InvalidArgumentError(p + " exceeds storage bytes (live regions): end=" +
                                  std::to_string(end) + " storage=" +
                                  std::to_string(storage_bytes));
    }
  }
  return OkStatus();
}

bool RegionsCoverRange(const std::vector<RegionSpec>& regions, size_t start, size_t end) {
  // Walk a cursor through [start, end); each step jumps to the furthest end
  // of a packed run (of any region) containing the cursor.
  size_t cursor = start;
  while (cursor < end) {
    size_t next = cursor;
    for (const RegionSpec& r : regions) {
      if (r.num_units <= 0) continue;
      const size_t off = static_cast<size_t>(r.offset_bytes);
      const size_t stride = static_cast<size_t>(r.stride_bytes);
      const size_t packed = static_cast<size_t>(r.unit_bytes) *
                            static_cast<size_t>(r.units_per_stride);
      if (cursor < off || packed == 0) continue;
      size_t unit = 0;
      if (r.num_units > 1) {
        if (stride == 0) continue;
        unit = (cursor - off) / stride;
        if (unit >= static_cast<size_t>(r.num_units)) continue;
      }
      const size_t s = off + unit * stride;
      if (cursor < s || cursor >= s + packed) continue;
      next = std::max(next, std::min(s + packed, end));
    }
    if (next == cursor) return false;
    cursor = next;
  }
  return true;
}

StatusOr<std::vector<PoolBlockCopyExtent>> ComputePoolBlockCopyExtents(
    const PoolSpec& pool, const std::vector<int64_t>& block_ids) {
  const std::string p = "pool " + pool.tag;
  std::vector<PoolBlockCopyExtent> ext;
  for (int64_t id : block_ids) {
    if (id < 0 || id >= pool.num_blocks) {
      return OutOfRangeError(p + " block_id " + std::to_string(id) + " out of range [0, " +
                             std::to_string(pool.num_blocks) + ")");
    }
    int64_t delta = 0, base = 0;
    if (!Mul(id, pool.block_stride_bytes, &delta)) return Overflow(p + " block offset");
    if (!Add(pool.base_offset_bytes, delta, &base)) return Overflow(p + " block base");
    for (const RegionSpec& r : pool.regions) {
      const std::string rr = p + " region " + r.name;
      int64_t packed = 0;
      if (!Mul(r.unit_bytes, r.units_per_stride, &packed)) return Overflow(rr + " packed bytes");
      if (r.num_units == 0 || packed == 0) continue;
      int64_t rbase = 0;
      if (!Add(base, r.offset_bytes, &rbase)) return Overflow(rr + " offset");
      if (r.stride_bytes == packed) {
        // Abutting units: the region is one contiguous extent.
        int64_t bytes = 0;
        if (!Mul(r.num_units, packed, &bytes)) return Overflow(rr + " live bytes");
        ext.push_back({rbase, bytes});
        continue;
      }
      for (int64_t u = 0; u < r.num_units; ++u) {
        int64_t ud = 0, off = 0;
        if (!Mul(u, r.stride_bytes, &ud)) return Overflow(rr + " unit offset");
        if (!Add(rbase, ud, &off)) return Overflow(rr + " unit address");
        ext.push_back({off, packed});
      }
    }
  }
  std::sort(ext.begin(), ext.end(), [](const PoolBlockCopyExtent& a, const PoolBlockCopyExtent& b) {
    return a.offset_bytes != b.offset_bytes ? a.offset_bytes < b.offset_bytes
                                            : a.size_bytes < b.size_bytes;
  });
  std::vector<PoolBlockCopyExtent> merged;
  for (const PoolBlockCopyExtent& e : ext) {
    int64_t end = 0;
    if (!Add(e.offset_bytes, e.size_bytes, &end)) return Overflow(p + " copy extent end");
    if (!merged.empty()) {
      PoolBlockCopyExtent& prev = merged.back();
      const int64_t prev_end = prev.offset_bytes + prev.size_bytes;
      if (e.offset_bytes <= prev_end) {
        prev.size_bytes = std::max(prev_end, end) - prev.offset_bytes;
        continue;
      }
    }
    merged.push_back(e);
  }
  return merged;
}

StatusOr<std::vector<PoolLiveSegment>> ExpandPoolLiveSegments(const PoolSpec& pool) {
  const std::string p = "pool " + pool.tag;
  const int64_t stride = pool.block_stride_bytes;
  if (stride <= 0) return InvalidArgumentError(p + " has non-positive block stride");
  std::vector<std::pair<int64_t, int64_t>> runs;
  auto add_run = [&](int64_t start, int64_t end) -> Status {
    if (end > stride) {
      return InvalidArgumentError(p + " live region exceeds its block stride: end=" +
                                  std::to_string(end) + ", stride=" + std::to_string(stride));
    }
    runs.emplace_back(start, end);
    return OkStatus();
  };
  for (const RegionSpec& r : pool.regions) {
    if (r.offset_bytes < 0 || r.stride_bytes < 0 || r.unit_bytes < 0 || r.num_units < 0) {
      return InvalidArgumentError(p + " has negative region geometry");
    }
    if (r.units_per_stride <= 0) {
      return InvalidArgumentError(p + " has non-positive units_per_stride");
    }
    int64_t packed = 0;
    if (!Mul(r.unit_bytes, r.units_per_stride, &packed)) {
      return InvalidArgumentError(p + " region byte geometry overflows");
    }
    if (r.num_units > 0 && packed <= 0) return InvalidArgumentError(p + " has an empty live region");
    if (r.num_units > 1 && r.stride_bytes <= 0) {
      return InvalidArgumentError(p + " has a non-positive region stride");
    }
    if (r.num_units > 0 && r.stride_bytes < packed) {
      return InvalidArgumentError(p + " has overlapping units within one region");
    }
    if (static_cast<int64_t>(runs.size()) + r.num_units > kMaxLiveSegments) {
      return InvalidArgumentError(p + " exceeds the live-region expansion bound");
    }
    if (r.num_units > 0 && r.stride_bytes == packed) {
      int64_t bytes = 0;
      if (!Mul(r.num_units, packed, &bytes)) {
        return InvalidArgumentError(p + " region byte geometry overflows");
      }
      KVX_RETURN_IF_ERROR(add_run(r.offset_bytes, r.offset_bytes + bytes));
      continue;
    }
    for (int64_t u = 0; u < r.num_units; ++u) {
      int64_t ud = 0;
      if (!Mul(u, r.stride_bytes, &ud)) {
        return InvalidArgumentError(p + " region byte geometry overflows");
      }
      const int64_t s = r.offset_bytes + ud;
      KVX_RETURN_IF_ERROR(add_run(s, s + packed));
    }
  }
  std::sort(runs.begin(), runs.end());
  std::vector<std::pair<int64_t, int64_t>> phys;
  for (const auto& run : runs) {
    if (!phys.empty() && run.first < phys.back().second) {
      return InvalidArgumentError(p + " has overlapping live regions at byte " +
                                  std::to_string(run.first));
    }
    if (!phys.empty() && run.first == phys.back().second) {
      phys.back().second = run.second;
    } else {
      phys.push_back(run);
    }
  }
  std::vector<PoolLiveSegment> out;
  int64_t logical = 0;
  for (const auto& run : phys) {
    out.push_back({logical, run.first, run.second - run.first});
    logical += run.second - run.first;
  }
  return out;
}

StatusOr<std::pair<int64_t, int64_t>> PhysicalLiveRangeToLogical(
    const std::vector<PoolLiveSegment>& segments, int64_t physical_offset, int64_t size) {
  if (physical_offset < 0 || size <= 0) {
    return InvalidArgumentError("physical live range offset/size is invalid");
  }
  const int64_t end = physical_offset + size;
  for (const PoolLiveSegment& s : segments) {
    if (s.physical_offset <= physical_offset && end <= s.physical_offset + s.size) {
      const int64_t l = s.logical_offset + physical_offset - s.physical_offset;
      return std::make_pair(l, l + size);
    }
  }
  return InvalidArgumentError("physical range [" + std::to_string(physical_offset) + ", " +
                              std::to_string(end) +
                              ") crosses padding or lies outside declared live regions");
}

StatusOr<std::vector<LiveCopyChunk>> TranslateLiveCopy(
    const std::vector<PoolLiveSegment>& src, const std::vector<PoolLiveSegment>& dst,
    int64_t src_offset, int64_t dst_offset, int64_t size) {
  if (src_offset < 0 || dst_offset < 0 || size <= 0) {
    return InvalidArgumentError("Compact-live copy offsets/size are invalid");
  }
  // Physical position of a compact offset and the live bytes left in its run.
  auto locate = [](const std::vector<PoolLiveSegment>& segs,
                   int64_t logical) -> StatusOr<std::pair<int64_t, int64_t>> {
    for (const PoolLiveSegment& s : segs) {
      if (s.logical_offset <= logical && logical < s.logical_offset + s.size) {
        return std::make_pair(s.physical_offset + logical - s.logical_offset,
                              s.logical_offset + s.size - logical);
      }
    }
    return InvalidArgumentError("Compact-live offset " + std::to_string(logical) +
                                " is out of range");
  };
  std::vector<LiveCopyChunk> out;
  int64_t left = size, sc = src_offset, dc = dst_offset;
  while (left > 0) {
    KVX_ASSIGN_OR_RETURN(auto s, locate(src, sc));
    KVX_ASSIGN_OR_RETURN(auto d, locate(dst, dc));
    const int64_t n = std::min({left, s.second, d.second});
    out.push_back({s.first, d.first, n});
    if (static_cast<int64_t>(out.size()) > kMaxLiveSegments) {
      return InvalidArgumentError("Compact-live copy exceeds the segment expansion bound");
    }
    sc += n;
    dc += n;
    left -= n;
  }
  return out;
}

}  // namespace kvx
