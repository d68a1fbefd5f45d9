"""ORACLE -- test infrastructure only.

Pure-Python restatement of the byte-level pool geometry
(tpu_sync/kv_cache/pool_layout.cc), for small pools:

  region_extent_end    RegionSpec::extent_end_bytes (pool_layout.cc:100-126):
                       offset + (num_units - 1) * stride + units_per_stride *
                       unit_bytes, or offset when there are no units.
  storage_extent_end   PoolSpec::storage_extent_end_bytes (:231-254): base +
                       (num_blocks - 1) * block_stride + the largest region
                       extent end.
  copy_extents         ComputePoolBlockCopyExtents (:275-379): per block id,
                       one extent per abutting region (stride == packed) or
                       one per unit, at base + id * block_stride + region
                       offset (+ unit * stride); sorted by (offset, size) and
                       merged when an extent starts at or before the end of
                       the previous one.
  live_segments        ExpandPoolLiveSegments (:381-480): the runs of one
                       block, sorted; overlap is an error, abutting runs
                       merge; each run gets the compact (logical) offset of
                       the live bytes before it.
  physical_to_logical  PhysicalLiveRangeToLogical (:482-503): the range must
                       lie inside one run.
  translate_live_copy  TranslateLiveCopy (:555-602): walk source and
                       destination compact offsets together, cutting a chunk
                       at every run boundary of either side.
  regions_cover_range  RegionsCoverRange (:256-273) with RegionCoversOffset
                       (:64-87): a cursor advances to the furthest end of a
                       packed run containing it.

Regions are tuples (name, offset, stride, unit_bytes, num_units,
units_per_stride); a pool is a dict with keys tag, base, block_stride,
num_blocks, regions.

Parity status: every function is pinned by the known answers of the
reference's pool_layout_test.cc (tests/golden/pool_cases.json) and by brute
force over a byte mask of the live bytes (tests/test_pool_layout.py), which
fixes extents, segments, overlap detection and chunk boundaries
independently of the restated walk.
"""


class PoolError(ValueError):
    pass


def packed(region):
    return region[3] * region[5]


def region_extent_end(region):
    _, off, stride, unit, num, ups = region
    if num == 0:
        return off
    return off + (num - 1) * stride + ups * unit


def storage_extent_end(pool):
    live_end = max([region_extent_end(r) for r in pool["regions"]] + [0])
    return pool["base"] + (pool["num_blocks"] - 1) * pool["block_stride"] + live_end


def copy_extents(pool, block_ids):
    ext = []
    for b in block_ids:
        if b < 0 or b >= pool["num_blocks"]:
            raise PoolError("out of range")
        base = pool["base"] + b * pool["block_stride"]
        for r in pool["regions"]:
            _, off, stride, unit, num, ups = r
            pb = unit * ups
            if num == 0 or pb == 0:
                continue
            if stride == pb:
                ext.append((base + off, num * pb))
            else:
                ext.extend((base + off + u * stride, pb) for u in range(num))
    ext.sort()
    merged = []
    for o, s in ext:
        if merged and o <= merged[-1][0] + merged[-1][1]:
            po, ps = merged[-1]
            merged[-1] = (po, max(po + ps, o + s) - po)
        else:
            merged.append((o, s))
    return merged


def live_segments(pool):
    stride_b = pool["block_stride"]
    runs = []
    for r in pool["regions"]:
        _, off, stride, unit, num, ups = r
        pb = unit * ups
        if num > 0 and stride < pb:
            raise PoolError("overlapping units within one region")
        if num > 0 and stride == pb:
            spans = [(off, off + num * pb)]
        else:
            spans = [(off + u * stride, off + u * stride + pb) for u in range(num)]
        for s, e in spans:
            if e > stride_b:
                raise PoolError("live region exceeds its block stride")
            runs.append((s, e))
    runs.sort()
    phys = []
    for s, e in runs:
        if phys and s < phys[-1][1]:
            raise PoolError("overlapping live regions")
        if phys and s == phys[-1][1]:
            phys[-1] = (phys[-1][0], e)
        else:
            phys.append((s, e))
    out, logical = [], 0
    for s, e in phys:
        out.append((logical, s, e - s))
        logical += e - s
    return out


def physical_to_logical(segments, physical_offset, size):
    if physical_offset < 0 or size <= 0:
        raise PoolError("physical live range offset/size is invalid")
    end = physical_offset + size
    for lo, po, sz in segments:
        if po <= physical_offset and end <= po + sz:
            lg = lo + physical_offset - po
            return lg, lg + size
    raise PoolError("crosses padding")


def translate_live_copy(src_segments, dst_segments, src_offset, dst_offset, size):
    if src_offset < 0 or dst_offset < 0 or size <= 0:
        raise PoolError("Compact-live copy offsets/size are invalid")

    def locate(segs, logical):
        for lo, po, sz in segs:
            if lo <= logical < lo + sz:
                return po + logical - lo, lo + sz - logical
        raise PoolError("Compact-live offset out of range")

    out, left, sc, dc = [], size, src_offset, dst_offset
    while left > 0:
        sp, sa = locate(src_segments, sc)
        dp, da = locate(dst_segments, dc)
        n = min(left, sa, da)
        out.append((sp, dp, n))
        sc += n
        dc += n
        left -= n
    return out


def regions_cover_range(regions, start, end):
    cursor = start
    while cursor < end:
        nxt = cursor
        for _, off, stride, unit, num, ups in regions:
            pb = unit * ups
            if num <= 0 or cursor < off or pb == 0:
                continue
            u = 0
            if num > 1:
                if stride == 0:
                    continue
                u = (cursor - off) // stride
                if u >= num:
                    continue
            s = off + u * stride
            if s <= cursor < s + pb:
                nxt = max(nxt, min(s + pb, end))
        if nxt == cursor:
            return False
        cursor = nxt
    return True
