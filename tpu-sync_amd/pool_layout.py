"""Storage / pool / region descriptors for block admission.

The reference's Python descriptors (tpu_sync/api/torch/pool_layout.py:30-199):
a *storage* is one wrapped allocation (a KVCacheManager block array, index =
layer); a *pool* is an array of equally strided blocks inside one storage;
*regions* describe the live bytes of one block. ``tag`` and ``dtype_tag`` are
labels for the caller: kept with the pool, usable to select pools by tag and
returned by ``to_dict``, but this package gives them no meaning.

The geometry functions below (copy extents, live segments, compact-live copy
translation) run the library's native restatement of
tpu_sync/kv_cache/pool_layout.cc through the C-ABI.
"""

from __future__ import annotations

import ctypes
import dataclasses
from typing import List, Mapping, Sequence, Tuple

from . import _capi


@dataclasses.dataclass(frozen=True)
class RegionSpec:
    name: str
    offset_bytes: int
    stride_bytes: int
    unit_bytes: int
    num_units: int
    units_per_stride: int = 1

    @property
    def live_bytes(self) -> int:
        return self.unit_bytes * self.num_units * self.units_per_stride

    @property
    def extent_end_bytes(self) -> int:
        if self.num_units == 0:
            return self.offset_bytes
        return (self.offset_bytes + (self.num_units - 1) * self.stride_bytes
                + self.units_per_stride * self.unit_bytes)

    def validate(self, slot_bytes: int) -> None:
        """pool_layout.py:55-82: the same checks and messages."""
        if not self.name:
            raise ValueError("region name must be non-empty")
        for field in ("offset_bytes", "stride_bytes", "unit_bytes", "num_units",
                      "units_per_stride"):
            if getattr(self, field) < 0:
                raise ValueError(f"region {self.name} {field} must be >= 0")
        if self.num_units > 0 and self.unit_bytes <= 0:
            raise ValueError(f"region {self.name} unit_bytes must be positive")
        if self.num_units > 1 and self.stride_bytes <= 0:
            raise ValueError(f"region {self.name} stride_bytes must be positive")
        if self.units_per_stride <= 0:
            raise ValueError(f"region {self.name} units_per_stride must be positive")
        if self.num_units > 0 and self.stride_bytes < self.units_per_stride * self.unit_bytes:
            raise ValueError(f"region {self.name} stride_bytes is smaller than packed units")
        if self.extent_end_bytes > slot_bytes:
            raise ValueError(f"region {self.name} exceeds slot bytes: "
                             f"end={self.extent_end_bytes} slot={slot_bytes}")

    def to_dict(self) -> dict:
        return dataclasses.asdict(self)


@dataclasses.dataclass(frozen=True)
class PoolSpec:
    tag: str
    storage_index: int
    base_offset_bytes: int
    block_stride_bytes: int
    num_blocks: int
    regions: Tuple[RegionSpec, ...]
    dtype_tag: str = ""

    @property
    def storage_extent_end_bytes(self) -> int:
        """Byte offset, from the start of the storage, just past the live
        bytes of the pool's last block (its furthest-reaching region)."""
        live_end = max((r.extent_end_bytes for r in self.regions), default=0)
        return self.base_offset_bytes + (self.num_blocks - 1) * self.block_stride_bytes + live_end

    @property
    def live_bytes_per_block(self) -> int:
        return sum(r.live_bytes for r in self.regions)

    def validate(self, storage_bytes: int | None = None) -> None:
        """pool_layout.py:121-145: the same checks and messages."""
        if not self.tag:
            raise ValueError("pool tag must be non-empty")
        if self.storage_index < 0:
            raise ValueError(f"pool {self.tag} storage_index must be >= 0")
        if self.block_stride_bytes <= 0:
            raise ValueError(f"pool {self.tag} block_stride_bytes must be positive")
        if self.num_blocks <= 0:
            raise ValueError(f"pool {self.tag} num_blocks must be positive")
        if self.base_offset_bytes < 0:
            raise ValueError(f"pool {self.tag} base_offset_bytes must be >= 0")
        if not self.regions:
            raise ValueError(f"pool {self.tag} must contain at least one region")
        for r in self.regions:
            r.validate(self.block_stride_bytes)
        if storage_bytes is not None and self.storage_extent_end_bytes > storage_bytes:
            raise ValueError(f"pool {self.tag} exceeds storage bytes (live regions): "
                             f"end={self.storage_extent_end_bytes} storage={storage_bytes}")

    def to_dict(self) -> dict:
        return {"tag": self.tag, "storage_index": self.storage_index,
                "base_offset_bytes": self.base_offset_bytes,
                "block_stride_bytes": self.block_stride_bytes,
                "num_blocks": self.num_blocks,
                "regions": [r.to_dict() for r in self.regions],
                "dtype_tag": self.dtype_tag}


def coerce_region_spec(value) -> RegionSpec:
    if isinstance(value, RegionSpec):
        return value
    return RegionSpec(name=str(value["name"]), offset_bytes=int(value["offset_bytes"]),
                      stride_bytes=int(value["stride_bytes"]),
                      unit_bytes=int(value["unit_bytes"]), num_units=int(value["num_units"]),
                      units_per_stride=int(value.get("units_per_stride", 1)))


def coerce_pool_spec(value) -> PoolSpec:
    if isinstance(value, PoolSpec):
        return value
    regions = value["regions"]
    if not isinstance(regions, Sequence):
        raise TypeError("pool regions must be a sequence")
    return PoolSpec(tag=str(value["tag"]), storage_index=int(value["storage_index"]),
                    base_offset_bytes=int(value.get("base_offset_bytes", 0)),
                    block_stride_bytes=int(value["block_stride_bytes"]),
                    num_blocks=int(value["num_blocks"]),
                    regions=tuple(coerce_region_spec(r) for r in regions),
                    dtype_tag=str(value.get("dtype_tag", "")))


# -- C-ABI marshalling -------------------------------------------------------
class _NativePool:
    """A kvx_pool_spec and the buffers it points into."""

    def __init__(self, pool: PoolSpec):
        self.tag = pool.tag.encode()
        self.dtype = pool.dtype_tag.encode()
        self.names = [r.name.encode() for r in pool.regions]
        n = len(pool.regions)
        self.regions = (_capi.RegionSpecC * max(n, 1))()
        for i, r in enumerate(pool.regions):
            self.regions[i] = _capi.RegionSpecC(self.names[i], r.offset_bytes, r.stride_bytes,
                                                r.unit_bytes, r.num_units, r.units_per_stride)
        self.c = _capi.PoolSpecC(self.tag, pool.storage_index, pool.base_offset_bytes,
                                 pool.block_stride_bytes, pool.num_blocks, self.regions, n,
                                 self.dtype)


def native_pools(pools: Sequence[PoolSpec]):
    """(kvx_pool_spec array, keep-alive list) for a pool table."""
    keep = [_NativePool(p) for p in pools]
    arr = (_capi.PoolSpecC * max(len(keep), 1))()
    for i, k in enumerate(keep):
        arr[i] = k.c
    return arr, keep


def _grow_call(fn, per, *args):
    """Calls fn(*args, out, cap, n_out), growing `out` until it fits."""
    cap = 64
    while True:
        out = (ctypes.c_int64 * (per * cap))()
        n = ctypes.c_int64()
        _capi.check(fn(*args, out, cap, ctypes.byref(n)))
        if n.value <= cap:
            return [tuple(out[per * i:per * i + per]) for i in range(n.value)]
        cap = n.value


def validate_native(pool: PoolSpec, storage_bytes: int = -1) -> None:
    """PoolSpec::Validate in the library (raises KvxError)."""
    p = _NativePool(pool)
    _capi.check(_capi.load().kvx_pool_validate(ctypes.byref(p.c), storage_bytes))


def storage_extent_end_native(pool: PoolSpec) -> int:
    p = _NativePool(pool)
    return _capi.load().kvx_pool_storage_extent_end(ctypes.byref(p.c))


def compute_pool_block_copy_extents(pool: PoolSpec, block_ids: Sequence[int]
                                    ) -> List[Tuple[int, int]]:
    """Sorted, coalesced (offset_bytes, size_bytes) live extents of `block_ids`."""
    p = _NativePool(pool)
    ids, n = _capi.i64_array(block_ids)
    return _grow_call(_capi.load().kvx_pool_copy_extents, 2, ctypes.byref(p.c), ids, n)


def expand_pool_live_segments(pool: PoolSpec) -> List[Tuple[int, int, int]]:
    """(logical_offset, physical_offset, size) runs of one block's live bytes."""
    p = _NativePool(pool)
    return _grow_call(_capi.load().kvx_pool_live_segments, 3, ctypes.byref(p.c))


def physical_live_range_to_logical(pool: PoolSpec, physical_offset: int,
                                   size: int) -> Tuple[int, int]:
    p = _NativePool(pool)
    b, e = ctypes.c_int64(), ctypes.c_int64()
    _capi.check(_capi.load().kvx_pool_physical_to_logical(
        ctypes.byref(p.c), physical_offset, size, ctypes.byref(b), ctypes.byref(e)))
    return b.value, e.value


def translate_live_copy(src: PoolSpec, dst: PoolSpec, src_offset: int, dst_offset: int,
                        size: int) -> List[Tuple[int, int, int]]:
    """(src_physical, dst_physical, size) chunks of a compact-live copy."""
    ps, pd = _NativePool(src), _NativePool(dst)
    return _grow_call(_capi.load().kvx_pool_translate_live_copy, 3, ctypes.byref(ps.c),
                      ctypes.byref(pd.c), src_offset, dst_offset, size)


def regions_cover_range(regions: Sequence[RegionSpec], start: int, end: int) -> bool:
    p = _NativePool(PoolSpec("", 0, 0, 0, 0, tuple(regions)))
    return bool(_capi.load().kvx_regions_cover_range(p.regions, len(regions), start, end))
