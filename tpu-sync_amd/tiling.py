"""Tiled tensor layouts on the device (libkvx's tiled-copy kernel).

Mirrors the reference's tiling routines (tpu_sync/weight_sync/
tiling_utils.h:27-36): ``tiled_buffer_elements`` is GetTiledBufferElements,
``tile_buffer`` / ``detile_buffer`` are TileBuffer / DetileBuffer, here on
device tensors and enqueued on a stream instead of run on the host. A
``TiledLayout`` carries what the reference reads from an xla::Shape with its
xla::Layout: element size, logical dimensions, minor-to-major order and the
tiles applied in turn, e.g. ``TiledLayout(2, (4096, 4096), tiles=[(8, 128),
(2, 1)])`` for a bf16 matrix in the ``{1,0:T(8,128)(2,1)}`` layout.
"""
import ctypes
from typing import Optional, Sequence

from . import _capi
from .kv_cache_manager import RaidenFuture, _stream_ptr


class TiledLayout:
    """Element size, logical dims (row-major), minor_to_major (default:
    row-major, i.e. rank-1 ... 0) and up to 4 tiles (each 1-8 dims >= 1)."""

    __slots__ = ("itemsize", "dims", "minor_to_major", "tiles")

    def __init__(self, itemsize: int, dims: Sequence[int], tiles: Sequence[Sequence[int]] = (),
                 minor_to_major: Optional[Sequence[int]] = None):
        self.itemsize = int(itemsize)
        self.dims = tuple(int(d) for d in dims)
        if minor_to_major is None:
            minor_to_major = tuple(range(len(self.dims) - 1, -1, -1))
        self.minor_to_major = tuple(int(m) for m in minor_to_major)
        self.tiles = [tuple(int(x) for x in t) for t in tiles]
        if len(self.dims) > 8 or len(self.tiles) > 4 or any(len(t) > 8 for t in self.tiles):
            raise ValueError("at most 8 dimensions and 4 tiles of at most 8 dimensions")

    def to_c(self) -> _capi.TiledLayoutC:
        c = _capi.TiledLayoutC()
        c.itemsize = self.itemsize
        c.rank = len(self.dims)
        for i, d in enumerate(self.dims):
            c.dims[i] = d
        for i, m in enumerate(self.minor_to_major):
            c.minor_to_major[i] = m
        c.num_tiles = len(self.tiles)
        for t, tile in enumerate(self.tiles):
            c.tile_rank[t] = len(tile)
            for i, d in enumerate(tile):
                c.tile_dims[t][i] = d
        return c

    @property
    def logical_elements(self) -> int:
        n = 1
        for d in self.dims:
            n *= d
        return n

    @property
    def logical_bytes(self) -> int:
        return self.logical_elements * self.itemsize

    @property
    def tiled_bytes(self) -> int:
        """Bytes of the tiled buffer, padding included (the logical bytes when
        the layout has no tiles)."""
        if not self.tiles or not self.dims:
            return self.logical_bytes
        return tiled_buffer_elements(self) * self.itemsize

    def __repr__(self):
        return (f"TiledLayout(itemsize={self.itemsize}, dims={self.dims}, "
                f"minor_to_major={self.minor_to_major}, tiles={self.tiles})")


def tiled_buffer_elements(layout: TiledLayout) -> int:
    """GetTiledBufferElements: elements of the tiled buffer, padding included."""
    c = layout.to_c()
    out = ctypes.c_int64()
    _capi.check(_capi.load().kvx_tiled_buffer_elements(ctypes.byref(c), ctypes.byref(out)),
                "tiled_buffer_elements")
    return out.value


def _call(fn, where, layout, linear, tiled, stream):
    device = linear.device.index or 0
    lptr, lbytes = _capi.device_buffer(linear, "linear buffer", device)
    tptr, tbytes = _capi.device_buffer(tiled, "tiled buffer", device)
    if lbytes < layout.logical_bytes:
        raise ValueError(f"linear buffer holds {lbytes} bytes, the layout needs "
                         f"{layout.logical_bytes}")
    if tbytes < layout.tiled_bytes:
        raise ValueError(f"tiled buffer holds {tbytes} bytes, the layout needs "
                         f"{layout.tiled_bytes}")
    if stream is None:
        import torch
        stream = torch.cuda.current_stream(linear.device)
    c = layout.to_c()
    out = ctypes.c_void_p()
    a, b = (lptr, tptr) if fn == "kvx_tile_buffer" else (tptr, lptr)
    _capi.check(getattr(_capi.load(), fn)(device, ctypes.byref(c), a, b,
                                          ctypes.c_void_p(_stream_ptr(stream)),
                                          ctypes.byref(out)), where)
    return RaidenFuture(out, (linear, tiled), where)


def tile_buffer(layout: TiledLayout, src_linear, dst_tiled, stream=None) -> RaidenFuture:
    """TileBuffer on the device: row-major ``src_linear`` -> ``dst_tiled``
    (padding written as zero), enqueued on ``stream`` (default: torch's
    current stream)."""
    return _call("kvx_tile_buffer", "tile_buffer", layout, src_linear, dst_tiled, stream)


def detile_buffer(layout: TiledLayout, src_tiled, dst_linear, stream=None) -> RaidenFuture:
    """DetileBuffer on the device: ``src_tiled`` -> row-major ``dst_linear``."""
    return _call("kvx_detile_buffer", "detile_buffer", layout, dst_linear, src_tiled, stream)
