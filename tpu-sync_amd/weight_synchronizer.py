"""Weight synchronizer over libkvx (one MI355X).

Mirrors the reference's Python surface (tpu_sync/api/torch/
weight_synchronizer.py:19-140): ``WeightSynchronizer(device_tensors)`` over
``[layers][shards]`` contiguous device tensors, ``d2h()`` / ``h2d()`` of the
whole parameter set, ``get_host_buffer(layer, shard)`` as a zero-copy CPU
tensor view, ``num_layers`` / ``num_shards`` / ``slice_byte_size``. The host
copies share one pinned buffer laid out by a per-tensor offset table, and
``d2h`` / ``h2d`` run the offset-table pack / unpack kernel through a device
staging ring so the parameters cross PCIe as a few large DMAs.

Resharding is the reference's strided push-entry expansion
(tpu_sync/weight_sync/weight_synchronizer_base.cc:626-666) executed on the
device: ``copy_strided(entries)`` runs any list of
``(src, dst, size, count, src_stride, dst_stride)`` entries in one launch,
and ``column_split_entries`` builds the entries of a column split whose
bounds follow ``compute_nd_shard_slices`` (tpu_sync/kv_cache/
nd_slice_math.py:23-70: equal tiles, remainder to the last shard).
Networked pushes and their listener are not part of this package.

A weight may be stored tiled on the device (``layouts``, one
``tiling.TiledLayout`` or None per tensor): its host copy is then the
row-major image, as the reference's D2hLayer / H2dLayer produce by detiling /
tiling on the host (weight_synchronizer_base.cc:357-389, 473-510); here the
detile / tile runs in HBM on the staging chunks.
"""
import ctypes
import itertools
from typing import Any, List, Optional, Sequence, Tuple

from . import _capi
from .kv_cache_manager import RaidenFuture, _stream_ptr


def compute_nd_shard_slices(global_shape: Sequence[int], mesh_shape: Sequence[int]
                            ) -> List[List[Tuple[int, int]]]:
    """Per-shard [start, end) bounds of every dimension, shards in row-major
    order; the last shard of a dimension takes the remainder."""
    if len(global_shape) != len(mesh_shape):
        raise ValueError(f"Tensor rank ({len(global_shape)}) and sharding mesh rank"
                         f" ({len(mesh_shape)}) must match exactly.")
    for d, m in enumerate(mesh_shape):
        if m <= 0:
            raise ValueError(f"Mesh shape at dimension {d} must be positive.")
    tiles = [g // m for g, m in zip(global_shape, mesh_shape)]
    out = []
    for coord in itertools.product(*[range(m) for m in mesh_shape]):
        box = []
        for d, c in enumerate(coord):
            start = c * tiles[d]
            end = (c + 1) * tiles[d] if c < mesh_shape[d] - 1 else global_shape[d]
            box.append((start, end))
        out.append(box)
    return out


class StridedEntry:
    """One strided push entry with device addresses."""

    __slots__ = ("src", "dst", "size", "count", "src_stride", "dst_stride")

    def __init__(self, src: int, dst: int, size: int, count: int = 1,
                 src_stride: int = 0, dst_stride: int = 0):
        self.src, self.dst, self.size = int(src), int(dst), int(size)
        self.count, self.src_stride, self.dst_stride = int(count), int(src_stride), int(dst_stride)

    def as_tuple(self):
        return (self.src, self.dst, self.size, self.count, self.src_stride, self.dst_stride)


def column_split_entries(weight, outputs: Sequence[Any]) -> List[StridedEntry]:
    """Entries copying column chunk j of a row-major 2-D ``weight`` [R, C]
    into contiguous ``outputs[j]`` ([R, C_j]); chunk bounds from
    compute_nd_shard_slices((R, C), (1, k))."""
    if weight.dim() != 2:
        raise ValueError("column_split_entries needs a 2-D weight")
    wptr, _ = _capi.device_buffer(weight, "weight")
    device = weight.device.index or 0
    rows, cols = int(weight.shape[0]), int(weight.shape[1])
    item = weight.element_size()
    k = len(outputs)
    bounds = compute_nd_shard_slices((rows, cols), (1, k))
    entries = []
    for j, box in enumerate(bounds):
        c0, c1 = box[1]
        out = outputs[j]
        if tuple(out.shape) != (rows, c1 - c0) or not out.is_contiguous():
            raise ValueError(f"output {j} must be a contiguous [{rows}, {c1 - c0}] tensor")
        if out.dtype != weight.dtype:
            raise ValueError(f"output {j} has dtype {out.dtype}, the weight {weight.dtype}")
        optr, _ = _capi.device_buffer(out, f"output {j}", device)
        if c1 == c0 or rows == 0:
            continue  # an empty chunk moves nothing
        entries.append(StridedEntry(wptr + c0 * item, optr,
                                    (c1 - c0) * item, rows, cols * item, (c1 - c0) * item))
    return entries


class StridedPlan:
    """Entries converted once into the C-ABI's entry array, for callers that
    run the same entries repeatedly (the same column split every sync). The
    first copy_strided of the plan on a device also builds and uploads its
    device table there (kvx_strided_plan_create); later runs on that device
    are one launch each. The tensors the entries address must outlive the
    plan's runs; close() (or garbage collection) frees the device tables
    after the runs in flight."""

    def __init__(self, entries: Sequence[StridedEntry], profile_kernels: bool = False):
        import numpy as np
        self.n = len(entries)
        self._profile = bool(profile_kernels)
        self._arr = (_capi.StridedEntryC * max(self.n, 1))()
        self._device_plans = {}  # device -> kvx_strided_plan handle
        if self.n:
            rows = np.frombuffer(self._arr, dtype=np.uint64).reshape(-1, 8)
            vals = np.array([e.as_tuple() for e in entries], dtype=np.uint64)
            rows[:, 0:2] = vals[:, 0:2]     # src, dst
            rows[:, 2:4] = 0                # src/dst offsets (folded into src/dst)
            rows[:, 4:8] = vals[:, 2:6]     # size, count, src_stride, dst_stride

    def _device_plan(self, device: int) -> ctypes.c_void_p:
        h = self._device_plans.get(device)
        if h is None:
            h = ctypes.c_void_p()
            _capi.check(_capi.load().kvx_strided_plan_create(device, self._arr, self.n,
                                                             ctypes.byref(h)),
                        "StridedPlan")
            self._device_plans[device] = h
            if self._profile:
                _capi.check(_capi.load().kvx_strided_plan_profile(h, 1), "StridedPlan profile")
        return h

    def kernel_times(self, reset: bool = False, device: int = 0) -> dict:
        """With profile_kernels: launches, summed duration (ms, HIP events right
        around each launch on its stream) and algorithmic HBM bytes (2 x bytes
        moved) of the plan's runs on `device` so far."""
        h = self._device_plans.get(device)
        if h is None:
            return {"launches": 0, "total_ms": 0.0, "bytes": 0}
        n, ms, nb = ctypes.c_int64(), ctypes.c_double(), ctypes.c_int64()
        _capi.check(_capi.load().kvx_strided_plan_kernel_times(
            h, int(reset), ctypes.byref(n), ctypes.byref(ms), ctypes.byref(nb)), "kernel_times")
        return {"launches": n.value, "total_ms": ms.value, "bytes": nb.value}

    def close(self) -> None:
        plans, self._device_plans = getattr(self, "_device_plans", {}), {}
        for h in plans.values():
            _capi.load().kvx_strided_plan_destroy(h)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def copy_strided(entries, stream=None, device: int = 0, keep_alive=None) -> RaidenFuture:
    """Runs every entry (a sequence of StridedEntry, or a StridedPlan) in one
    kernel launch on `stream` (default: torch's current stream)."""
    if stream is None:
        import torch
        stream = torch.cuda.current_stream(device)
    out = ctypes.c_void_p()
    if isinstance(entries, StridedPlan):
        _capi.check(_capi.load().kvx_strided_plan_run(entries._device_plan(device),
                                                      ctypes.c_void_p(_stream_ptr(stream)),
                                                      ctypes.byref(out)), "copy_strided")
        return RaidenFuture(out, keep_alive, "copy_strided")
    plan = StridedPlan(entries)
    _capi.check(_capi.load().kvx_copy_strided(device, plan._arr, plan.n,
                                              ctypes.c_void_p(_stream_ptr(stream)),
                                              ctypes.byref(out)), "copy_strided")
    return RaidenFuture(out, keep_alive, "copy_strided")


class WeightSynchronizer:
    """Host staging of a model's weights (one device tensor per layer/shard)."""

    def __init__(self, device_tensors: List[List[Any]], local_port: Optional[int] = None,
                 parallelism: int = 1, listener_port: Optional[int] = None,
                 bind_ip: Optional[str] = None, unsafe_skip_buffer_lock: bool = True,
                 auto_h2d: bool = False, *, host_alloc: str = "pinned",
                 chunk_bytes: int = 0, staging_chunks: int = 0,
                 profile_kernels: bool = False, numa_local: bool = True,
                 layouts: Optional[List[List[Any]]] = None):
        del local_port, parallelism, listener_port, bind_ip, unsafe_skip_buffer_lock, auto_h2d
        layers = [list(x) if isinstance(x, (list, tuple)) else [x] for x in device_tensors]
        num_shards = len(layers[0]) if layers else 1
        if any(len(s) != num_shards for s in layers):
            raise RuntimeError("Number of shards mismatch across layers")
        ptrs, sizes, device = [], [], None
        for shards in layers:
            for t in shards:
                if getattr(t, "is_cuda", False) and not t.is_contiguous():
                    raise RuntimeError("weight tensors must be contiguous")
                if device is None and getattr(t, "is_cuda", False):
                    device = t.device.index or 0
                ptr, nbytes = _capi.device_buffer(t, "weight tensor", device)
                ptrs.append(ptr)
                sizes.append(nbytes)
        device = device or 0
        self._tensors = layers
        self._device = device
        cfg = _capi.WeightSyncConfig()
        cfg.device = device
        cfg.host_alloc = {"pinned": _capi.HOST_PINNED, "malloc": _capi.HOST_MALLOC}[host_alloc]
        cfg.num_layers = len(layers)
        cfg.num_shards = num_shards
        self._ptr_arr = (ctypes.c_uint64 * max(len(ptrs), 1))(*ptrs)
        self._size_arr = (ctypes.c_int64 * max(len(sizes), 1))(*sizes)
        cfg.device_ptrs = self._ptr_arr
        cfg.device_bytes = self._size_arr
        cfg.chunk_bytes = chunk_bytes
        cfg.staging_chunks = staging_chunks
        cfg.profile_kernels = int(bool(profile_kernels))
        cfg.numa_off = 0 if numa_local else 1
        self._layouts = None
        if layouts is not None:
            flat = [list(x) if isinstance(x, (list, tuple)) else [x] for x in layouts]
            if len(flat) != len(layers) or any(len(s) != num_shards for s in flat):
                raise RuntimeError("layouts must match device_tensors layer by layer")
            self._layouts = flat
            n = len(layers) * num_shards
            self._layout_arr = (_capi.TiledLayoutC * max(n, 1))()
            for k, lay in enumerate(x for shards in flat for x in shards):
                if lay is not None:
                    self._layout_arr[k] = lay.to_c()
            cfg.layouts = self._layout_arr
        h = ctypes.c_void_p()
        _capi.check(_capi.load().kvx_weight_sync_create(ctypes.byref(cfg), ctypes.byref(h)),
                    "WeightSynchronizer create")
        self._h = h

    def _fut(self, fn, where, *args, stream=None, keep=None):
        out = ctypes.c_void_p()
        _capi.check(fn(self._h, *args, ctypes.c_void_p(_stream_ptr(stream)),
                       ctypes.byref(out)), where)
        return RaidenFuture(out, keep if keep is not None else self, where)

    def d2h(self, stream=None) -> RaidenFuture:
        """Asynchronous copy of every weight to the host buffer."""
        return self._fut(_capi.load().kvx_weight_sync_d2h, "WeightSynchronizer D2h",
                         stream=stream)

    def h2d(self, stream=None) -> RaidenFuture:
        """Asynchronous copy of the host buffer back into every weight."""
        return self._fut(_capi.load().kvx_weight_sync_h2d, "WeightSynchronizer H2d",
                         stream=stream)

    def d2h_layer(self, layer_idx: int, stream=None) -> RaidenFuture:
        return self._fut(_capi.load().kvx_weight_sync_d2h_layer, "WeightSynchronizer D2hLayer",
                         layer_idx, stream=stream)

    def h2d_layer(self, layer_idx: int, stream=None) -> RaidenFuture:
        return self._fut(_capi.load().kvx_weight_sync_h2d_layer, "WeightSynchronizer H2dLayer",
                         layer_idx, stream=stream)

    def pack(self, staging, stream=None) -> RaidenFuture:
        """Packs every weight into a device tensor of total_bytes bytes laid
        out by the offset table (one kernel launch)."""
        ptr, nbytes = _capi.device_buffer(staging, "staging", self._device)
        if stream is None:
            import torch
            stream = torch.cuda.current_stream(staging.device)
        return self._fut(_capi.load().kvx_weight_sync_pack, "WeightSynchronizer pack",
                         ptr, nbytes, stream=stream, keep=(self, staging))

    def unpack(self, staging, stream=None) -> RaidenFuture:
        ptr, nbytes = _capi.device_buffer(staging, "staging", self._device)
        if stream is None:
            import torch
            stream = torch.cuda.current_stream(staging.device)
        return self._fut(_capi.load().kvx_weight_sync_unpack, "WeightSynchronizer unpack",
                         ptr, nbytes, stream=stream, keep=(self, staging))

    def host_buffer_info(self, layer_idx: int = 0, shard_idx: int = 0) -> Tuple[int, int, int]:
        """(host address, bytes, offset in the packed image) of one weight."""
        p, n, o = ctypes.c_uint64(), ctypes.c_int64(), ctypes.c_int64()
        _capi.check(_capi.load().kvx_weight_sync_host_buffer(
            self._h, layer_idx, shard_idx, ctypes.byref(p), ctypes.byref(n), ctypes.byref(o)))
        return p.value, n.value, o.value

    def get_host_buffer(self, layer_idx: int = 0, shard_idx: int = 0):
        """Zero-copy CPU tensor view of one weight's host copy (its dtype and
        shape)."""
        import torch
        ptr, nbytes, _ = self.host_buffer_info(layer_idx, shard_idx)
        t = self._tensors[layer_idx][shard_idx]
        buf = (ctypes.c_uint8 * nbytes).from_address(ptr)
        lay = self._layouts[layer_idx][shard_idx] if self._layouts else None
        if lay is not None and lay.tiles:
            # The host copy of a tiled weight is its row-major image.
            dtype = {1: torch.uint8, 2: torch.int16, 4: torch.int32, 8: torch.int64}[lay.itemsize]
            if t.element_size() == lay.itemsize:
                dtype = t.dtype
            return torch.frombuffer(buf, dtype=torch.uint8).view(dtype).view(lay.dims)
        return torch.frombuffer(buf, dtype=torch.uint8).view(t.dtype).view(t.shape)

    def host_image(self):
        """numpy uint8 view of the whole packed host buffer."""
        import numpy as np
        lib = _capi.load()
        base, total = lib.kvx_weight_sync_host_base(self._h), self.total_bytes
        return np.ctypeslib.as_array((ctypes.c_uint8 * total).from_address(base))

    @property
    def total_bytes(self) -> int:
        return _capi.load().kvx_weight_sync_total_bytes(self._h)

    @property
    def num_layers(self) -> int:
        return len(self._tensors)

    @property
    def num_shards(self) -> int:
        return len(self._tensors[0]) if self._tensors else 0

    @property
    def slice_byte_size(self) -> int:
        t = self._tensors[0][0]
        return t.numel() * t.element_size() // max(int(t.shape[0]), 1) if t.dim() else 0

    def wait(self) -> None:
        _capi.check(_capi.load().kvx_weight_sync_wait(self._h))

    def kernel_times(self, pack: bool = True, reset: bool = False) -> dict:
        n, ms, b = ctypes.c_int64(), ctypes.c_double(), ctypes.c_int64()
        _capi.check(_capi.load().kvx_weight_sync_kernel_times(
            self._h, int(pack), int(reset), ctypes.byref(n), ctypes.byref(ms), ctypes.byref(b)))
        return {"launches": n.value, "total_ms": ms.value, "bytes": b.value}

    def close(self) -> None:
        h, self._h = getattr(self, "_h", None), None
        lib = _capi._lib if _capi is not None else None  # None at interpreter exit
        if h and lib is not None:
            lib.kvx_weight_sync_destroy(h)

    def __del__(self):
        self.close()
