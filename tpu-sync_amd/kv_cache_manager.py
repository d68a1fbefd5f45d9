"""PyTorch-facing KV cache manager over libkvx (MI355X).

Mirrors the reference's Python surface
(tpu_sync/api/torch/kv_cache_manager.py:55-439 and the nanobind module
tpu_sync/frameworks/torch/tpu_raiden_torch_module.cc:339-395): ``d2h`` /
``h2d`` by major-dimension block offsets returning a future with
``Await`` / ``IsReady`` / ``PollError``, ``d2h_auto_allocate``,
``read_block_bytes`` / ``write_block_bytes`` and the CPU-only constructor
``create_host_only_for_testing``. Errors raise ``RuntimeError`` subclasses
whose text follows the reference's "KVCacheManager D2h failed: <msg>".

This module only passes pointers: device tensors by ``data_ptr()`` and
streams by ``cuda_stream``. All copying happens in libkvx.
"""
import ctypes
from typing import Any, List, Optional, Sequence, Tuple

from . import _capi


_pending_callbacks = {}  # OnReady trampolines the library has not called yet


class RaidenFuture:
    """Async completion of one copy (tpu_sync/core/raiden_future.h:25-36)."""

    def __init__(self, handle, keep_alive=None, where=""):
        self._h = handle
        self._keep = keep_alive
        self._where = where

    def Await(self) -> None:
        """Blocks until the copy finished; raises on failure."""
        _capi.check(_capi.load().kvx_future_await(self._h), self._where)

    def IsReady(self) -> bool:
        return bool(_capi.load().kvx_future_is_ready(self._h))

    def PollError(self) -> None:
        """Non-blocking: raises if the copy already failed."""
        _capi.check(_capi.load().kvx_future_poll_error(self._h), self._where)

    def wait_on_stream(self, stream=None) -> None:
        """Orders `stream` (default: torch's current stream) after the copy."""
        if stream is None:
            import torch
            stream = torch.cuda.current_stream()
        _capi.check(_capi.load().kvx_future_wait_on_stream(
            self._h, ctypes.c_void_p(_stream_ptr(stream))), self._where)

    def OnReady(self, fn) -> None:
        """Calls fn(code) once the copy is done (code 0 on success, else the
        absl status code), from a library thread unless it is already done;
        raiden_future.h / PjRtCopyFuture::OnReady."""
        key = object()

        def tramp(_user, code):
            _pending_callbacks.pop(key, None)
            fn(int(code))

        cb = _capi.READY_FN(tramp)
        _pending_callbacks[key] = cb  # alive until the library calls it
        rc = _capi.load().kvx_future_on_ready(self._h, cb, None)
        if rc != 0:
            _pending_callbacks.pop(key, None)
            _capi.check(rc, self._where)

    # Pythonic aliases.
    await_ = Await
    is_ready = IsReady
    poll_error = PollError
    on_ready = OnReady

    def __del__(self):
        h, self._h = getattr(self, "_h", None), None
        lib = _capi._lib if _capi is not None else None  # None at interpreter exit
        if h and lib is not None:
            lib.kvx_future_release(h)


def _stream_ptr(stream) -> int:
    if stream is None:
        return 0
    if isinstance(stream, int):
        return stream
    return int(getattr(stream, "cuda_stream", stream))


def _flatten_caches(kv_caches) -> Tuple[List[List[Any]], int]:
    layers = []
    for entry in kv_caches:
        shards = list(entry) if isinstance(entry, (list, tuple)) else [entry]
        layers.append(shards)
    num_shards = len(layers[0]) if layers else 0
    if any(len(s) != num_shards for s in layers):
        raise RuntimeError("Number of shards mismatch across layers")
    return layers, num_shards


def probe_stream_queues(streams) -> int:
    """Pairs of `streams` (torch.cuda.Stream objects or raw hipStream_t
    values of the current device, at most 64) whose short probe kernels ran
    one after the other, i.e. that share a hardware queue."""
    vals = [int(getattr(s, "cuda_stream", s)) for s in streams]
    arr = (ctypes.c_uint64 * max(len(vals), 1))(*vals)
    out = ctypes.c_int32()
    _capi.check(_capi.load().kvx_probe_stream_queues(arr, len(vals), ctypes.byref(out)))
    return int(out.value)



def measure_link_peaks(nbytes: int = 1 << 30, reps: int = 5) -> dict:
    """Pinned-host <-> device copy rates (GB/s) of the current device on the
    SDMA engines the pageable lanes use: device-to-host and host-to-device
    alone and both at once, the best of 3 rounds of `reps` copies of `nbytes`
    (1..16 GiB; 2 x nbytes of device and of pinned host memory are held for
    the call). `engines`: the device-to-host engine bit << 16 | the
    host-to-device bit."""
    out = (ctypes.c_double * 3)()
    eng = ctypes.c_uint32()
    _capi.check(_capi.load().kvx_measure_link_peaks(nbytes, reps, out, ctypes.byref(eng)),
                "kvx_measure_link_peaks")
    return {"d2h_gbps": out[0], "h2d_gbps": out[1], "bidir_gbps": out[2],
            "engines": int(eng.value)}

class LogicalBlockManager:
    """Host block allocator (tpu_sync/kv_cache/logical_block_manager.h:35-93)."""

    def __init__(self, num_blocks: int = 0, _handle=None, _owner=None):
        lib = _capi.load()
        if _handle is not None:
            self._h, self._owned, self._owner = _handle, False, _owner
        else:
            h = ctypes.c_void_p()
            _capi.check(lib.kvx_block_manager_create(num_blocks, ctypes.byref(h)))
            self._h, self._owned, self._owner = h, True, None

    def allocate(self, num_blocks: int, lock: bool = False) -> List[int]:
        out = (ctypes.c_int32 * max(num_blocks, 1))()
        _capi.check(_capi.load().kvx_block_manager_allocate(self._h, num_blocks,
                                                            int(lock), out))
        return list(out[:num_blocks])

    def _ids_call(self, fn, ids):
        arr, n = _capi.i32_array(ids)
        _capi.check(fn(self._h, arr, n))

    def allocate_target(self, ids: Sequence[int]) -> None:
        self._ids_call(_capi.load().kvx_block_manager_allocate_target, ids)

    def unlock(self, ids: Sequence[int]) -> None:
        self._ids_call(_capi.load().kvx_block_manager_unlock, ids)

    def deallocate(self, ids: Sequence[int]) -> None:
        self._ids_call(_capi.load().kvx_block_manager_deallocate, ids)

    def access_block(self, block_id: int) -> None:
        _capi.check(_capi.load().kvx_block_manager_access(self._h, block_id))

    def is_allocated(self, block_id: int) -> bool:
        return bool(_capi.load().kvx_block_manager_is_allocated(self._h, block_id))

    def is_locked(self, block_id: int) -> bool:
        return bool(_capi.load().kvx_block_manager_is_locked(self._h, block_id))

    @property
    def total_blocks(self) -> int:
        return _capi.load().kvx_block_manager_total_blocks(self._h)

    @property
    def num_free_blocks(self) -> int:
        return _capi.load().kvx_block_manager_num_free(self._h)

    @property
    def num_allocated_blocks(self) -> int:
        return _capi.load().kvx_block_manager_num_allocated(self._h)

    @property
    def num_locked_blocks(self) -> int:
        return _capi.load().kvx_block_manager_num_locked(self._h)

    def __del__(self):
        h = getattr(self, "_h", None)
        lib = _capi._lib if _capi is not None else None  # None at interpreter exit
        if h and getattr(self, "_owned", False) and lib is not None:
            lib.kvx_block_manager_destroy(h)
            self._h = None


class KVCacheManager:
    """Paged KV cache manager on one MI355X.

    Args:
      kv_caches: one contiguous device tensor per layer (K and V buffers count
        as separate layers), or a list of per-shard tensors per layer. Every
        tensor's first dimension is the block (major) dimension.
      host_blocks_to_allocate: host mirror blocks per (layer, shard).
      max_blocks / num_slots: alternatively, a staging-slot layout; the host
        mirror then holds max_blocks * num_slots blocks.
      host_alloc: "pinned" (hipHostMalloc), "malloc" or "shm". Default (None):
        the library chooses "shm" when shm_key or RAIDEN_SHM_KEY is set, else
        "pinned"; shm names left None take RAIDEN_SHM_KEY, RAIDEN_SHM_MODEL_UID
        and RAIDEN_SHM_SERVER_NAME, as the reference's CreateHostMemoryAllocator
        reads them (tpu_sync/core/utils.h:48-91).
      raiden_controller_address: joins the KVCacheStore whose controller
        has this address (in this process) as its transfer worker.
      scale_tables: per-layer side tables with the same major dimension (for
        an fp8 cache, [num_blocks, kv_heads] float32 scales); they are block
        arrays num_kv_layers.. and move with every copy of the same block ids.
      numa: host mirror placement: "auto" (the GPU's NUMA node), "off", or a
        node number.
      dispatch: "env" (queued when RAIDEN_ENABLE_ASYNC_DISPATCH=1), "queued"
        (d2h/h2d return at once; one background thread plans and issues the
        copies in submission order, errors arrive through the future) or
        "inline".
      staging_chunk_bytes / staging_chunks: device staging ring per direction.
      transfer_mode: "auto" (staged when a copy's host runs average at least
        4 MiB per storage, zero-copy below; copies of more than 32 staging
        chunks, and staged copies beyond 32 chunks in flight per direction,
        through the lanes), "staged", "zero_copy" (pinned
        mirror only) or "lanes" (a pinned mirror's short runs through the
        bounce lanes, for callers that load and save at once);
        zero_copy_workgroups caps a zero-copy launch.
      host_copy_threads: a pageable host mirror ("malloc", "shm") moves
        through pinned bounce buffers that this many host threads fill and
        drain (0: 8; -1: per-run pageable copies by the HIP runtime).
      gather_workgroups_per_cu: device gathers (not zero-copy ones) reserve
        LDS so that at most this many share a CU, which serves their random
        reads faster but keeps LDS-heavy kernels of other streams off those
        CUs while they run (0: 2; -1: no limit).
      The remaining reference arguments (ports, worker id, timeout,
      parallelism, unsafe_skip_buffer_lock) configure its networking, which
      this single-GPU build does not have; they are accepted and ignored.
    """

    def __init__(self, kv_caches: List[Any], local_control_port: int = 0,
                 max_blocks: Optional[int] = None, num_slots: Optional[int] = None,
                 timeout_s: float = 120.0, unsafe_skip_buffer_lock: bool = True,
                 host_blocks_to_allocate: Optional[int] = None, parallelism: int = 4,
                 node_id: int = 0, listener_port: Optional[int] = None,
                 raiden_worker_port: int = 0,
                 raiden_controller_address: Optional[str] = None,
                 worker_id: Optional[str] = None, *, host_alloc: Optional[str] = None,
                 staging_chunk_bytes: int = 0, staging_chunks: int = 0,
                 direct_min_bytes: int = 0, shm_key: Optional[str] = None,
                 shm_server_name: Optional[str] = None,
                 model_uid: Optional[str] = None, profile_kernels: bool = False,
                 transfer_mode: str = "auto", zero_copy_workgroups: int = 0,
                 scale_tables: Optional[List[Any]] = None, numa: Any = "auto",
                 dispatch: str = "env", host_copy_threads: int = 0,
                 gather_workgroups_per_cu: int = 0):
        if host_blocks_to_allocate is None:
            if max_blocks is None or num_slots is None:
                raise ValueError("Must specify either (max_blocks, num_slots) or"
                                 " host_blocks_to_allocate.")
            host_blocks_to_allocate = max_blocks * num_slots
        # Side tables (e.g. per-(block, head) fp8 scales, [major_dim, ...])
        # travel with the KV payload: they become block arrays after the KV
        # layers, so every copy and gather moves payload and scales of the
        # same block ids together, in the same kernel launch.
        self.num_kv_layers = len(kv_caches)
        kv_caches = list(kv_caches) + list(scale_tables or [])
        layers, num_shards = _flatten_caches(kv_caches)
        ptrs, sizes = [], []
        major_dim = 0
        device = None
        for shards in layers:
            for t in shards:
                if getattr(t, "is_cuda", False) and not t.is_contiguous():
                    raise RuntimeError("kv cache tensors must be contiguous")
                if device is None and getattr(t, "is_cuda", False):
                    device = t.device.index or 0
                ptr, nbytes = _capi.device_buffer(t, "kv cache tensor", device)
                ptrs.append(ptr)
                sizes.append(nbytes)
        device = device or 0
        self._device = device
        if layers:
            major_dim = int(layers[0][0].shape[0])
        self._tensors = layers  # borrowed device buffers stay alive
        # host_alloc None: the library picks shm when shm_key or RAIDEN_SHM_KEY
        # is set, else pinned; unset shm names take RAIDEN_SHM_* there.
        self._init(device, len(layers), num_shards, ptrs, sizes, major_dim, 0,
                   host_blocks_to_allocate, host_alloc, staging_chunk_bytes,
                   staging_chunks, direct_min_bytes, shm_key, shm_server_name,
                   model_uid, profile_kernels, transfer_mode, zero_copy_workgroups, numa,
                   dispatch, host_copy_threads, gather_workgroups_per_cu)
        self.node_id = node_id
        if max_blocks is not None and num_slots is not None:
            # kv_cache_manager_with_transfer.cc:483-503: slot geometry, then
            # the slot pool (every slot's host ids allocated and locked).
            self.configure_host_staging_slots(num_slots, max_blocks)
            self.initialize_slot_pool(num_slots)
        if raiden_controller_address:
            _capi.check(_capi.load().kvx_manager_register_with_controller(
                self._h, raiden_controller_address.encode()), "RegisterWorker")

    @property
    def queued_dispatch(self) -> bool:
        return bool(_capi.load().kvx_manager_queued_dispatch(self._h))

    def dispatch_log(self) -> str:
        """Kinds of the last dispatched copies ('D' = d2h, 'H' = h2d), oldest first."""
        buf = ctypes.create_string_buffer(256)
        n = ctypes.c_int64()
        _capi.check(_capi.load().kvx_manager_dispatch_log(self._h, buf, 256, ctypes.byref(n)))
        return buf.raw[:min(n.value, 256)].decode()

    @property
    def assigned_numa_node(self) -> int:
        """NUMA node the host mirrors were placed on, or -1."""
        return int(_capi.load().kvx_manager_numa_node(self._h))

    @property
    def host_alloc(self) -> str:
        """The host mirror's memory kind: "malloc", "pinned" or "shm"."""
        kind = _capi.load().kvx_manager_host_alloc(self._h)
        return {_capi.HOST_MALLOC: "malloc", _capi.HOST_PINNED: "pinned",
                _capi.HOST_SHM: "shm"}[kind]

    @property
    def shm_warm(self) -> bool:
        """True when the shared-memory host tier attached to a surviving segment."""
        return bool(_capi.load().kvx_manager_shm_warm(self._h))

    def _init(self, device, num_layers, num_shards, ptrs, sizes, major_dim,
              slice_byte_size, host_blocks, host_alloc, chunk_bytes, chunks,
              direct_min_bytes, shm_key, shm_server_name, model_uid,
              profile_kernels=False, transfer_mode="auto", zero_copy_workgroups=0,
              numa="auto", dispatch="env", host_copy_threads=0,
              gather_workgroups_per_cu=0):
        lib = _capi.load()
        kinds = {"malloc": _capi.HOST_MALLOC, "pinned": _capi.HOST_PINNED,
                 "shm": _capi.HOST_SHM, None: _capi.HOST_AUTO}
        cfg = _capi.ManagerConfig()
        cfg.device = device
        cfg.host_alloc = kinds[host_alloc]
        cfg.num_layers = num_layers
        cfg.num_shards = num_shards
        if ptrs:
            self._ptr_arr = (ctypes.c_uint64 * len(ptrs))(*ptrs)
            self._size_arr = (ctypes.c_int64 * len(sizes))(*sizes)
            cfg.device_ptrs = self._ptr_arr
            cfg.device_bytes = self._size_arr
        cfg.major_dim = major_dim
        cfg.slice_byte_size = slice_byte_size
        cfg.host_blocks = host_blocks
        cfg.staging_chunk_bytes = chunk_bytes
        cfg.staging_chunks = chunks
        cfg.direct_min_bytes = direct_min_bytes
        cfg.shm_key = shm_key.encode() if shm_key else None
        cfg.shm_server_name = shm_server_name.encode() if shm_server_name else None
        cfg.model_uid = model_uid.encode() if model_uid else None
        cfg.profile_kernels = int(bool(profile_kernels))
        cfg.transfer_mode = _capi.MODES[transfer_mode]
        cfg.zero_copy_workgroups = zero_copy_workgroups
        cfg.dispatch = {"env": 0, "queued": 1, "inline": 2}[dispatch]
        cfg.host_copy_threads = host_copy_threads
        cfg.gather_workgroups_per_cu = gather_workgroups_per_cu
        if numa == "auto":
            cfg.numa_policy = 0
        elif numa in ("off", None):
            cfg.numa_policy = 1
        else:
            cfg.numa_policy, cfg.numa_node = 2, int(numa)
        h = ctypes.c_void_p()
        _capi.check(lib.kvx_manager_create(ctypes.byref(cfg), ctypes.byref(h)),
                    "KVCacheManager create")
        self._h = h

    @classmethod
    def create_host_only_for_testing(cls, *, num_layers: int, num_shards: int = 1,
                                     slice_byte_size: int, node_id: int = 0,
                                     local_port: Optional[int] = None,
                                     host_blocks: int, parallelism: int = 4,
                                     host_alloc: str = "malloc",
                                     shm_key: Optional[str] = None,
                                     shm_server_name: Optional[str] = None,
                                     model_uid: Optional[str] = None) -> "KVCacheManager":
        """CPU-only manager backed by library-owned host memory ("shm": a
        shared-memory segment named by shm_key or RAIDEN_SHM_KEY)."""
        obj = cls.__new__(cls)
        obj._tensors = []
        obj._device = None  # no device: gather/scatter fail in the library
        obj._init(0, num_layers, num_shards, [], [], 0, slice_byte_size, host_blocks,
                  host_alloc, 0, 0, 0, shm_key, shm_server_name, model_uid)
        obj.node_id = node_id
        return obj

    # -- copies -------------------------------------------------------------
    def _transfer(self, fn, where, src, dst, sizes, slot_idx, layer_idx, shard_idx,
                  stream):
        s, ns = _capi.i64_array(src)
        d, nd = _capi.i64_array(dst)
        z, nz = _capi.i64_array(sizes if sizes is not None else [])
        out = ctypes.c_void_p()
        _capi.check(fn(self._h, s, ns, d, nd, z, nz,
                       -1 if slot_idx is None else slot_idx,
                       -1 if layer_idx is None else layer_idx,
                       -1 if shard_idx is None else shard_idx,
                       ctypes.c_void_p(_stream_ptr(stream)), ctypes.byref(out)), where)
        return RaidenFuture(out, self, where)

    def d2h(self, src_offsets: Sequence[int] = (), dst_offsets: Sequence[int] = (),
            copy_sizes: Optional[Sequence[int]] = None, *, slot_idx=None,
            layer_idx=None, shard_idx=None, stream=None,
            src_offsets_major_dim=None, dst_offsets_major_dim=None,
            copy_sizes_major_dim=None) -> RaidenFuture:
        """Device-to-host copy of whole blocks (defaults to 1 block per entry)."""
        src = src_offsets_major_dim if src_offsets_major_dim is not None else src_offsets
        dst = dst_offsets_major_dim if dst_offsets_major_dim is not None else dst_offsets
        sizes = copy_sizes_major_dim if copy_sizes_major_dim is not None else copy_sizes
        if sizes is None:
            sizes = [1] * len(src)
        return self._transfer(_capi.load().kvx_manager_d2h, "KVCacheManager D2h", src,
                              dst, sizes, slot_idx, layer_idx, shard_idx, stream)

    def h2d(self, src_offsets: Sequence[int] = (), dst_offsets: Sequence[int] = (),
            copy_sizes: Optional[Sequence[int]] = None, *, slot_idx=None,
            layer_idx=None, shard_idx=None, stream=None,
            src_offsets_major_dim=None, dst_offsets_major_dim=None,
            copy_sizes_major_dim=None) -> RaidenFuture:
        """Host-to-device copy of whole blocks (defaults to 1 block per entry)."""
        src = src_offsets_major_dim if src_offsets_major_dim is not None else src_offsets
        dst = dst_offsets_major_dim if dst_offsets_major_dim is not None else dst_offsets
        sizes = copy_sizes_major_dim if copy_sizes_major_dim is not None else copy_sizes
        if sizes is None:
            sizes = [1] * len(src)
        return self._transfer(_capi.load().kvx_manager_h2d, "KVCacheManager H2d", src,
                              dst, sizes, slot_idx, layer_idx, shard_idx, stream)

    # Reference spellings.
    D2h = d2h
    H2d = h2d

    def d2h_auto_allocate(self, src_offsets_major_dim: Sequence[int] = (),
                          copy_sizes_major_dim: Sequence[int] = (), *, stream=None
                          ) -> Tuple[List[int], RaidenFuture]:
        s, ns = _capi.i64_array(src_offsets_major_dim)
        z, nz = _capi.i64_array(copy_sizes_major_dim)
        total = sum(max(int(v), 0) for v in copy_sizes_major_dim)
        ids = (ctypes.c_int32 * max(total, 1))()
        n_out = ctypes.c_int64()
        out = ctypes.c_void_p()
        where = "KVCacheManager D2hAutoAllocate"
        _capi.check(_capi.load().kvx_manager_d2h_auto_allocate(
            self._h, s, ns, z, nz, ids, total, ctypes.byref(n_out),
            ctypes.c_void_p(_stream_ptr(stream)), ctypes.byref(out)), where)
        return list(ids[:n_out.value]), RaidenFuture(out, self, where)

    D2hAutoAllocate = d2h_auto_allocate

    def _device_copy(self, fn, where, block_ids, staging, order, layer_idx, shard_idx,
                     stream):
        ptr, nbytes = _capi.device_buffer(staging, "staging", self._device)
        ids, n = _capi.i64_array(block_ids)
        out = ctypes.c_void_p()
        if stream is None:
            import torch
            stream = torch.cuda.current_stream(staging.device)
        _capi.check(fn(self._h, ids, n, ptr, nbytes, order,
                       -1 if layer_idx is None else layer_idx,
                       -1 if shard_idx is None else shard_idx,
                       ctypes.c_void_p(_stream_ptr(stream)), ctypes.byref(out)), where)
        return RaidenFuture(out, (self, staging), where)

    def gather(self, block_ids: Sequence[int], staging, *, block_major: bool = False,
               layer_idx=None, shard_idx=None, stream=None) -> RaidenFuture:
        """Extracts blocks into a contiguous device staging tensor (one kernel)."""
        order = _capi.BLOCK_MAJOR if block_major else _capi.LAYER_MAJOR
        return self._device_copy(_capi.load().kvx_manager_gather, "KVCacheManager gather",
                                 block_ids, staging, order, layer_idx, shard_idx, stream)

    def scatter(self, block_ids: Sequence[int], staging, *, block_major: bool = False,
                layer_idx=None, shard_idx=None, stream=None) -> RaidenFuture:
        """Inserts a contiguous device staging tensor into the paged pool."""
        order = _capi.BLOCK_MAJOR if block_major else _capi.LAYER_MAJOR
        return self._device_copy(_capi.load().kvx_manager_scatter, "KVCacheManager scatter",
                                 block_ids, staging, order, layer_idx, shard_idx, stream)

    # -- staging slots and host blocks --------------------------------------
    def configure_host_staging_slots(self, num_slots: int, max_major_per_slot: int) -> None:
        _capi.check(_capi.load().kvx_manager_configure_host_staging_slots(
            self._h, num_slots, max_major_per_slot))

    def host_span(self, layer_idx: int, shard_idx: int, slot_idx: int,
                  num_major: int) -> Tuple[int, int, int]:
        """(host address, nbytes, base_major) of a staging-slot span."""
        ptr, nbytes, base = ctypes.c_uint64(), ctypes.c_int64(), ctypes.c_int64()
        _capi.check(_capi.load().kvx_manager_host_span(
            self._h, layer_idx, shard_idx, slot_idx, num_major, ctypes.byref(ptr),
            ctypes.byref(nbytes), ctypes.byref(base)))
        return ptr.value, nbytes.value, base.value

    def get_block_host_pointer(self, layer_idx: int, shard_idx: int, block_id: int) -> int:
        ptr = ctypes.c_uint64()
        _capi.check(_capi.load().kvx_manager_block_host_ptr(
            self._h, layer_idx, shard_idx, block_id, ctypes.byref(ptr)))
        return ptr.value

    def read_block_bytes(self, layer_idx: int, block_id: int, shard_idx: int = 0) -> bytes:
        n = self.block_bytes(layer_idx)
        buf = ctypes.create_string_buffer(max(n, 1))
        _capi.check(_capi.load().kvx_manager_read_block(self._h, layer_idx, block_id,
                                                        shard_idx, buf, n))
        return buf.raw[:n]

    def write_block_bytes(self, layer_idx: int, block_id: int, payload: bytes,
                          shard_idx: int = 0) -> None:
        payload = bytes(payload)
        _capi.check(_capi.load().kvx_manager_write_block(
            self._h, layer_idx, block_id, shard_idx, payload, len(payload)))

    def host_view(self, layer_idx: int, shard_idx: int = 0):
        """numpy uint8 view of one (layer, shard) host mirror (no copy)."""
        import numpy as np
        lib = _capi.load()
        ptr = lib.kvx_manager_host_ptr(self._h, layer_idx, shard_idx)
        size = lib.kvx_manager_host_size(self._h, layer_idx, shard_idx)
        if not ptr or size <= 0:
            return np.zeros(0, np.uint8)
        return np.ctypeslib.as_array((ctypes.c_uint8 * size).from_address(ptr))

    # -- staging-slot pool --------------------------------------------------
    def initialize_slot_pool(self, num_slots: int) -> None:
        _capi.check(_capi.load().kvx_manager_initialize_slot_pool(self._h, num_slots),
                    "InitializeSlotPool")

    def acquire_slot(self) -> int:
        out = ctypes.c_int64()
        _capi.check(_capi.load().kvx_manager_acquire_slot(self._h, ctypes.byref(out)),
                    "AcquireSlot")
        return out.value

    def release_slot(self, slot_idx: int) -> None:
        _capi.load().kvx_manager_release_slot(self._h, slot_idx)

    def num_free_slots(self) -> int:
        return int(_capi.load().kvx_manager_num_free_slots(self._h))

    def slot_block_ids(self, slot_idx: int) -> List[int]:
        cap = 4096
        while True:
            out, n = (ctypes.c_int64 * cap)(), ctypes.c_int64()
            _capi.check(_capi.load().kvx_manager_slot_block_ids(self._h, slot_idx, out, cap,
                                                                ctypes.byref(n)))
            if n.value <= cap:
                return list(out[:n.value])
            cap = n.value

    def layer_spans(self, slot_idx: int, num_blocks: int) -> List[dict]:
        """Per-(layer, shard) contiguous host runs of a slot's first blocks."""
        cap = max(self.num_layers * self.num_shards * max(num_blocks, 1), 1)
        out, n = (_capi.HostSpanC * cap)(), ctypes.c_int64()
        _capi.check(_capi.load().kvx_manager_layer_spans(self._h, slot_idx, num_blocks, out,
                                                         cap, ctypes.byref(n)), "LayerSpans")
        keys = ("ptr", "nbytes", "slot_idx", "base_major", "num_major", "layer_idx",
                "shard_idx")
        return [{k: getattr(out[i], k) for k in keys} for i in range(n.value)]

    def issue_h2d(self, slot_idx: int, num_blocks: int, local_block_ids: Sequence[int], *,
                  stream=None) -> dict:
        """Slot host ids -> device ids: {future, host_spans, total_bytes,
        copy_segments} (kv_cache_manager_with_transfer.cc:1751-1805)."""
        ids, n = _capi.i64_array(local_block_ids)
        out, total, segs = ctypes.c_void_p(), ctypes.c_int64(), ctypes.c_int64()
        _capi.check(_capi.load().kvx_manager_issue_h2d(
            self._h, slot_idx, num_blocks, ids, n, ctypes.c_void_p(_stream_ptr(stream)),
            ctypes.byref(out), ctypes.byref(total), ctypes.byref(segs)), "IssueH2D")
        return {"future": RaidenFuture(out, self, "IssueH2D"),
                "host_spans": self.layer_spans(slot_idx, num_blocks),
                "total_bytes": total.value, "copy_segments": segs.value}

    def stage_for_push(self, src_block_ids: Sequence[int], *, stream=None) -> dict:
        """Acquires a slot and stages device blocks into its host ids, one
        future per layer; release the slot with release_slot once consumed."""
        ids, n = _capi.i64_array(src_block_ids)
        layers = self.num_layers
        futs = (ctypes.c_void_p * max(layers, 1))()
        slot, segs = ctypes.c_int64(), ctypes.c_int64()
        host = (ctypes.c_int64 * max(n, 1))()
        _capi.check(_capi.load().kvx_manager_stage_for_push(
            self._h, ids, n, ctypes.c_void_p(_stream_ptr(stream)), ctypes.byref(slot), host,
            futs, ctypes.byref(segs)), "StageForPush")
        return {"slot_idx": slot.value, "host_block_ids": list(host[:n]),
                "layer_futures": [RaidenFuture(ctypes.c_void_p(futs[l]), self, "StageForPush")
                                  for l in range(layers)],
                "copy_segments": segs.value}

    def prepare_load(self, remote_block_ids: Sequence[int], local_block_ids: Sequence[int],
                     local_host_block_ids: Optional[Sequence[int]] = None) -> dict:
        """Host ids for a receive and its load plan: {slot_idx, host_block_ids,
        plan} (slot_idx -1 when the caller gave the host ids)."""
        from .copy_plan import _PlanBuffers
        r, n = _capi.i64_array(remote_block_ids)
        l, nl = _capi.i64_array(local_block_ids)
        if nl != n or (local_host_block_ids is not None and len(local_host_block_ids) != n):
            raise _capi.KvxError(3, "remote_block_ids, local_block_ids, and "
                                    "local_host_block_ids must have same length", "StartRead")
        h = None
        if local_host_block_ids is not None:
            h, _ = _capi.i64_array(local_host_block_ids)
        buf = _PlanBuffers(n)
        slot = ctypes.c_int64()
        host = (ctypes.c_int64 * max(n, 1))()
        _capi.check(_capi.load().kvx_manager_prepare_load(
            self._h, r, l, n, h, ctypes.byref(slot), host, ctypes.byref(buf.out)), "StartRead")
        return {"slot_idx": slot.value, "host_block_ids": list(host[:n]),
                "plan": buf.result(n, remote_block_ids, local_block_ids)}

    # -- block pools -------------------------------------------------------
    def register_pools(self, pools: Sequence[Any]) -> dict:
        """Registers explicit block pools over the wrapped storages
        (tpu_sync/api/torch/kv_cache_manager.py:239-283): Python-side checks
        first, then the library's, which also grows a storage's host mirror
        to the pool's last live byte. Returns the admission summary."""
        from . import pool_layout
        coerced = tuple(pool_layout.coerce_pool_spec(p) for p in pools)
        if not coerced:
            raise ValueError("pool table must be non-empty")
        num_storages = self.num_layers
        for i, p in enumerate(coerced):
            try:
                p.validate()
            except Exception as exc:
                raise ValueError(f"invalid pool {i}: {exc}") from exc
            if p.storage_index >= num_storages:
                raise ValueError(f"pool {i} ({p.tag}) storage_index {p.storage_index} "
                                 f"out of range: manager wraps {num_storages} storages")
        arr, keep = pool_layout.native_pools(coerced)
        _capi.check(_capi.load().kvx_manager_register_pools(self._h, arr, len(coerced)),
                    "KVCacheManager register_pools")
        del keep
        tags = {}
        for p in coerced:
            tags[p.tag] = tags.get(p.tag, 0) + 1
        summary = {"admitted": True, "pools": len(coerced),
                   "storages": len({p.storage_index for p in coerced}), "tags": tags}
        self._admission_summary = dict(summary)
        return dict(summary)

    def admission_summary(self) -> dict:
        summary = getattr(self, "_admission_summary", None)
        return {"admitted": False} if summary is None else dict(summary)

    def num_pools(self) -> int:
        return int(_capi.load().kvx_manager_num_pools(self._h))

    def has_explicit_pools(self) -> bool:
        return bool(_capi.load().kvx_manager_has_explicit_pools(self._h))

    def pool_ids_with_tag(self, tag: str) -> List[int]:
        fn = _capi.load().kvx_manager_pool_indices_with_tag
        cap = max(self.num_pools(), 1)
        out = (ctypes.c_int64 * cap)()
        n = ctypes.c_int64()
        _capi.check(fn(self._h, tag.encode(), out, cap, ctypes.byref(n)))
        return [int(v) for v in out[:n.value]]

    def pool_spec(self, pool_idx: int) -> dict:
        """One pool's descriptor as a dict (pool_layout_nanobind.h:98-112)."""
        lib = _capi.load()
        spec = _capi.PoolSpecC()
        nreg = ctypes.c_int64()
        names = ctypes.c_void_p()
        _capi.check(lib.kvx_manager_pool_spec(self._h, pool_idx, ctypes.byref(spec), None, 0,
                                              ctypes.byref(nreg), ctypes.byref(names)))
        _capi.take_strings(names)
        regs = (_capi.RegionSpecC * max(nreg.value, 1))()
        _capi.check(lib.kvx_manager_pool_spec(self._h, pool_idx, ctypes.byref(spec), regs,
                                              nreg.value, ctypes.byref(nreg),
                                              ctypes.byref(names)))
        s = [b.decode() for b in _capi.take_strings(names)]
        regions = [{"name": s[2 + i], "offset_bytes": regs[i].offset_bytes,
                    "stride_bytes": regs[i].stride_bytes, "unit_bytes": regs[i].unit_bytes,
                    "num_units": regs[i].num_units,
                    "units_per_stride": regs[i].units_per_stride}
                   for i in range(nreg.value)]
        return {"tag": s[0], "storage_index": spec.storage_index,
                "base_offset_bytes": spec.base_offset_bytes,
                "block_stride_bytes": spec.block_stride_bytes,
                "num_blocks": spec.num_blocks, "regions": regions, "dtype_tag": s[1]}

    def get_block_ref(self, pool_idx: int, block_id: int, shard_idx: int = 0) -> dict:
        """Host-side reference to one pool block (pool_layout_nanobind.h:114-129)."""
        ptr, stride = ctypes.c_uint64(), ctypes.c_int64()
        _capi.check(_capi.load().kvx_manager_pool_block_ref(
            self._h, pool_idx, shard_idx, block_id, ctypes.byref(ptr), ctypes.byref(stride)),
            "KVCacheManager get_pool_block_ref")
        spec = self.pool_spec(pool_idx)
        return {"ptr": ptr.value, "block_stride_bytes": stride.value, "tag": spec["tag"],
                "dtype_tag": spec["dtype_tag"], "pool_idx": pool_idx,
                "shard_idx": shard_idx, "block_id": block_id, "regions": spec["regions"]}

    def _pool_copy(self, fn, where, pool_idx, block_ids, shard_idx, stream):
        ids, n = _capi.i64_array(block_ids)
        out = ctypes.c_void_p()
        _capi.check(fn(self._h, pool_idx, ids, n, -1 if shard_idx is None else shard_idx,
                       ctypes.c_void_p(_stream_ptr(stream)), ctypes.byref(out)), where)
        return RaidenFuture(out, self, where)

    def d2h_pool_blocks(self, pool_idx: int, block_ids: Sequence[int],
                        shard_idx: Optional[int] = None, *, stream=None) -> RaidenFuture:
        """Partial D2H of whole pool blocks into the host mirror (live bytes)."""
        return self._pool_copy(_capi.load().kvx_manager_d2h_pool_blocks,
                               "KVCacheManager d2h_pool_blocks", pool_idx, block_ids,
                               shard_idx, stream)

    def h2d_pool_blocks(self, pool_idx: int, block_ids: Sequence[int],
                        shard_idx: Optional[int] = None, *, stream=None) -> RaidenFuture:
        """Partial H2D of whole pool blocks from the host mirror (live bytes)."""
        return self._pool_copy(_capi.load().kvx_manager_h2d_pool_blocks,
                               "KVCacheManager h2d_pool_blocks", pool_idx, block_ids,
                               shard_idx, stream)

    # -- geometry ----------------------------------------------------------
    @property
    def num_layers(self) -> int:
        return _capi.load().kvx_manager_num_layers(self._h)

    @property
    def num_shards(self) -> int:
        return _capi.load().kvx_manager_num_shards(self._h)

    @property
    def host_blocks(self) -> int:
        return _capi.load().kvx_manager_host_blocks(self._h)

    def bytes_per_block(self) -> int:
        return _capi.load().kvx_manager_bytes_per_block(self._h)

    def block_bytes(self, block_array_idx: int) -> int:
        return _capi.load().kvx_manager_block_bytes(self._h, block_array_idx)

    def layer_block_byte_size(self, layer_idx: int) -> int:
        return _capi.load().kvx_manager_layer_block_byte_size(self._h, layer_idx)

    def get_host_pointer(self, layer_idx: int, shard_idx: int = 0) -> int:
        return int(_capi.load().kvx_manager_host_ptr(self._h, layer_idx, shard_idx))

    def get_host_size(self, layer_idx: int, shard_idx: int = 0) -> int:
        return int(_capi.load().kvx_manager_host_size(self._h, layer_idx, shard_idx))

    def get_block_array_host_pointer(self, block_array_idx: int, shard_idx: int = 0) -> int:
        return int(_capi.load().kvx_manager_block_array_host_ptr(self._h, block_array_idx,
                                                                 shard_idx))

    def get_block_array_host_size(self, block_array_idx: int, shard_idx: int = 0) -> int:
        return int(_capi.load().kvx_manager_block_array_host_size(self._h, block_array_idx,
                                                                  shard_idx))

    def get_block_chunks(self, block_array_idx: int, shard_idx: int, block_ids: Sequence[int],
                         total_bytes: int) -> List[Tuple[int, int]]:
        """(host pointer, size) ranges carrying total_bytes of the blocks."""
        ids, n = _capi.i64_array(block_ids)
        cap = 256
        while True:
            ptrs, sizes = (ctypes.c_uint64 * cap)(), (ctypes.c_int64 * cap)()
            got = ctypes.c_int64()
            _capi.check(_capi.load().kvx_manager_block_chunks(
                self._h, block_array_idx, shard_idx, ids, n, total_bytes, ptrs, sizes, cap,
                ctypes.byref(got)))
            if got.value <= cap:
                return [(ptrs[i], sizes[i]) for i in range(got.value)]
            cap = got.value

    def num_block_arrays(self) -> int:
        return _capi.load().kvx_manager_num_block_arrays(self._h)

    def get_allocated_host_dram_bytes(self) -> int:
        return _capi.load().kvx_manager_allocated_host_bytes(self._h)

    def host_block_manager(self) -> LogicalBlockManager:
        h = _capi.load().kvx_manager_host_block_manager(self._h)
        return LogicalBlockManager(_handle=ctypes.c_void_p(h), _owner=self)

    def wait_for_pending_work(self) -> None:
        _capi.check(_capi.load().kvx_manager_wait_for_pending_work(self._h))

    def engine_stats(self) -> dict:
        out = (ctypes.c_int64 * 8)()
        _capi.check(_capi.load().kvx_manager_engine_stats(self._h, out))
        keys = ("direct_copies", "staged_copies", "memcpy_calls", "kernel_launches",
                "chunks", "zero_copy_copies", "extent_kernel_copies", "bounce_copies")
        return dict(zip(keys, list(out)))

    @property
    def stream_placement(self) -> dict:
        """How the transfer engine's four streams landed on hardware queues:
        a probe at creation (one short kernel per stream, all at once) finds
        pairs that ran one after the other, i.e. share a queue, and such a
        set is created again, up to 3 times. serialized_pairs: pairs left on
        one queue (0: each on its own; -1: the probe could not run);
        attempts: stream sets created."""
        out = (ctypes.c_int32 * 2)()
        _capi.check(_capi.load().kvx_manager_stream_placement(self._h, out))
        return {"serialized_pairs": int(out[0]), "attempts": int(out[1])}

    @property
    def lane_dma_engines(self) -> Optional[Tuple[int, int]]:
        """SDMA engine bits (device-to-host, host-to-device) of the pageable
        lanes' DMAs; None while no lane has run or when they use
        hipMemcpyAsync."""
        v = int(_capi.load().kvx_manager_lane_dma_engines(self._h))
        if v < 0:
            raise RuntimeError("lane_dma_engines: manager has no transfer engine")
        return (v >> 16, v & 0xFFFF) if v else None

    def kernel_times(self, gather: bool = True, reset: bool = False) -> dict:
        """Profiled launches of the gather (or scatter) kernel: count, total ms
        (HIP events on the kernel's stream) and algorithmic HBM bytes."""
        n, ms, nbytes = ctypes.c_int64(), ctypes.c_double(), ctypes.c_int64()
        _capi.check(_capi.load().kvx_manager_kernel_times(
            self._h, int(gather), int(reset), ctypes.byref(n), ctypes.byref(ms),
            ctypes.byref(nbytes)))
        return {"launches": n.value, "total_ms": ms.value, "bytes": nbytes.value}

    def close(self) -> None:
        h, self._h = getattr(self, "_h", None), None
        lib = _capi._lib if _capi is not None else None  # None at interpreter exit
        if h and lib is not None:
            lib.kvx_manager_destroy(h)

    def __del__(self):
        self.close()
