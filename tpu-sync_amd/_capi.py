"""ctypes binding of libkvx.so (the C-ABI declared in include/kvx.h).

Only pointers and sizes cross this boundary: device tensors are passed as
``tensor.data_ptr()``, streams as ``stream.cuda_stream``. The library must
have been built (``make -C tpu-sync_amd/csrc``); importing this module
without it raises, there is no fallback path.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
# KVX_LIBRARY names another build of the same library (the sanitizer builds of
# the Makefile's asan / tsan targets); by default the in-tree libkvx.so.
LIB_PATH = os.environ.get("KVX_LIBRARY") or os.path.join(_HERE, "libkvx.so")

STATUS_NAMES = {
    0: "OK", 1: "CANCELLED", 2: "UNKNOWN", 3: "INVALID_ARGUMENT",
    4: "DEADLINE_EXCEEDED", 5: "NOT_FOUND", 6: "ALREADY_EXISTS",
    7: "PERMISSION_DENIED", 8: "RESOURCE_EXHAUSTED", 9: "FAILED_PRECONDITION",
    10: "ABORTED", 11: "OUT_OF_RANGE", 12: "UNIMPLEMENTED", 13: "INTERNAL",
    14: "UNAVAILABLE", 15: "DATA_LOSS",
}

HOST_MALLOC, HOST_PINNED, HOST_SHM, HOST_AUTO = 0, 1, 2, 3
MODES = {"auto": 0, "staged": 1, "zero_copy": 2, "lanes": 3}
LAYER_MAJOR, BLOCK_MAJOR = 0, 1


class KvxError(RuntimeError):
    """A non-OK status from libkvx; ``code`` is the absl::StatusCode number."""

    def __init__(self, code, message, where=""):
        self.code = code
        self.status = STATUS_NAMES.get(code, str(code))
        prefix = f"{where} failed: " if where else ""
        super().__init__(f"{prefix}{message}")


class ManagerConfig(ctypes.Structure):
    _fields_ = [
        ("device", ctypes.c_int32),
        ("host_alloc", ctypes.c_int32),
        ("num_layers", ctypes.c_int64),
        ("num_shards", ctypes.c_int64),
        ("device_ptrs", ctypes.POINTER(ctypes.c_uint64)),
        ("device_bytes", ctypes.POINTER(ctypes.c_int64)),
        ("major_dim", ctypes.c_int64),
        ("slice_byte_size", ctypes.c_int64),
        ("host_blocks", ctypes.c_int64),
        ("staging_chunk_bytes", ctypes.c_int64),
        ("staging_chunks", ctypes.c_int64),
        ("direct_min_bytes", ctypes.c_int64),
        ("shm_key", ctypes.c_char_p),
        ("shm_server_name", ctypes.c_char_p),
        ("model_uid", ctypes.c_char_p),
        ("profile_kernels", ctypes.c_int32),
        ("transfer_mode", ctypes.c_int32),
        ("zero_copy_workgroups", ctypes.c_int64),
        ("numa_policy", ctypes.c_int32),
        ("numa_node", ctypes.c_int32),
        ("dispatch", ctypes.c_int32),
        ("host_copy_threads", ctypes.c_int32),
        ("gather_workgroups_per_cu", ctypes.c_int32),
    ]


class BlockSlice(ctypes.Structure):
    """kvx_block_slice: RaidenBlockId across the C-ABI."""
    _fields_ = [
        ("host_block_id", ctypes.c_int32),
        ("device_block_id", ctypes.c_int32),
        ("status", ctypes.c_int32),
        ("data_replica_idx", ctypes.c_int32),
        ("job_name", ctypes.c_char_p),
        ("job_replica_id", ctypes.c_char_p),
        ("data_name", ctypes.c_char_p),
    ]


class StoreConfig(ctypes.Structure):
    _fields_ = [
        ("capacity", ctypes.c_int64),
        ("job_name", ctypes.c_char_p),
        ("job_replica_id", ctypes.c_char_p),
        ("data_name", ctypes.c_char_p),
        ("data_replica_idx", ctypes.c_int32),
        ("num_shards", ctypes.c_int32),
        ("shard_size_bytes", ctypes.c_int64),
        ("store_server_ip", ctypes.c_char_p),
        ("raiden_controller_port", ctypes.c_int32),
        ("metadata_shm_key", ctypes.c_char_p),
        ("model_uid", ctypes.c_char_p),
        ("no_auto_recover", ctypes.c_int32),
        ("host_blocks", ctypes.c_int64),
    ]


class TiledLayoutC(ctypes.Structure):
    _fields_ = [
        ("itemsize", ctypes.c_int32),
        ("rank", ctypes.c_int32),
        ("dims", ctypes.c_int64 * 8),
        ("minor_to_major", ctypes.c_int32 * 8),
        ("num_tiles", ctypes.c_int32),
        ("tile_rank", ctypes.c_int32 * 4),
        ("reserved", ctypes.c_int32),
        ("tile_dims", (ctypes.c_int64 * 8) * 4),
    ]


class WeightSyncConfig(ctypes.Structure):
    _fields_ = [
        ("device", ctypes.c_int32),
        ("host_alloc", ctypes.c_int32),
        ("num_layers", ctypes.c_int64),
        ("num_shards", ctypes.c_int64),
        ("device_ptrs", ctypes.POINTER(ctypes.c_uint64)),
        ("device_bytes", ctypes.POINTER(ctypes.c_int64)),
        ("chunk_bytes", ctypes.c_int64),
        ("staging_chunks", ctypes.c_int64),
        ("profile_kernels", ctypes.c_int32),
        ("numa_off", ctypes.c_int32),
        ("layouts", ctypes.POINTER(TiledLayoutC)),
    ]


class StridedEntryC(ctypes.Structure):
    _fields_ = [
        ("src", ctypes.c_uint64),
        ("dst", ctypes.c_uint64),
        ("src_offset_bytes", ctypes.c_int64),
        ("dst_offset_bytes", ctypes.c_int64),
        ("size_bytes", ctypes.c_int64),
        ("count", ctypes.c_int64),
        ("src_stride_bytes", ctypes.c_int64),
        ("dst_stride_bytes", ctypes.c_int64),
    ]


class RegionSpecC(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char_p),
        ("offset_bytes", ctypes.c_int64),
        ("stride_bytes", ctypes.c_int64),
        ("unit_bytes", ctypes.c_int64),
        ("num_units", ctypes.c_int64),
        ("units_per_stride", ctypes.c_int64),
    ]


class PoolSpecC(ctypes.Structure):
    _fields_ = [
        ("tag", ctypes.c_char_p),
        ("storage_index", ctypes.c_int64),
        ("base_offset_bytes", ctypes.c_int64),
        ("block_stride_bytes", ctypes.c_int64),
        ("num_blocks", ctypes.c_int64),
        ("regions", ctypes.POINTER(RegionSpecC)),
        ("num_regions", ctypes.c_int64),
        ("dtype_tag", ctypes.c_char_p),
    ]


class LoadPlanOut(ctypes.Structure):
    _fields_ = [
        ("producer_remote_block_ids", ctypes.POINTER(ctypes.c_int64)),
        ("transport_host_block_ids", ctypes.POINTER(ctypes.c_int64)),
        ("h2d_local_block_ids", ctypes.POINTER(ctypes.c_int64)),
        ("h2d_host_block_ids", ctypes.POINTER(ctypes.c_int64)),
        ("num_h2d", ctypes.c_int64),
        ("h2d_src", ctypes.POINTER(ctypes.c_int64)),
        ("h2d_dst", ctypes.POINTER(ctypes.c_int64)),
        ("h2d_sizes", ctypes.POINTER(ctypes.c_int64)),
        ("num_runs", ctypes.c_int64),
    ]


class HostSpanC(ctypes.Structure):
    _fields_ = [
        ("ptr", ctypes.c_uint64),
        ("nbytes", ctypes.c_int64),
        ("slot_idx", ctypes.c_int64),
        ("base_major", ctypes.c_int64),
        ("num_major", ctypes.c_int64),
        ("layer_idx", ctypes.c_int64),
        ("shard_idx", ctypes.c_int64),
    ]


class ChunkHeaderC(ctypes.Structure):
    _fields_ = [
        ("version", ctypes.c_uint16),
        ("op", ctypes.c_uint8),
        ("flags", ctypes.c_uint8),
        ("buffer_id", ctypes.c_uint16),
        ("reserved", ctypes.c_uint16),
        ("metadata_size", ctypes.c_uint16),
        ("remote_id", ctypes.c_uint32),
        ("local_id", ctypes.c_uint32),
        ("count_or_size", ctypes.c_uint32),
        ("uuid", ctypes.c_uint64),
    ]


class ChunkMetadataC(ctypes.Structure):
    _fields_ = [
        ("layer_idx", ctypes.c_uint32),
        ("dst_shard_idx", ctypes.c_uint32),
        ("dst_offset_bytes", ctypes.c_uint64),
        ("size_bytes", ctypes.c_uint64),
    ]


class PushItemC(ctypes.Structure):
    _fields_ = [(k, ctypes.c_int64) for k in ("layer", "shard", "k", "staging_offset", "size")]


# kvx_ready_fn(user, code)
READY_FN = ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.c_int32)

# kvx_transfer_fn(user, d2h, src, dst, n) -> status
TRANSFER_FN = ctypes.CFUNCTYPE(ctypes.c_int32, ctypes.c_void_p, ctypes.c_int32,
                               ctypes.POINTER(ctypes.c_int64),
                               ctypes.POINTER(ctypes.c_int64), ctypes.c_int64)


_i32, _i64, _u64 = ctypes.c_int32, ctypes.c_int64, ctypes.c_uint64
_vp, _i64p, _i32p = ctypes.c_void_p, ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int32)
_u64p = ctypes.POINTER(ctypes.c_uint64)
_int = ctypes.c_int

# name: (restype, argtypes)
PROTOTYPES = {
    "kvx_last_error": (ctypes.c_char_p, []),
    "kvx_version": (ctypes.c_char_p, []),
    "kvx_manager_create": (_int, [ctypes.POINTER(ManagerConfig), ctypes.POINTER(_vp)]),
    "kvx_manager_destroy": (None, [_vp]),
    "kvx_manager_d2h": (_int, [_vp, _i64p, _i64, _i64p, _i64, _i64p, _i64, _i64, _i64,
                               _i64, _vp, ctypes.POINTER(_vp)]),
    "kvx_manager_h2d": (_int, [_vp, _i64p, _i64, _i64p, _i64, _i64p, _i64, _i64, _i64,
                               _i64, _vp, ctypes.POINTER(_vp)]),
    "kvx_manager_d2h_auto_allocate": (_int, [_vp, _i64p, _i64, _i64p, _i64, _i32p, _i64,
                                             _i64p, _vp, ctypes.POINTER(_vp)]),
    "kvx_manager_gather": (_int, [_vp, _i64p, _i64, _u64, _i64, _i32, _i64, _i64, _vp,
                                  ctypes.POINTER(_vp)]),
    "kvx_manager_scatter": (_int, [_vp, _i64p, _i64, _u64, _i64, _i32, _i64, _i64, _vp,
                                   ctypes.POINTER(_vp)]),
    "kvx_manager_gather_no_alloc": (_int, [_vp, _i64p, _i64, _u64, _i64, _i32, _i64, _i64,
                                           _vp]),
    "kvx_manager_configure_host_staging_slots": (_int, [_vp, _i64, _i64]),
    "kvx_manager_host_span": (_int, [_vp, _i64, _i64, _i64, _i64, _u64p, _i64p, _i64p]),
    "kvx_manager_block_host_ptr": (_int, [_vp, _i64, _i64, _i32, _u64p]),
    "kvx_manager_read_block": (_int, [_vp, _i64, _i32, _i64, _vp, _i64]),
    "kvx_manager_write_block": (_int, [_vp, _i64, _i32, _i64, _vp, _i64]),
    "kvx_manager_num_layers": (_i64, [_vp]),
    "kvx_manager_num_shards": (_i64, [_vp]),
    "kvx_manager_major_dim": (_i64, [_vp]),
    "kvx_manager_host_blocks": (_i64, [_vp]),
    "kvx_manager_bytes_per_block": (_i64, [_vp]),
    "kvx_manager_layer_block_byte_size": (_i64, [_vp, _i64]),
    "kvx_manager_num_block_arrays": (_i64, [_vp]),
    "kvx_manager_block_bytes": (_i64, [_vp, _i64]),
    "kvx_manager_block_array_host_ptr": (_u64, [_vp, _i64, _i64]),
    "kvx_manager_block_array_host_size": (_i64, [_vp, _i64, _i64]),
    "kvx_manager_allocated_host_bytes": (_i64, [_vp]),
    "kvx_manager_wait_for_pending_work": (_int, [_vp]),
    "kvx_manager_engine_stats": (_int, [_vp, _i64p]),
    "kvx_manager_lane_dma_engines": (ctypes.c_int32, [_vp]),
    "kvx_manager_stream_placement": (_int, [_vp, _i32p]),
    "kvx_probe_stream_queues": (_int, [_u64p, _i32, _i32p]),
    "kvx_measure_link_peaks": (_int, [ctypes.c_uint64, _i32, ctypes.POINTER(ctypes.c_double),
                                      ctypes.POINTER(ctypes.c_uint32)]),
    "kvx_manager_kernel_times": (_int, [_vp, _i32, _i32, _i64p,
                                        ctypes.POINTER(ctypes.c_double), _i64p]),
    "kvx_future_is_ready": (_int, [_vp]),
    "kvx_future_poll_error": (_int, [_vp]),
    "kvx_future_await": (_int, [_vp]),
    "kvx_future_wait_on_stream": (_int, [_vp, _vp]),
    "kvx_future_on_ready": (_int, [_vp, ctypes.c_void_p, _vp]),
    "kvx_future_release": (None, [_vp]),
    "kvx_block_manager_create": (_int, [_i32, ctypes.POINTER(_vp)]),
    "kvx_block_manager_destroy": (None, [_vp]),
    "kvx_manager_host_block_manager": (_vp, [_vp]),
    "kvx_block_manager_allocate": (_int, [_vp, _i32, _i32, _i32p]),
    "kvx_block_manager_allocate_target": (_int, [_vp, _i32p, _i64]),
    "kvx_block_manager_unlock": (_int, [_vp, _i32p, _i64]),
    "kvx_block_manager_deallocate": (_int, [_vp, _i32p, _i64]),
    "kvx_block_manager_access": (_int, [_vp, _i32]),
    "kvx_block_manager_is_allocated": (_i32, [_vp, _i32]),
    "kvx_block_manager_is_locked": (_i32, [_vp, _i32]),
    "kvx_block_manager_total_blocks": (_i32, [_vp]),
    "kvx_block_manager_num_free": (_i32, [_vp]),
    "kvx_block_manager_num_allocated": (_i32, [_vp]),
    "kvx_block_manager_num_locked": (_i32, [_vp]),
    "kvx_gather_blocks": (_int, [_u64, _i64, _i64, _i64, _u64, _i64, _u64, _i32, _u64, _vp]),
    "kvx_scatter_blocks": (_int, [_u64, _i64, _i64, _i64, _u64, _i64, _u64, _i32, _u64, _vp]),
    "kvx_manager_register_with_controller": (_int, [_vp, ctypes.c_char_p]),
    "kvx_manager_host_alloc": (_i32, [_vp]),
    "kvx_manager_shm_warm": (_i32, [_vp]),
    # host tier
    "kvx_strings_count": (_i64, [_vp]),
    "kvx_strings_get": (_int, [_vp, _i64, ctypes.POINTER(_vp), _i64p]),
    "kvx_strings_release": (None, [_vp]),
    "kvx_strings_flat": (_int, [_vp, ctypes.POINTER(_vp), ctypes.POINTER(_i64p)]),
    "kvx_slices_count": (_i64, [_vp]),
    "kvx_slices_get": (_int, [_vp, _i64, ctypes.POINTER(_vp), _i64p,
                              ctypes.POINTER(BlockSlice)]),
    "kvx_slices_release": (None, [_vp]),
    "kvx_slices_flat": (_int, [_vp, ctypes.POINTER(_vp), ctypes.POINTER(_i64p),
                               ctypes.POINTER(ctypes.POINTER(BlockSlice))]),
    "kvx_store_create": (_int, [ctypes.POINTER(StoreConfig), ctypes.POINTER(_vp)]),
    "kvx_store_destroy": (None, [_vp]),
    "kvx_store_controller_address": (ctypes.c_char_p, [_vp]),
    "kvx_store_capacity": (_i64, [_vp]),
    "kvx_store_size": (_i64, [_vp]),
    "kvx_store_recovered_blocks": (_i64, [_vp]),
    "kvx_store_metadata_warm": (_i32, [_vp]),
    "kvx_store_host_block_manager": (_vp, [_vp]),
    "kvx_store_lookup": (_int, [_vp, _vp, _i64p, _i64, _i32, ctypes.POINTER(_vp)]),
    "kvx_store_insert": (_int, [_vp, _vp, _i64p, _i64, ctypes.POINTER(BlockSlice), _i64,
                                _i32]),
    "kvx_store_release": (_int, [_vp, _vp, _i64p, _i64]),
    "kvx_store_save": (_int, [_vp, _vp, _i64p, _i64]),
    "kvx_store_load": (_int, [_vp, _vp, _i64p, _i64, _i32p, _i64]),
    "kvx_store_load_slices": (_int, [_vp, _vp, _i64p, _i64, ctypes.POINTER(BlockSlice), _i64,
                                     _i32p, _i64]),
    "kvx_store_poll_save_status": (_int, [_vp, ctypes.POINTER(_vp)]),
    "kvx_store_poll_load_status": (_int, [_vp, ctypes.POINTER(_vp)]),
    "kvx_store_pin_count": (_i32, [_vp, _vp, _i64]),
    "kvx_store_recover_from_local_manifest": (_int, [_vp, _i64p]),
    "kvx_store_evictable_keys": (_int, [_vp, _i64, ctypes.POINTER(_vp)]),
    "kvx_store_evict": (_int, [_vp, _vp, _i64p, _i64, _i64p]),
    "kvx_store_candidate_keys": (_int, [_vp, ctypes.POINTER(_vp)]),
    "kvx_store_set_transfer_fn": (_int, [_vp, TRANSFER_FN, _vp]),
    "kvx_lru_create": (_int, [_i64, ctypes.POINTER(_vp)]),
    "kvx_lru_destroy": (None, [_vp]),
    "kvx_lru_put": (_int, [_vp, _vp, _i64, _i64, _i32p, ctypes.POINTER(_vp), _i64p]),
    "kvx_lru_put_back": (_int, [_vp, _vp, _i64, _i64]),
    "kvx_lru_find": (_i32, [_vp, _i32, _vp, _i64, _i64p]),
    "kvx_lru_contains": (_i32, [_vp, _vp, _i64]),
    "kvx_lru_pin": (_i32, [_vp, _vp, _i64]),
    "kvx_lru_unpin": (_i32, [_vp, _vp, _i64]),
    "kvx_lru_erase": (_i32, [_vp, _vp, _i64]),
    "kvx_lru_pin_count": (_i32, [_vp, _vp, _i64]),
    "kvx_lru_evict": (_i32, [_vp, ctypes.POINTER(_vp), _i64p]),
    "kvx_lru_evictable_keys": (_int, [_vp, _i64, ctypes.POINTER(_vp)]),
    "kvx_lru_candidate_keys": (_int, [_vp, ctypes.POINTER(_vp)]),
    "kvx_lru_clear": (None, [_vp]),
    "kvx_lru_sizes": (_int, [_vp, _i64p]),
    "kvx_metadata_required_size": (_i64, [_i32]),
    "kvx_metadata_format": (_int, [_vp, _i64, _i32, ctypes.c_char_p]),
    "kvx_metadata_attach": (_int, [_vp, _i64, _i32, ctypes.c_char_p]),
    "kvx_metadata_set": (_int, [_vp, _i64, _i32, ctypes.c_char_p, _i32, _vp, _i64, _u64]),
    "kvx_metadata_clear": (_int, [_vp, _i64, _i32, ctypes.c_char_p, _i32]),
    "kvx_metadata_valid_entries": (_int, [_vp, _i64, _i32, ctypes.c_char_p, _i32p, _u64p,
                                          _i64p, ctypes.POINTER(_vp)]),
    "kvx_metadata_shm_attach_or_format": (_int, [ctypes.c_char_p, _i32, ctypes.c_char_p,
                                                 ctypes.POINTER(_vp), _i32p]),
    "kvx_metadata_shm_region": (_int, [_vp, _u64p, _i64p]),
    "kvx_metadata_shm_reformat": (_int, [_vp]),
    "kvx_metadata_shm_release": (None, [_vp]),
    # weight sync
    "kvx_weight_sync_create": (_int, [ctypes.POINTER(WeightSyncConfig), ctypes.POINTER(_vp)]),
    "kvx_weight_sync_destroy": (None, [_vp]),
    "kvx_weight_sync_d2h": (_int, [_vp, _vp, ctypes.POINTER(_vp)]),
    "kvx_weight_sync_h2d": (_int, [_vp, _vp, ctypes.POINTER(_vp)]),
    "kvx_weight_sync_d2h_layer": (_int, [_vp, _i64, _vp, ctypes.POINTER(_vp)]),
    "kvx_weight_sync_h2d_layer": (_int, [_vp, _i64, _vp, ctypes.POINTER(_vp)]),
    "kvx_weight_sync_pack": (_int, [_vp, _u64, _i64, _vp, ctypes.POINTER(_vp)]),
    "kvx_weight_sync_unpack": (_int, [_vp, _u64, _i64, _vp, ctypes.POINTER(_vp)]),
    "kvx_weight_sync_total_bytes": (_i64, [_vp]),
    "kvx_weight_sync_host_base": (_u64, [_vp]),
    "kvx_weight_sync_host_buffer": (_int, [_vp, _i64, _i64, _u64p, _i64p, _i64p]),
    "kvx_weight_sync_wait": (_int, [_vp]),
    "kvx_weight_sync_kernel_times": (_int, [_vp, _i32, _i32, _i64p,
                                            ctypes.POINTER(ctypes.c_double), _i64p]),
    "kvx_copy_strided": (_int, [_i32, ctypes.POINTER(StridedEntryC), _i64, _vp,
                                ctypes.POINTER(_vp)]),
    "kvx_strided_plan_create": (_int, [_i32, ctypes.POINTER(StridedEntryC), _i64,
                                       ctypes.POINTER(_vp)]),
    "kvx_strided_plan_run": (_int, [_vp, _vp, ctypes.POINTER(_vp)]),
    "kvx_strided_plan_destroy": (None, [_vp]),
    "kvx_strided_plan_profile": (_int, [_vp, _i32]),
    "kvx_strided_plan_kernel_times": (_int, [_vp, _i32, _i64p, ctypes.POINTER(ctypes.c_double),
                                             _i64p]),
    "kvx_tiled_buffer_elements": (_int, [ctypes.POINTER(TiledLayoutC), ctypes.POINTER(_i64)]),
    "kvx_tile_buffer": (_int, [_i32, ctypes.POINTER(TiledLayoutC), _u64, _u64, _vp,
                               ctypes.POINTER(_vp)]),
    "kvx_detile_buffer": (_int, [_i32, ctypes.POINTER(TiledLayoutC), _u64, _u64, _vp,
                                 ctypes.POINTER(_vp)]),
    "kvx_manager_numa_node": (_i32, [_vp]),
    "kvx_manager_host_ptr": (_u64, [_vp, _i64, _i64]),
    "kvx_manager_host_size": (_i64, [_vp, _i64, _i64]),
    "kvx_manager_block_array_block_ptr": (_u64, [_vp, _i64, _i64, _i64]),
    "kvx_manager_block_chunks": (_int, [_vp, _i64, _i64, _i64p, _i64, _i64, _u64p, _i64p, _i64,
                                        _i64p]),
    "kvx_manager_queued_dispatch": (_i32, [_vp]),
    "kvx_manager_dispatch_log": (_int, [_vp, ctypes.c_char_p, _i64, _i64p]),
    "kvx_gpu_numa_node": (_i32, [_i32]),
    "kvx_host_page_numa_node": (_i32, [_u64]),
    "kvx_numa_pin_current_thread": (_int, [_i32]),
    "kvx_chunk_header_serialize": (None, [ctypes.POINTER(ChunkHeaderC), ctypes.c_char_p]),
    "kvx_chunk_header_deserialize": (_int, [ctypes.c_char_p, _i64, ctypes.POINTER(ChunkHeaderC)]),
    "kvx_chunk_metadata_serialize": (None, [ctypes.POINTER(ChunkMetadataC), ctypes.c_char_p]),
    "kvx_chunk_metadata_deserialize": (_int, [ctypes.c_char_p, _i64, _i32,
                                              ctypes.POINTER(ChunkMetadataC)]),
    "kvx_block_ids_serialize": (None, [_i64p, _i64, ctypes.c_char_p]),
    "kvx_block_ids_deserialize": (None, [ctypes.c_char_p, _i64, _i64p]),
    "kvx_manager_build_push_frame": (_int, [_vp, _u64, ctypes.c_uint32, _i64, _i32, _i32, _i64p,
                                            _i64p, _i64, ctypes.c_char_p, ctypes.c_char_p,
                                            ctypes.c_char_p, ctypes.POINTER(PushItemC), _i64,
                                            _i64p, _i64p]),
    "kvx_manager_parse_push_stream": (_int, [_vp, ctypes.c_char_p, _i64, _vp, _i64,
                                             ctypes.POINTER(ChunkHeaderC), _i64p, _i32p, _i64p,
                                             _i64p, _i64, _i64p, _i64p]),
    "kvx_offsets_impl": (_int, [_i64p, _i64, _i32, _i64p, _i64p, _i64p, _i64p]),
    "kvx_build_coalesced_copy_spec": (_int, [_i64p, _i64p, _i64, _i64p, _i64p, _i64p,
                                             _i64p]),
    "kvx_build_load_copy_plan": (_int, [_i64p, _i64p, _i64p, _i64,
                                        ctypes.POINTER(LoadPlanOut)]),
    "kvx_manager_initialize_slot_pool": (_int, [_vp, _i64]),
    "kvx_manager_acquire_slot": (_int, [_vp, _i64p]),
    "kvx_manager_release_slot": (None, [_vp, _i64]),
    "kvx_manager_num_free_slots": (_i64, [_vp]),
    "kvx_manager_slot_block_ids": (_int, [_vp, _i64, _i64p, _i64, _i64p]),
    "kvx_manager_layer_spans": (_int, [_vp, _i64, _i64, ctypes.POINTER(HostSpanC), _i64,
                                       _i64p]),
    "kvx_manager_issue_h2d": (_int, [_vp, _i64, _i64, _i64p, _i64, _vp, ctypes.POINTER(_vp),
                                     _i64p, _i64p]),
    "kvx_manager_stage_for_push": (_int, [_vp, _i64p, _i64, _vp, _i64p, _i64p,
                                          ctypes.POINTER(_vp), _i64p]),
    "kvx_manager_prepare_load": (_int, [_vp, _i64p, _i64p, _i64, _i64p, _i64p, _i64p,
                                        ctypes.POINTER(LoadPlanOut)]),
    "kvx_pool_validate": (_int, [ctypes.POINTER(PoolSpecC), _i64]),
    "kvx_pool_storage_extent_end": (_i64, [ctypes.POINTER(PoolSpecC)]),
    "kvx_pool_copy_extents": (_int, [ctypes.POINTER(PoolSpecC), _i64p, _i64, _i64p, _i64,
                                     _i64p]),
    "kvx_pool_live_segments": (_int, [ctypes.POINTER(PoolSpecC), _i64p, _i64, _i64p]),
    "kvx_pool_physical_to_logical": (_int, [ctypes.POINTER(PoolSpecC), _i64, _i64, _i64p,
                                            _i64p]),
    "kvx_pool_translate_live_copy": (_int, [ctypes.POINTER(PoolSpecC),
                                            ctypes.POINTER(PoolSpecC), _i64, _i64, _i64,
                                            _i64p, _i64, _i64p]),
    "kvx_regions_cover_range": (_i32, [ctypes.POINTER(RegionSpecC), _i64, _i64, _i64]),
    "kvx_manager_register_pools": (_int, [_vp, ctypes.POINTER(PoolSpecC), _i64]),
    "kvx_manager_num_pools": (_i64, [_vp]),
    "kvx_manager_has_explicit_pools": (_i32, [_vp]),
    "kvx_manager_pool_indices_with_tag": (_int, [_vp, ctypes.c_char_p, _i64p, _i64, _i64p]),
    "kvx_manager_pool_spec": (_int, [_vp, _i64, ctypes.POINTER(PoolSpecC),
                                     ctypes.POINTER(RegionSpecC), _i64, _i64p,
                                     ctypes.POINTER(_vp)]),
    "kvx_manager_pool_block_ref": (_int, [_vp, _i64, _i64, _i64, _u64p, _i64p]),
    "kvx_manager_d2h_pool_blocks": (_int, [_vp, _i64, _i64p, _i64, _i64, _vp,
                                           ctypes.POINTER(_vp)]),
    "kvx_manager_h2d_pool_blocks": (_int, [_vp, _i64, _i64p, _i64, _i64, _vp,
                                           ctypes.POINTER(_vp)]),
}

_lib = None


def load():
    """Loads libkvx.so once and declares every prototype."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `make -C tpu-sync_amd/csrc` "
            "(or __graft_entry__.build()); there is no CPU fallback")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in PROTOTYPES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def last_error():
    return load().kvx_last_error().decode(errors="replace")


def device_buffer(t, what, device=None):
    """(data_ptr, nbytes) of a tensor handed to a kernel, checked before any
    launch. A tensor that is not on a HIP device, is on another device than
    ``device``, is not contiguous (an expanded or strided view), or claims
    more bytes than its storage holds past its offset raises ValueError:
    the kernels address numel * element_size bytes from data_ptr."""
    if not getattr(t, "is_cuda", False):
        raise ValueError(f"{what} must be a tensor on a HIP device, got {getattr(t, 'device', t)}")
    index = t.device.index if t.device.index is not None else 0
    if device is not None and index != device:
        raise ValueError(f"{what} is on device {index}, expected device {device}")
    if not t.is_contiguous():
        raise ValueError(f"{what} must be contiguous")
    nbytes = t.numel() * t.element_size()
    held = t.untyped_storage().nbytes() - t.storage_offset() * t.element_size()
    if nbytes > held:
        raise ValueError(f"{what} spans {nbytes} bytes but its storage holds {held}")
    return t.data_ptr(), nbytes


def check(code, where=""):
    if code != 0:
        raise KvxError(code, last_error(), where)


def i64_array(values):
    vals = [int(v) for v in values]
    arr = (ctypes.c_int64 * max(len(vals), 1))(*vals)
    return arr, len(vals)


def i32_array(values):
    vals = [int(v) for v in values]
    arr = (ctypes.c_int32 * max(len(vals), 1))(*vals)
    return arr, len(vals)


def pack_bytes(items):
    """Packs byte strings back to back: (buffer, offsets[n + 1], n). The
    offsets pointer keeps its numpy array alive."""
    import numpy as np
    items = [b if type(b) is bytes else bytes(b) for b in items]
    n = len(items)
    offs = np.zeros(n + 1, dtype=np.int64)
    if n:
        np.cumsum(np.fromiter(map(len, items), dtype=np.int64, count=n), out=offs[1:])
    blob = b"".join(items)
    buf = ctypes.create_string_buffer(blob, max(len(blob), 1))
    return buf, offs.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)), n


def split_flat(data, offsets, n):
    """Items [offsets[i], offsets[i + 1]) of a flat byte buffer of n items."""
    if n == 0:
        return []
    offs = offsets[:n + 1]
    blob = ctypes.string_at(data, offs[n]) if offs[n] else b""
    return [blob[offs[i]:offs[i + 1]] for i in range(n)]


def take_strings(handle):
    """Copies a kvx_strings list into Python bytes (one library call for the
    whole list) and releases it."""
    lib = load()
    if not handle:
        return []
    try:
        n = lib.kvx_strings_count(handle)
        if n == 0:
            return []
        data, offsets = ctypes.c_void_p(), _i64p()
        check(lib.kvx_strings_flat(handle, ctypes.byref(data), ctypes.byref(offsets)))
        return split_flat(data, offsets, n)
    finally:
        lib.kvx_strings_release(handle)
