"""MI355X-native KV block extract/insert and pinned-host offload/reload.

Import name ``tpu_sync_amd``; the package lives in the ``tpu-sync_amd``
directory. The compute path is libkvx.so (host C++ + gfx950 HIP kernels);
this package is a thin ctypes layer that only passes pointers.
"""
from . import _capi
from ._capi import KvxError
from .kv_cache_manager import (KVCacheManager, LogicalBlockManager, RaidenFuture,
                               probe_stream_queues, measure_link_peaks)
from .kv_cache_store import (BlockStatus, KVCacheMetadata, KVCacheMetadataShmRegion,
                             KVCacheStore, LRUCache, RaidenBlockId, RaidenId)
from . import copy_plan, pool_layout, tiling, transport
from .pool_layout import PoolSpec, RegionSpec
from .weight_synchronizer import (StridedEntry, StridedPlan, WeightSynchronizer,
                                  column_split_entries, compute_nd_shard_slices, copy_strided)

__all__ = ["KVCacheManager", "LogicalBlockManager", "RaidenFuture", "KvxError", "probe_stream_queues", "measure_link_peaks",
           "KVCacheStore", "RaidenId", "RaidenBlockId", "BlockStatus", "LRUCache",
           "KVCacheMetadata", "KVCacheMetadataShmRegion", "WeightSynchronizer",
           "StridedEntry", "StridedPlan", "copy_strided", "column_split_entries",
           "compute_nd_shard_slices", "pool_layout", "copy_plan", "tiling", "transport", "PoolSpec", "RegionSpec",
           "library_path"]


def library_path() -> str:
    return _capi.LIB_PATH
