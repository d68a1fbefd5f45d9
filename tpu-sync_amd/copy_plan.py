"""Block-id lists to run-coalesced copy specs and the receive-side load plan
(tpu_sync/core/kv_cache_manager_with_transfer.cc:294-426), computed by the
library. A spec is a dict of parallel lists ``src_offsets``, ``dst_offsets``,
``sizes`` (in blocks)."""
from __future__ import annotations

import ctypes
from typing import Dict, List, Sequence

from . import _capi


def _spec(src, dst, sizes, n):
    return {"src_offsets": list(src[:n]), "dst_offsets": list(dst[:n]),
            "sizes": list(sizes[:n])}


def offsets_impl(block_ids: Sequence[int], source_is_compact: bool) -> Dict[str, List[int]]:
    """Runs of consecutive ids paired with compact positions 0..n-1."""
    ids, n = _capi.i64_array(block_ids)
    m = max(n, 1)
    src, dst, sz = (ctypes.c_int64 * m)(), (ctypes.c_int64 * m)(), (ctypes.c_int64 * m)()
    runs = ctypes.c_int64()
    _capi.check(_capi.load().kvx_offsets_impl(ids, n, int(bool(source_is_compact)), src, dst,
                                              sz, ctypes.byref(runs)), "OffsetsImpl")
    return _spec(src, dst, sz, runs.value)


def build_coalesced_copy_spec(src_block_ids: Sequence[int],
                              dst_block_ids: Sequence[int]) -> Dict[str, List[int]]:
    s, n = _capi.i64_array(src_block_ids)
    d, nd = _capi.i64_array(dst_block_ids)
    if nd != n:
        raise _capi.KvxError(3, "src and dst block lists must have same length",
                             "BuildCoalescedCopySpec")
    m = max(n, 1)
    src, dst, sz = (ctypes.c_int64 * m)(), (ctypes.c_int64 * m)(), (ctypes.c_int64 * m)()
    runs = ctypes.c_int64()
    _capi.check(_capi.load().kvx_build_coalesced_copy_spec(s, d, n, src, dst, sz,
                                                           ctypes.byref(runs)),
                "BuildCoalescedCopySpec")
    return _spec(src, dst, sz, runs.value)


class _PlanBuffers:
    def __init__(self, n):
        m = max(n, 1)
        self.arrays = [(ctypes.c_int64 * m)() for _ in range(7)]
        a = self.arrays
        self.out = _capi.LoadPlanOut(a[0], a[1], a[2], a[3], 0, a[4], a[5], a[6], 0)

    def result(self, n, remote, local):
        a, o = self.arrays, self.out
        return {"num_blocks": n, "requested_remote_block_ids": list(remote),
                "requested_local_block_ids": list(local),
                "producer_remote_block_ids": list(a[0][:n]),
                "transport_host_block_ids": list(a[1][:n]),
                "h2d_local_block_ids": list(a[2][:o.num_h2d]),
                "h2d_host_block_ids": list(a[3][:o.num_h2d]),
                "h2d_copy": _spec(a[4], a[5], a[6], o.num_runs)}


def build_load_copy_plan(remote_block_ids: Sequence[int], local_block_ids: Sequence[int],
                         local_host_block_ids: Sequence[int]) -> dict:
    r, n = _capi.i64_array(remote_block_ids)
    l, nl = _capi.i64_array(local_block_ids)
    h, nh = _capi.i64_array(local_host_block_ids)
    if not n == nl == nh:
        raise _capi.KvxError(3, "remote_block_ids, local_block_ids, and local_host_block_ids"
                                " must have same length", "BuildLoadCopyPlan")
    buf = _PlanBuffers(n)
    _capi.check(_capi.load().kvx_build_load_copy_plan(r, l, h, n, ctypes.byref(buf.out)),
                "BuildLoadCopyPlan")
    return buf.result(n, remote_block_ids, local_block_ids)
