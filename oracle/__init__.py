"""ORACLE -- test infrastructure only.

CPU restatement of the reference's host-side algorithms for the KV block
extract/insert path (see kvx_oracle.c for the file:line each C function
follows). Only tests/, ``__graft_entry__.smoke()`` and the CPU-baseline leg
of ``bench.py`` import this package, and only as the checker or the timed
CPU baseline. The product library never calls it.

Parity status of each function (what pins it):
  validate / coalesce / offsets_impl / build_coalesced_copy_spec:
      brute force (expanding runs reproduces the 1-block list) and the
      reference tests' known answers (tests/golden/reference_cases.json).
  build_load_copy_plan (pure Python, below):
      invariants fixed independently of the restated loop -- the
      transport order is the stable sort by remote id of the (remote, host)
      pairs, expanding the H2D runs gives exactly one (host -> local) copy
      per distinct local id with that id's host id, and conflicting
      duplicates are rejected (tests/test_copy_plan.py).
  transfer (D2h/H2d byte semantics), read_block / write_block,
  extract / insert:
      numpy fancy indexing (pool[:, ids]) as an independent library routine,
      round trips, untouched-block checks and the reference's e2e known
      answers (shift copy, partial chunks, auto-allocate).
  tiled_elements / tile / detile (XLA nested tiling, element by element):
      the reference tiling tests' known answers (tests/golden/tiling_cases.json:
      element counts and values at given physical positions, padding zeros),
      an independent numpy formulation of 2-D tiling (pad, reshape, swap
      axes) and of the (P, 1) row packing, round trips, and brute-force
      bijection / padding checks (tests/test_tiling_oracle.py).
  detile_std (the reference's threaded standard-form host detile, the timed
  CPU baseline of tiled weight sync): against detile on every reference case
  of the standard form and random standard layouts, 1-8 threads.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libkvx_oracle.so")
_lib = None

_i64p = ctypes.POINTER(ctypes.c_int64)
_u8pp = ctypes.POINTER(ctypes.c_void_p)


def build():
    """Compiles the C oracle with gcc (CPU only)."""
    import subprocess
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        l = ctypes.CDLL(_LIB_PATH)
        l.oracle_validate.argtypes = [_i64p, ctypes.c_int64, _i64p, ctypes.c_int64,
                                      _i64p, ctypes.c_int64]
        for fn in (l.oracle_coalesce, l.oracle_build_coalesced_copy_spec):
            fn.restype = ctypes.c_int64
        l.oracle_coalesce.argtypes = [_i64p, _i64p, _i64p, ctypes.c_int64,
                                      _i64p, _i64p, _i64p]
        l.oracle_build_coalesced_copy_spec.argtypes = [_i64p, _i64p, ctypes.c_int64,
                                                       _i64p, _i64p, _i64p]
        l.oracle_offsets_impl.restype = ctypes.c_int64
        l.oracle_offsets_impl.argtypes = [_i64p, ctypes.c_int64, ctypes.c_int,
                                          _i64p, _i64p, _i64p]
        l.oracle_transfer.argtypes = [ctypes.c_int, _u8pp, _i64p, _u8pp, _i64p,
                                      _i64p, _i64p, ctypes.c_int64,
                                      _i64p, ctypes.c_int64, _i64p, ctypes.c_int64,
                                      _i64p, ctypes.c_int64]
        l.oracle_read_block.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                        ctypes.c_int, ctypes.c_void_p]
        l.oracle_write_block.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                         ctypes.c_int, ctypes.c_void_p, ctypes.c_int64]
        _i32p = ctypes.POINTER(ctypes.c_int32)
        l.oracle_tiled_elements.restype = ctypes.c_int64
        l.oracle_tiled_elements.argtypes = [ctypes.c_int, _i64p, _i32p, ctypes.c_int,
                                            _i32p, _i64p]
        for fn in (l.oracle_tile, l.oracle_detile):
            fn.argtypes = [ctypes.c_int, ctypes.c_int, _i64p, _i32p, ctypes.c_int, _i32p,
                           _i64p, ctypes.c_void_p, ctypes.c_void_p]
        l.oracle_detile_std.argtypes = [ctypes.c_int, ctypes.c_int64, ctypes.c_int64,
                                         ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                                         ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                         ctypes.c_int]
        for fn in (l.oracle_extract, l.oracle_insert):
            fn.argtypes = [_u8pp, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                           _i64p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int,
                           ctypes.c_int]
        _lib = l
    return _lib


def _arr(a):
    a = np.ascontiguousarray(np.asarray(a, dtype=np.int64))
    return a, a.ctypes.data_as(_i64p)


def validate(src, dst, sizes):
    s, sp = _arr(src)
    d, dp = _arr(dst)
    z, zp = _arr(sizes)
    return lib().oracle_validate(sp, len(s), dp, len(d), zp, len(z))


def _runs(fn, ids):
    n = len(ids)
    outs = [np.zeros(max(n, 1), np.int64) for _ in range(3)]
    ptrs = [o.ctypes.data_as(_i64p) for o in outs]
    m = fn(*ptrs)
    return [o[:m].tolist() for o in outs]


def coalesce(src, dst, sizes):
    s, sp = _arr(src)
    d, dp = _arr(dst)
    z, zp = _arr(sizes)
    return _runs(lambda *p: lib().oracle_coalesce(sp, dp, zp, len(s), *p), s)


def offsets_impl(ids, source_is_compact):
    a, ap = _arr(ids)
    return _runs(lambda *p: lib().oracle_offsets_impl(ap, len(a), int(source_is_compact), *p), a)


def build_coalesced_copy_spec(src_ids, dst_ids):
    s, sp = _arr(src_ids)
    d, dp = _arr(dst_ids)
    if len(s) != len(d):
        raise ValueError("src and dst block lists must have same length")
    return _runs(lambda *p: lib().oracle_build_coalesced_copy_spec(sp, dp, len(s), *p), s)


def build_load_copy_plan(remote, local, host):
    """BuildLoadCopyPlan (tpu_sync/core/kv_cache_manager_with_transfer.cc:
    357-426): transport order = stable sort by remote id; H2D order = stable
    sort by local id, a repeated local id dropped (it must carry the same
    host id); h2d_copy = BuildCoalescedCopySpec(h2d hosts, h2d locals)."""
    if not len(remote) == len(local) == len(host):
        raise ValueError("remote_block_ids, local_block_ids, and local_host_block_ids "
                         "must have same length")
    order_r = sorted(range(len(remote)), key=lambda i: remote[i])
    order_l = sorted(range(len(local)), key=lambda i: local[i])
    h2d_local, h2d_host = [], []
    for i in order_l:
        if h2d_local and h2d_local[-1] == local[i]:
            if h2d_host[-1] != host[i]:
                raise ValueError("Duplicate local block IDs must map to the same host block ID")
            continue
        h2d_local.append(local[i])
        h2d_host.append(host[i])
    s, d, z = build_coalesced_copy_spec(h2d_host, h2d_local) if h2d_local else ([], [], [])
    return {"producer_remote_block_ids": [remote[i] for i in order_r],
            "transport_host_block_ids": [host[i] for i in order_r],
            "h2d_local_block_ids": h2d_local, "h2d_host_block_ids": h2d_host,
            "h2d_copy": {"src_offsets": s, "dst_offsets": d, "sizes": z}}


def _ptrs(bufs):
    arr = (ctypes.c_void_p * len(bufs))(*[b.ctypes.data if b is not None else None
                                          for b in bufs])
    return ctypes.cast(arr, _u8pp), arr


def transfer(d2h, dev, host, block_bytes, phys_bytes, src, dst, sizes):
    """D2h (d2h=True) / H2d between lists of uint8 numpy buffers; returns code."""
    dp, keep1 = _ptrs(dev)
    hp, keep2 = _ptrs(host)
    db, dbp = _arr([d.nbytes for d in dev])
    hb, hbp = _arr([h.nbytes if h is not None else 0 for h in host])
    bb, bbp = _arr(block_bytes)
    pb, pbp = _arr(phys_bytes)
    s, sp = _arr(src)
    d, dpp = _arr(dst)
    z, zp = _arr(sizes)
    return lib().oracle_transfer(int(bool(d2h)), dp, dbp, hp, hbp, bbp, pbp, len(dev),
                                 sp, len(s), dpp, len(d), zp, len(z))


def read_block(host, block_bytes, block_id):
    out = np.zeros(block_bytes, np.uint8)
    rc = lib().oracle_read_block(host.ctypes.data, host.nbytes, block_bytes, block_id,
                                 out.ctypes.data)
    return rc, out


def write_block(host, block_bytes, block_id, payload):
    payload = np.ascontiguousarray(payload, dtype=np.uint8)
    return lib().oracle_write_block(host.ctypes.data, host.nbytes, block_bytes, block_id,
                                    payload.ctypes.data, payload.nbytes)


def extract(pools, block_bytes, ids, order=0, nthreads=1, staging=None):
    """Packs blocks `ids` of every pool into staging; returns (code, staging)."""
    pp, keep = _ptrs(pools)
    a, ap = _arr(ids)
    if staging is None:
        staging = np.zeros(len(pools) * len(a) * block_bytes, np.uint8)
    rc = lib().oracle_extract(pp, len(pools), pools[0].nbytes, block_bytes, ap, len(a),
                              staging.ctypes.data, order, nthreads)
    return rc, staging


def insert(pools, block_bytes, ids, staging, order=0, nthreads=1):
    pp, keep = _ptrs(pools)
    a, ap = _arr(ids)
    staging = np.ascontiguousarray(staging, dtype=np.uint8)
    return lib().oracle_insert(pp, len(pools), pools[0].nbytes, block_bytes, ap, len(a),
                               staging.ctypes.data, order, nthreads)


def _layout_arrays(layout):
    """(itemsize, dims, minor_to_major, tiles) of a dict or an object."""
    get = (lambda k: layout[k]) if isinstance(layout, dict) else (lambda k: getattr(layout, k))
    itemsize = int(get("itemsize"))
    dims = np.ascontiguousarray(np.asarray(get("dims"), dtype=np.int64).reshape(-1))
    mtm = np.ascontiguousarray(np.asarray(get("minor_to_major"), dtype=np.int32).reshape(-1))
    tiles = [list(t) for t in get("tiles")]
    trank = np.asarray([len(t) for t in tiles] or [0], dtype=np.int32)
    tdims = np.zeros((max(len(tiles), 1), 8), dtype=np.int64)
    for i, t in enumerate(tiles):
        tdims[i, : len(t)] = t
    if dims.size == 0:
        dims = np.zeros(1, np.int64)
        mtm = np.zeros(1, np.int32)
        rank = 0
    else:
        rank = int(dims.size)
    i32 = ctypes.POINTER(ctypes.c_int32)
    keep = (dims, mtm, trank, tdims)
    args = (rank, dims.ctypes.data_as(_i64p), mtm.ctypes.data_as(i32), len(tiles),
            trank.ctypes.data_as(i32), tdims.ctypes.data_as(_i64p))
    return itemsize, args, keep


def tiled_elements(layout):
    """GetTiledBufferElements of a layout (dict or object with itemsize, dims,
    minor_to_major, tiles)."""
    _, args, keep = _layout_arrays(layout)
    return int(lib().oracle_tiled_elements(*args))


def logical_elements(layout):
    _, args, keep = _layout_arrays(layout)
    return int(np.prod(keep[0])) if args[0] > 0 else 1


def tile(layout, linear):
    """TileBuffer: linear bytes -> tiled bytes (padding zero)."""
    itemsize, args, keep = _layout_arrays(layout)
    linear = np.ascontiguousarray(np.asarray(linear).view(np.uint8).reshape(-1))
    n = tiled_elements(layout) if len(layout["tiles"] if isinstance(layout, dict)
                                      else layout.tiles) else logical_elements(layout)
    out = np.full(n * itemsize, 0xA5, np.uint8)
    rc = lib().oracle_tile(itemsize, *args, linear.ctypes.data, out.ctypes.data)
    if rc != 0:
        raise ValueError("oracle_tile failed: %d" % rc)
    return out


def detile(layout, tiled):
    """DetileBuffer: tiled bytes -> linear bytes."""
    itemsize, args, keep = _layout_arrays(layout)
    tiled = np.ascontiguousarray(np.asarray(tiled).view(np.uint8).reshape(-1))
    out = np.zeros(logical_elements(layout) * itemsize, np.uint8)
    rc = lib().oracle_detile(itemsize, *args, tiled.ctypes.data, out.ctypes.data)
    if rc != 0:
        raise ValueError("oracle_detile failed: %d" % rc)
    return out


def detile_std(itemsize, B, H, W, tH, tW, P, tiled, linear=None, nthreads=1):
    """Standard-form detile with threads (bytes in, bytes out)."""
    tiled = np.ascontiguousarray(np.asarray(tiled).view(np.uint8).reshape(-1))
    if linear is None:
        linear = np.zeros(B * H * W * itemsize, np.uint8)
    rc = lib().oracle_detile_std(itemsize, B, H, W, tH, tW, P, tiled.ctypes.data,
                                 linear.ctypes.data, nthreads)
    if rc != 0:
        raise ValueError("oracle_detile_std failed: %d" % rc)
    return linear
