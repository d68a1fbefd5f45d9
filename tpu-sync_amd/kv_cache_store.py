"""Tier-2 host KV store over libkvx (local flows, one GPU).

Mirrors the reference's Python surface (tpu_sync/api/torch/kv_cache_store.py:
38-594 over tpu_sync/frameworks/torch/tpu_raiden_torch_module.cc:600-800):
``lookup`` pins what it returns, ``insert`` pins what it takes, ``save`` /
``load`` consume those pins on success and are polled with
``poll_save_status`` / ``poll_load_status``. The store's controller lives in
this process; a KVCacheManager created with
``raiden_controller_address=store.raiden_controller_address`` becomes its
transfer worker. Peers, the global registry and remote saves/loads/reads are
out of scope: a REMOTE slice is refused and a registry address raises.

With RAIDEN_SHM_KEY set the store keeps a crash-persistent metadata table in
shared memory under "<key>_metadata[_<RAIDEN_SHM_SERVER_NAME>]" and rebuilds
its index from a surviving table at construction
(tpu_sync/kv_cache/kv_cache_store_wrapper.cc:46-57, 112-185).
"""
import ctypes
import enum
from typing import List, Optional, Sequence, Tuple

import numpy as np

from . import _capi
from .kv_cache_manager import LogicalBlockManager


class BlockStatus(enum.IntEnum):
    """tpu_sync/kv_cache/kv_cache_store_backend.h:39-45."""
    INIT = 0
    REMOTE = 1
    HBM = 2
    HOST = 3
    HOST_AND_HBM = 4


class RaidenId:
    """Identity of a store (tpu_sync/api/torch/kv_cache_store.py:38-86)."""

    def __init__(self, job_name: str = "", job_replica_id: str = "",
                 data_name: str = "", data_replica_idx: int = 0):
        self._job_name = job_name
        self._job_replica_id = job_replica_id
        self._data_name = data_name
        self._data_replica_idx = int(data_replica_idx)

    @property
    def job_name(self) -> str:
        return self._job_name

    @property
    def job_replica_id(self) -> str:
        return self._job_replica_id

    @property
    def data_name(self) -> str:
        return self._data_name

    @property
    def data_replica_idx(self) -> int:
        return self._data_replica_idx

    def _key(self):
        return (self._job_name, self._job_replica_id, self._data_name,
                self._data_replica_idx)

    def __eq__(self, other) -> bool:
        return isinstance(other, RaidenId) and self._key() == other._key()

    def __hash__(self):
        return hash(self._key())

    def __repr__(self) -> str:
        return ("RaidenId(job_name=%r, job_replica_id=%r, data_name=%r, "
                "data_replica_idx=%d)" % self._key())


class RaidenBlockId:
    """Where a block lives (tpu_sync/api/torch/kv_cache_store.py:89-151)."""

    __slots__ = ("_raiden_id", "_host_block_id", "_device_block_id", "_status")

    def __init__(self, raiden_id: Optional[RaidenId] = None, host_block_id: int = -1,
                 device_block_id: int = -1, status: BlockStatus = BlockStatus.INIT):
        self._raiden_id = raiden_id if raiden_id is not None else RaidenId()
        self._host_block_id = int(host_block_id)
        self._device_block_id = int(device_block_id)
        self._status = BlockStatus(status)

    raiden_id = property(lambda self: self._raiden_id)
    host_block_id = property(lambda self: self._host_block_id)
    device_block_id = property(lambda self: self._device_block_id)
    status = property(lambda self: self._status)
    job_name = property(lambda self: self._raiden_id.job_name)
    job_replica_id = property(lambda self: self._raiden_id.job_replica_id)
    data_name = property(lambda self: self._raiden_id.data_name)
    data_replica_idx = property(lambda self: self._raiden_id.data_replica_idx)

    @classmethod
    def _of(cls, raiden_id: "RaidenId", host_block_id: int, device_block_id: int,
            status: BlockStatus) -> "RaidenBlockId":
        """Construction from already-typed fields (the library's lists)."""
        b = cls.__new__(cls)
        b._raiden_id = raiden_id
        b._host_block_id = host_block_id
        b._device_block_id = device_block_id
        b._status = status
        return b

    def __eq__(self, other) -> bool:
        return (isinstance(other, RaidenBlockId) and self._raiden_id == other._raiden_id
                and self._host_block_id == other._host_block_id
                and self._device_block_id == other._device_block_id
                and self._status == other._status)

    def __repr__(self) -> str:
        return (f"RaidenBlockId({self._raiden_id!r}, host_block_id={self._host_block_id}, "
                f"device_block_id={self._device_block_id}, status={self._status.name})")


# kvx_block_slice as numpy lays it out: four int32 fields, then the three
# name pointers.
_SLICE_DTYPE = np.dtype([("host", "<i4"), ("dev", "<i4"), ("status", "<i4"),
                         ("replica", "<i4"), ("names", "<u8", (3,))])
assert _SLICE_DTYPE.itemsize == ctypes.sizeof(_capi.BlockSlice)
_STATUS_BY_VALUE = {int(s): s for s in BlockStatus}
_STATUS_INT = {s: int(s) for s in BlockStatus}


def _c_slices(slices: Sequence):
    """kvx_block_slice array of `slices` (RaidenBlockId, or RaidenId for a
    bare owner): (pointer, count, objects that must outlive the call). Each
    distinct owner's names are encoded once."""
    keep = []
    owners = {}  # id(RaidenId) -> its row in `rows`
    rows = []  # the three name addresses of each distinct owner
    hosts, devs, stats, reps, which = [], [], [], [], []
    last_rid, last_row = None, 0
    status_int = _STATUS_INT
    for s in slices:
        if type(s) is not RaidenBlockId and isinstance(s, RaidenId):
            s = RaidenBlockId(raiden_id=s)
        rid = s._raiden_id
        if rid is not last_rid:
            row = owners.get(id(rid))
            if row is None:
                encoded = [rid.job_name.encode(), rid.job_replica_id.encode(),
                           rid.data_name.encode()]
                keep.extend(encoded)
                keep.append(rid)  # keeps id(rid) unique while the table is used
                row = len(rows)
                rows.append([ctypes.cast(ctypes.c_char_p(b), ctypes.c_void_p).value
                             for b in encoded])
                owners[id(rid)] = row
            last_rid, last_row = rid, row
        hosts.append(s._host_block_id)
        devs.append(s._device_block_id)
        stats.append(status_int[s._status])
        reps.append(rid._data_replica_idx)
        which.append(last_row)
    n = len(hosts)
    raw = np.zeros(max(n, 1), dtype=_SLICE_DTYPE)
    if n:
        raw["host"][:n] = hosts
        raw["dev"][:n] = devs
        raw["status"][:n] = stats
        raw["replica"][:n] = reps
        table = np.array([[a or 0 for a in r] for r in rows], dtype=np.uint64)
        raw["names"][:n] = table[0] if len(rows) == 1 else table[which]
    keep.append(raw)
    return raw.ctypes.data_as(ctypes.POINTER(_capi.BlockSlice)), n, keep


def _c_string(ptr: int) -> str:
    return ctypes.string_at(ptr).decode() if ptr else ""


def _take_slices(handle) -> List[Tuple[bytes, RaidenBlockId]]:
    """The (hash, RaidenBlockId) pairs of a kvx_slices list, fetched with one
    library call for the whole list; releases the list."""
    lib = _capi.load()
    try:
        n = lib.kvx_slices_count(handle)
        if n == 0:
            return []
        hashes, offsets = ctypes.c_void_p(), _capi._i64p()
        blocks = ctypes.POINTER(_capi.BlockSlice)()
        _capi.check(lib.kvx_slices_flat(handle, ctypes.byref(hashes), ctypes.byref(offsets),
                                        ctypes.byref(blocks)))
        keys = _capi.split_flat(hashes, offsets, n)
        raw = np.frombuffer(ctypes.string_at(blocks, n * _SLICE_DTYPE.itemsize),
                            dtype=_SLICE_DTYPE)
        hosts, devs = raw["host"].tolist(), raw["dev"].tolist()
        stats, reps = raw["status"].tolist(), raw["replica"].tolist()
        by_value = _STATUS_BY_VALUE
        names = raw["names"]
        if (names == names[0]).all() and (raw["replica"] == reps[0]).all():
            # One owner (the library shares equal owners' name pointers).
            p = names[0].tolist()
            rid = RaidenId(_c_string(p[0]), _c_string(p[1]), _c_string(p[2]), reps[0])
            owners = [rid] * n
        else:
            ids = {}  # one RaidenId per distinct owner
            owners = []
            for row, rep in zip(names.tolist(), reps):
                owner = (*row, rep)
                rid = ids.get(owner)
                if rid is None:
                    rid = RaidenId(_c_string(owner[0]), _c_string(owner[1]),
                                   _c_string(owner[2]), owner[3])
                    ids[owner] = rid
                owners.append(rid)
        # RaidenBlockId._of inlined: the objects of a long list are built
        # without a call each.
        new, cls = object.__new__, RaidenBlockId
        out = []
        for k, rid, h, d, v in zip(keys, owners, hosts, devs, stats):
            b = new(cls)
            b._raiden_id = rid
            b._host_block_id = h
            b._device_block_id = d
            b._status = by_value[v]
            out.append((k, b))
        return out
    finally:
        lib.kvx_slices_release(handle)


class KVCacheStore:
    """Host-tier KV store with the reference's pin contract.

    Args:
      capacity: host blocks the store may hold (LRU capacity and the size of
        its controller's host block allocator; the worker's host mirror must
        hold at least this many blocks).
      global_registry_address: must be empty (no registry on one node).
      raiden_id: identity recorded in the entries' RaidenBlockIds.
      num_shards, store_server_ip: required keywords, validated as the
        reference validates them (num_shards >= 1, ip non-empty and not a
        wildcard).
      raiden_controller_port: 0 picks an unused in-process address.
      metadata_shm_key / model_uid: crash-persistent table; None takes the
        library's defaults from RAIDEN_SHM_KEY (+ "_metadata", + "_" +
        RAIDEN_SHM_SERVER_NAME) and RAIDEN_SHM_MODEL_UID; "" disables it.
      recover_at_create: rebuild the index from a surviving table now.
      host_blocks: host blocks of the controller's allocator (default:
        capacity, as the reference sizes it).
    """

    def __init__(self, capacity: int, global_registry_address: str = "",
                 raiden_id: Optional[RaidenId] = None, *, num_shards: int,
                 store_server_ip: str, shard_size_bytes: int = 0,
                 raiden_controller_port: int = 0, expected_worker_count: int = 0,
                 kv_pool_group: str = "", metadata_shm_key: Optional[str] = None,
                 model_uid: Optional[str] = None, recover_at_create: bool = True,
                 host_blocks: int = 0):
        if global_registry_address:
            raise ValueError("a global registry is not available: this store serves "
                             "one node only")
        del expected_worker_count, kv_pool_group
        rid = raiden_id if raiden_id is not None else RaidenId()
        cfg = _capi.StoreConfig()
        cfg.capacity = int(capacity)
        # None passes NULL: the library applies the RAIDEN_SHM_* defaults.
        self._strs = [rid.job_name.encode(), rid.job_replica_id.encode(),
                      rid.data_name.encode(), store_server_ip.encode(),
                      None if metadata_shm_key is None else metadata_shm_key.encode(),
                      None if model_uid is None else model_uid.encode()]
        (cfg.job_name, cfg.job_replica_id, cfg.data_name, cfg.store_server_ip,
         cfg.metadata_shm_key, cfg.model_uid) = self._strs
        cfg.data_replica_idx = rid.data_replica_idx
        cfg.num_shards = int(num_shards)
        cfg.shard_size_bytes = int(shard_size_bytes)
        cfg.raiden_controller_port = int(raiden_controller_port)
        cfg.no_auto_recover = 0 if recover_at_create else 1
        cfg.host_blocks = int(host_blocks)
        self._transfer_cb = None
        h = ctypes.c_void_p()
        code = _capi.load().kvx_store_create(ctypes.byref(cfg), ctypes.byref(h))
        if code == 3 or code == 9:  # InvalidArgument / FailedPrecondition
            raise ValueError(_capi.last_error())
        _capi.check(code, "KVCacheStore create")
        self._h = h
        self._raiden_id = rid

    # -- identity ------------------------------------------------------------
    @property
    def raiden_id(self) -> RaidenId:
        return self._raiden_id

    @property
    def raiden_controller_address(self) -> str:
        return _capi.load().kvx_store_controller_address(self._h).decode()

    @property
    def store_server_address(self) -> str:
        return ""

    def capacity(self) -> int:
        return _capi.load().kvx_store_capacity(self._h)

    def size(self) -> int:
        return _capi.load().kvx_store_size(self._h)

    @property
    def recovered_blocks(self) -> int:
        return _capi.load().kvx_store_recovered_blocks(self._h)

    @property
    def metadata_warm(self) -> bool:
        return bool(_capi.load().kvx_store_metadata_warm(self._h))

    def host_block_manager(self) -> LogicalBlockManager:
        h = _capi.load().kvx_store_host_block_manager(self._h)
        return LogicalBlockManager(_handle=ctypes.c_void_p(h), _owner=self)

    # -- the three workflows --------------------------------------------------
    def lookup(self, block_hashes: List[bytes], enable_global: bool = False,
               pin_found: bool = True) -> List[Tuple[bytes, RaidenBlockId]]:
        """Cached (hash, RaidenBlockId) pairs up to the first miss; pins them
        unless pin_found is False."""
        del enable_global
        buf, offs, n = _capi.pack_bytes(block_hashes)
        out = ctypes.c_void_p()
        code = _capi.load().kvx_store_lookup(self._h, buf, offs, n, int(pin_found),
                                             ctypes.byref(out))
        if code != 0:
            raise RuntimeError("KVCacheStore lookup failed: " + _capi.last_error())
        return _take_slices(out)

    def insert(self, block_hashes: List[bytes], slices: List[RaidenBlockId],
               on_host: bool) -> bool:
        """Pins existing hashes and inserts+pins new ones, all or nothing.
        Raises ValueError for a REMOTE slice."""
        buf, offs, n = _capi.pack_bytes(block_hashes)
        arr, ns, _keep = _c_slices(slices)
        code = _capi.load().kvx_store_insert(self._h, buf, offs, n, arr, ns, int(on_host))
        if code == 3:
            raise ValueError(_capi.last_error())
        return code == 0

    def release(self, block_hashes: List[bytes]) -> None:
        buf, offs, n = _capi.pack_bytes(block_hashes)
        _capi.check(_capi.load().kvx_store_release(self._h, buf, offs, n))

    def save(self, block_hashes: List[bytes], dst_raiden_id: Optional[RaidenId] = None
             ) -> bool:
        """Local save HBM -> host, asynchronous; False if validation failed."""
        if dst_raiden_id is not None:
            return False  # no peers on one node
        buf, offs, n = _capi.pack_bytes(block_hashes)
        self._last_code = _capi.load().kvx_store_save(self._h, buf, offs, n)
        return self._last_code == 0

    def load(self, block_hashes: List[bytes], device_block_ids: List[int],
             slices: Optional[List[RaidenBlockId]] = None) -> bool:
        """Local load host -> device blocks, asynchronous; False if validation
        failed."""
        buf, offs, n = _capi.pack_bytes(block_hashes)
        dev, nd = _capi.i32_array(device_block_ids)
        lib = _capi.load()
        if slices is None:
            self._last_code = lib.kvx_store_load(self._h, buf, offs, n, dev, nd)
        else:
            arr, ns, _keep = _c_slices(slices)
            self._last_code = lib.kvx_store_load_slices(self._h, buf, offs, n, arr, ns,
                                                        dev, nd)
        return self._last_code == 0

    def last_error(self) -> str:
        """Message of the last failed call on this thread."""
        return _capi.last_error()

    def poll_save_status(self):
        """(done, failed, pending, existing, unregistered) hash lists."""
        out = (ctypes.c_void_p * 5)()
        _capi.check(_capi.load().kvx_store_poll_save_status(self._h, out))
        return tuple(_capi.take_strings(out[i]) for i in range(5))

    def poll_load_status(self):
        """(done, failed, pending) hash lists."""
        out = (ctypes.c_void_p * 3)()
        _capi.check(_capi.load().kvx_store_poll_load_status(self._h, out))
        return tuple(_capi.take_strings(out[i]) for i in range(3))

    def read_remote(self, block_hashes, slices, device_block_ids) -> bool:
        del block_hashes, slices, device_block_ids
        return False  # no peers on one node

    def poll_remote_read_status(self):
        return [], [], []

    def get_pin_count(self, block_hash: bytes) -> int:
        b = bytes(block_hash)
        return _capi.load().kvx_store_pin_count(self._h, b, len(b))

    def recover_from_local_manifest(self) -> int:
        n = ctypes.c_int64()
        _capi.check(_capi.load().kvx_store_recover_from_local_manifest(
            self._h, ctypes.byref(n)), "RecoverFromLocalManifest")
        return n.value

    def evictable_keys(self, count: int) -> List[bytes]:
        out = ctypes.c_void_p()
        _capi.check(_capi.load().kvx_store_evictable_keys(self._h, count, ctypes.byref(out)))
        return _capi.take_strings(out)

    def candidate_keys(self) -> List[bytes]:
        """Eviction candidates of the index, oldest first."""
        out = ctypes.c_void_p()
        _capi.check(_capi.load().kvx_store_candidate_keys(self._h, ctypes.byref(out)))
        return _capi.take_strings(out)

    def evict(self, block_hashes: List[bytes]) -> int:
        """Drops unpinned host-resident entries and frees their host blocks."""
        buf, offs, n = _capi.pack_bytes(block_hashes)
        out = ctypes.c_int64()
        _capi.check(_capi.load().kvx_store_evict(self._h, buf, offs, n, ctypes.byref(out)))
        return out.value

    def set_transfer_fn(self, fn) -> None:
        """Routes saves and loads through fn(d2h: bool, src: list, dst: list)
        -> status code (0 = OK) instead of the registered worker; None
        restores the worker."""
        if fn is None:
            self._transfer_cb = None
            _capi.check(_capi.load().kvx_store_set_transfer_fn(
                self._h, ctypes.cast(None, _capi.TRANSFER_FN), None))
            return

        def tramp(_user, d2h, src, dst, n):
            try:
                return int(fn(bool(d2h), [src[i] for i in range(n)],
                              [dst[i] for i in range(n)]))
            except Exception:  # a raising transfer is a failed transfer
                return 13

        self._transfer_cb = _capi.TRANSFER_FN(tramp)
        _capi.check(_capi.load().kvx_store_set_transfer_fn(self._h, self._transfer_cb, None))

    def close(self) -> None:
        h, self._h = getattr(self, "_h", None), None
        lib = _capi._lib if _capi is not None else None  # None at interpreter exit
        if h and lib is not None:
            lib.kvx_store_destroy(h)

    def __del__(self):
        self.close()


class LRUCache:
    """The host tier's pin-aware LRU index (tpu_sync/kv_cache/lru_cache.h)
    with bytes keys and int values."""

    GET, PEEK, PEEK_ANY, GET_AND_PIN = 0, 1, 2, 3

    def __init__(self, capacity: int):
        h = ctypes.c_void_p()
        _capi.check(_capi.load().kvx_lru_create(capacity, ctypes.byref(h)))
        self._h = h

    @staticmethod
    def _k(key) -> bytes:
        return key if isinstance(key, bytes) else str(key).encode()

    def put(self, key, value: int):
        """Returns the (key, value) demoted to the candidate list, or None."""
        k = self._k(key)
        ev, ek, evv = ctypes.c_int32(), ctypes.c_void_p(), ctypes.c_int64()
        _capi.check(_capi.load().kvx_lru_put(self._h, k, len(k), int(value), ctypes.byref(ev),
                                             ctypes.byref(ek), ctypes.byref(evv)))
        if not ev.value:
            return None
        return _capi.take_strings(ek)[0], evv.value

    def put_back(self, key, value: int) -> None:
        k = self._k(key)
        _capi.check(_capi.load().kvx_lru_put_back(self._h, k, len(k), int(value)))

    def _find(self, how, key):
        k = self._k(key)
        v = ctypes.c_int64()
        ok = _capi.load().kvx_lru_find(self._h, how, k, len(k), ctypes.byref(v))
        return v.value if ok else None

    def get(self, key):
        return self._find(self.GET, key)

    def peek(self, key):
        return self._find(self.PEEK, key)

    def peek_including_candidates(self, key):
        return self._find(self.PEEK_ANY, key)

    def get_and_pin(self, key):
        return self._find(self.GET_AND_PIN, key)

    def _bool(self, fn, key) -> bool:
        k = self._k(key)
        return bool(fn(self._h, k, len(k)))

    def contains(self, key) -> bool:
        return self._bool(_capi.load().kvx_lru_contains, key)

    def pin(self, key) -> bool:
        return self._bool(_capi.load().kvx_lru_pin, key)

    def unpin(self, key) -> bool:
        return self._bool(_capi.load().kvx_lru_unpin, key)

    def erase(self, key) -> bool:
        return self._bool(_capi.load().kvx_lru_erase, key)

    def pin_count(self, key) -> int:
        k = self._k(key)
        return _capi.load().kvx_lru_pin_count(self._h, k, len(k))

    def evict(self):
        ek, evv = ctypes.c_void_p(), ctypes.c_int64()
        if not _capi.load().kvx_lru_evict(self._h, ctypes.byref(ek), ctypes.byref(evv)):
            return None
        return _capi.take_strings(ek)[0], evv.value

    def evictable_keys(self, count: int) -> List[bytes]:
        out = ctypes.c_void_p()
        _capi.check(_capi.load().kvx_lru_evictable_keys(self._h, count, ctypes.byref(out)))
        return _capi.take_strings(out)

    def candidate_keys(self) -> List[bytes]:
        out = ctypes.c_void_p()
        _capi.check(_capi.load().kvx_lru_candidate_keys(self._h, ctypes.byref(out)))
        return _capi.take_strings(out)

    def clear(self) -> None:
        _capi.load().kvx_lru_clear(self._h)

    def sizes(self) -> dict:
        out = (ctypes.c_int64 * 4)()
        _capi.check(_capi.load().kvx_lru_sizes(self._h, out))
        return dict(zip(("capacity", "size", "active_size", "available_space"), list(out)))

    def __del__(self):
        h = getattr(self, "_h", None)
        lib = _capi._lib if _capi is not None else None  # None at interpreter exit
        if h and lib is not None:
            lib.kvx_lru_destroy(h)
            self._h = None


class KVCacheMetadata:
    """Crash-persistent metadata table over a caller-owned numpy region
    (tpu_sync/kv_cache/kv_cache_metadata.h:86-137)."""

    def __init__(self, region, num_blocks: int, model_uid: str = ""):
        self.region = region  # numpy uint8 array, 64-byte aligned
        self.num_blocks = int(num_blocks)
        self.model_uid = model_uid.encode()

    @staticmethod
    def required_size_bytes(num_blocks: int) -> int:
        return _capi.load().kvx_metadata_required_size(num_blocks)

    def _ptr(self):
        return ctypes.c_void_p(self.region.ctypes.data), self.region.nbytes

    def format(self) -> None:
        p, n = self._ptr()
        _capi.check(_capi.load().kvx_metadata_format(p, n, self.num_blocks, self.model_uid),
                    "KVCacheMetadata Format")

    def attach(self) -> None:
        p, n = self._ptr()
        _capi.check(_capi.load().kvx_metadata_attach(p, n, self.num_blocks, self.model_uid),
                    "KVCacheMetadata Attach")

    def set(self, block_id: int, block_hash: bytes, seq: int) -> None:
        p, n = self._ptr()
        h = bytes(block_hash)
        _capi.check(_capi.load().kvx_metadata_set(p, n, self.num_blocks, self.model_uid,
                                                  block_id, h, len(h), seq),
                    "KVCacheMetadata Set")

    def clear(self, block_id: int) -> None:
        p, n = self._ptr()
        _capi.check(_capi.load().kvx_metadata_clear(p, n, self.num_blocks, self.model_uid,
                                                    block_id), "KVCacheMetadata Clear")

    def valid_entries(self) -> List[Tuple[int, bytes, int]]:
        """[(block_id, hash, seq)] of the valid entries, by block id."""
        p, n = self._ptr()
        ids = (ctypes.c_int32 * max(self.num_blocks, 1))()
        seqs = (ctypes.c_uint64 * max(self.num_blocks, 1))()
        cnt, hs = ctypes.c_int64(), ctypes.c_void_p()
        _capi.check(_capi.load().kvx_metadata_valid_entries(
            p, n, self.num_blocks, self.model_uid, ids, seqs, ctypes.byref(cnt),
            ctypes.byref(hs)), "KVCacheMetadata ValidEntries")
        hashes = _capi.take_strings(hs)
        return [(ids[i], hashes[i], seqs[i]) for i in range(cnt.value)]


class KVCacheMetadataShmRegion:
    """Shared-memory segment holding a metadata table
    (tpu_sync/kv_cache/kv_cache_metadata_shm.h:33-86)."""

    def __init__(self, shm_key: str, num_blocks: int, model_uid: str = ""):
        h, warm = ctypes.c_void_p(), ctypes.c_int32()
        _capi.check(_capi.load().kvx_metadata_shm_attach_or_format(
            shm_key.encode(), num_blocks, model_uid.encode(), ctypes.byref(h),
            ctypes.byref(warm)), "KVCacheMetadataShmRegion AttachOrFormat")
        self._h = h
        self.warm = bool(warm.value)
        self.num_blocks = num_blocks
        self.model_uid = model_uid

    def region(self):
        """numpy uint8 view of the mapped segment."""
        import numpy as np
        p, n = ctypes.c_uint64(), ctypes.c_int64()
        _capi.check(_capi.load().kvx_metadata_shm_region(self._h, ctypes.byref(p),
                                                         ctypes.byref(n)))
        return np.ctypeslib.as_array((ctypes.c_uint8 * n.value).from_address(p.value))

    def metadata(self) -> KVCacheMetadata:
        return KVCacheMetadata(self.region(), self.num_blocks, self.model_uid)

    def reformat(self) -> None:
        _capi.check(_capi.load().kvx_metadata_shm_reformat(self._h))
        self.warm = False

    def close(self) -> None:
        h, self._h = getattr(self, "_h", None), None
        lib = _capi._lib if _capi is not None else None  # None at interpreter exit
        if h and lib is not None:
            lib.kvx_metadata_shm_release(h)

    def __del__(self):
        self.close()
