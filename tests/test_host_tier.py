"""Host tier on the CPU: the LRU index, the crash-persistent metadata table,
the shared-memory host pool and the KV store's local flows.

Each component runs the reference tests' known answers (restated as data in
tests/golden/ or as the cases below, each naming its source test) against
both the oracle restatement and the product through the C-ABI, and the two
are compared on random operation sequences. Store transfers go through a
recording transfer function here, as the reference's store tests use a mock
transfer manager; tests/test_gpu_store.py drives the same flows through the
real KV manager on the GPU.
"""
import json
import os
import random
import subprocess
import sys
import uuid

import numpy as np
import pytest

from oracle import host_tier as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def golden_lru():
    with open(os.path.join(ROOT, "tests", "golden", "lru_cases.json")) as f:
        return json.load(f)["cases"]


# ---------------------------------------------------------------------------
# LRU
# ---------------------------------------------------------------------------
class OracleLru:
    def __init__(self, cap):
        self.c = O.LRUCache(cap)

    def op(self, name, *a):
        c = self.c
        if name == "put":
            r = c.put(a[0], a[1])
            return None if r is None else [r[0], r[1]]
        if name == "put_back":
            return c.put_back(a[0], a[1])
        if name == "evict":
            r = c.evict()
            return None if r is None else [r[0], r[1]]
        fn = {"get": c.get, "peek": c.peek, "peek_any": c.peek_including_candidates,
              "get_and_pin": c.get_and_pin, "pin": c.pin, "unpin": c.unpin,
              "erase": c.erase, "contains": c.contains, "pin_count": c.pin_count,
              "evictable": c.evictable_keys}
        if name in fn:
            return fn[name](*a)
        if name == "candidates":
            return c.candidate_keys()
        if name == "clear":
            return c.clear()
        if name == "sizes":
            return {"capacity": c.capacity, "size": c.size(),
                    "active_size": c.active_size(), "available_space": c.available_space()}
        raise KeyError(name)


class ProductLru:
    def __init__(self, kvx, cap):
        self.c = kvx.LRUCache(cap)

    def op(self, name, *a):
        c = self.c
        dec = lambda ks: [k.decode() for k in ks]
        if name == "put":
            r = c.put(a[0], a[1])
            return None if r is None else [r[0].decode(), r[1]]
        if name == "put_back":
            return c.put_back(a[0], a[1])
        if name == "evict":
            r = c.evict()
            return None if r is None else [r[0].decode(), r[1]]
        if name == "evictable":
            return dec(c.evictable_keys(a[0]))
        if name == "candidates":
            return dec(c.candidate_keys())
        fn = {"get": c.get, "peek": c.peek, "peek_any": c.peek_including_candidates,
              "get_and_pin": c.get_and_pin, "pin": c.pin, "unpin": c.unpin,
              "erase": c.erase, "contains": c.contains, "pin_count": c.pin_count}
        if name in fn:
            return fn[name](*a)
        if name == "clear":
            return c.clear()
        if name == "sizes":
            return c.sizes()
        raise KeyError(name)


def run_lru_case(impl, case):
    for op in case["ops"]:
        name = op[0]
        if name in ("put",):
            got = impl.op(name, op[1], op[2])
            assert got == op[3], (case["source"], op, got)
        elif name == "put_back":
            impl.op(name, op[1], op[2])
        elif name in ("evict", "candidates"):
            got = impl.op(name)
            assert got == op[1], (case["source"], op, got)
        elif name == "clear":
            impl.op(name)
        elif name == "sizes":
            got = impl.op(name)
            for k, v in op[1].items():
                assert got[k] == v, (case["source"], op, got)
        else:
            got = impl.op(name, op[1])
            assert got == op[2], (case["source"], op, got)


def test_lru_reference_cases_oracle():
    for case in golden_lru():
        run_lru_case(OracleLru(case["capacity"]), case)


def test_lru_reference_cases_product(kvx):
    for case in golden_lru():
        run_lru_case(ProductLru(kvx, case["capacity"]), case)


def test_lru_differential_random(kvx):
    rng = random.Random(5)
    for trial in range(30):
        cap = rng.randint(1, 6)
        a, b = OracleLru(cap), ProductLru(kvx, cap)
        keys = [str(i) for i in range(rng.randint(2, 12))]
        for step in range(400):
            name = rng.choice(["put", "put", "put_back", "get", "peek", "peek_any",
                               "get_and_pin", "pin", "unpin", "unpin", "erase",
                               "contains", "pin_count", "evict", "evictable",
                               "candidates", "sizes"])
            if name in ("put", "put_back"):
                args = (rng.choice(keys), rng.randint(0, 99))
            elif name in ("evict", "candidates", "sizes"):
                args = ()
            elif name == "evictable":
                args = (rng.randint(0, 8),)
            else:
                args = (rng.choice(keys),)
            ga, gb = a.op(name, *args), b.op(name, *args)
            assert ga == gb, (trial, step, name, args, ga, gb)


# ---------------------------------------------------------------------------
# Metadata table
# ---------------------------------------------------------------------------
def aligned_region(num_blocks, extra=0):
    n = O.METADATA_HEADER + num_blocks * O.METADATA_ENTRY + extra
    raw = np.zeros(n + 64, np.uint8)
    off = (-raw.ctypes.data) % 64
    return raw[off:off + n]


def test_metadata_byte_layout_matches_struct_definition(kvx):
    """Format and Set write exactly the bytes the 128-byte header and entry
    definitions (kv_cache_metadata.h:34-70) spell out."""
    region = aligned_region(4)
    md = kvx.KVCacheMetadata(region, 4, "llama")
    md.format()
    assert bytes(region[:128]) == O.metadata_header(4, b"llama")
    assert bytes(region[:8]) == b"MKNEDIAR"  # "RAIDENKM" as a little-endian u64
    md.set(2, b"\x00hash\xff", 77)
    off = 128 + 2 * 128
    assert bytes(region[off:off + 128]) == O.metadata_entry(77, b"\x00hash\xff")
    assert not region[128:off].any() and not region[off + 128:].any()
    md.clear(2)
    assert region[off + 10] == 0
    assert O.metadata_valid_entries(region, 4) == []


def test_metadata_reference_cases(kvx):
    M = kvx.KVCacheMetadata
    # FormatCreatesEmptyTable (kv_cache_metadata_test.cc:49-55)
    r = aligned_region(4)
    m = M(r, 4)
    m.format()
    assert m.valid_entries() == []
    # FormatRejectsInvalidRegions (:57-70)
    with pytest.raises(kvx.KvxError) as e:
        M(r, 0).format()
    assert e.value.code == 3
    with pytest.raises(kvx.KvxError) as e:
        M(r[:128], 8).format()
    assert e.value.code == 3
    with pytest.raises(kvx.KvxError) as e:
        M(r[1:], 2).format()
    assert e.value.code == 3
    # SetAndClearRoundTrip (:72-84)
    m.set(1, b"hash_b", 2)
    m.set(3, b"hash_d", 1)
    assert m.valid_entries() == [(1, b"hash_b", 2), (3, b"hash_d", 1)]
    m.clear(1)
    assert m.valid_entries() == [(3, b"hash_d", 1)]
    # SetOverwritesPreviousBinding (:86-94)
    r2 = aligned_region(2)
    m2 = M(r2, 2)
    m2.format()
    m2.set(0, b"old_hash", 1)
    m2.set(0, b"new", 2)
    assert m2.valid_entries() == [(0, b"new", 2)]
    # SetValidatesArguments (:96-116)
    m2.format()
    for bid, h in ((-1, b"h"), (2, b"h"), (0, b""), (0, b"x" * 113)):
        with pytest.raises(kvx.KvxError) as e:
            m2.set(bid, h, 0)
        assert e.value.code == 3
    with pytest.raises(kvx.KvxError) as e:
        m2.clear(2)
    assert e.value.code == 3
    m2.set(0, b"y" * 112, 0)
    assert m2.valid_entries() == [(0, b"y" * 112, 0)]
    # HashesAreOpaqueBytes (:118-127)
    r1 = aligned_region(1)
    m1 = M(r1, 1)
    m1.format()
    m1.set(0, b"\x00\xff\x00raiden\x01", 7)
    assert m1.valid_entries() == [(0, b"\x00\xff\x00raiden\x01", 7)]
    # AttachRecoversEntriesFromSurvivingRegion (:129-143)
    r4 = aligned_region(4)
    M(r4, 4).format()
    M(r4, 4).set(0, b"hash_a", 3)
    M(r4, 4).set(2, b"hash_c", 4)
    M(r4, 4).attach()
    assert M(r4, 4).valid_entries() == [(0, b"hash_a", 3), (2, b"hash_c", 4)]
    # AttachRejectsUnformattedOrMismatchedRegions (:145-157)
    r8 = aligned_region(8)
    with pytest.raises(kvx.KvxError) as e:
        M(r8, 4).attach()
    assert e.value.code == 9
    M(r8, 4).format()
    with pytest.raises(kvx.KvxError) as e:
        M(r8, 8).attach()
    assert e.value.code == 9
    M(r8, 4).attach()
    # AttachValidatesModelUid (:159-173)
    ra = aligned_region(4)
    M(ra, 4, "model_a").format()
    M(ra, 4, "model_a").attach()
    for uid in ("model_b", ""):
        with pytest.raises(kvx.KvxError) as e:
            M(ra, 4, uid).attach()
        assert e.value.code == 9
    with pytest.raises(kvx.KvxError) as e:
        M(ra, 4, "x" * 64).format()
    assert e.value.code == 3
    # FormatWipesSurvivingEntries (:175-184)
    M(r2, 2).format()
    M(r2, 2).set(0, b"stale", 1)
    M(r2, 2).format()
    assert M(r2, 2).valid_entries() == []
    # UncommittedEntryIsInvisible (:186-199): a written but uncommitted slot.
    M(r2, 2).format()
    r2[128:128 + 16] = np.frombuffer(O.metadata_entry(9, b"torn", valid=0)[:16], np.uint8)
    r2[128 + 16:128 + 20] = np.frombuffer(b"torn", np.uint8)
    assert M(r2, 2).valid_entries() == []
    assert O.metadata_valid_entries(r2, 2) == []


@pytest.fixture
def shm_key():
    key = f"kvx_test_{os.getpid()}_{uuid.uuid4().hex[:8]}"
    yield key
    for suffix in ("", "_metadata"):
        try:
            os.unlink(f"/dev/shm/{key}{suffix}")
        except FileNotFoundError:
            pass


def test_metadata_shm_reference_cases(kvx, shm_key):
    R = kvx.KVCacheMetadataShmRegion
    # ColdStartFormatsEmptyTable (kv_cache_metadata_shm_test.cc:45-52)
    r = R(shm_key, 8, "model_a")
    assert not r.warm and r.metadata().valid_entries() == []
    # TableSurvivesProcessRestart (:54-72)
    r.metadata().set(1, b"hash_b", 2)
    r.metadata().set(3, b"hash_d", 1)
    r.close()
    r = R(shm_key, 8, "model_a")
    assert r.warm
    assert r.metadata().valid_entries() == [(1, b"hash_b", 2), (3, b"hash_d", 1)]
    # NumBlocksMismatchRecreates (:74-100)
    r.close()
    r = R(shm_key, 64, "model_a")
    assert not r.warm and r.metadata().valid_entries() == []
    r.metadata().set(1, b"hash_b", 2)
    r.close()
    r = R(shm_key, 8, "model_a")
    assert not r.warm and r.metadata().valid_entries() == []
    # ModelUidMismatchRecreates (:102-117)
    r.metadata().set(1, b"hash_b", 2)
    r.close()
    r = R(shm_key, 8, "model_b")
    assert not r.warm and r.metadata().valid_entries() == []
    # ReformatErasesEntries (:119-131)
    r.metadata().set(1, b"hash_b", 2)
    r.reformat()
    assert not r.warm and r.metadata().valid_entries() == []
    # The segment holds the format byte-for-byte.
    region = r.region()
    assert bytes(region[:128]) == O.metadata_header(8, b"model_b")
    r.close()


# ---------------------------------------------------------------------------
# Shared-memory host pool (host_memory_allocator_test.cc:83 cold/warm boot)
# ---------------------------------------------------------------------------
def test_shm_host_pool_cold_and_warm_boot(kvx, shm_key):
    def make(uid):
        return kvx.KVCacheManager.create_host_only_for_testing(
            num_layers=3, num_shards=2, slice_byte_size=96, host_blocks=5,
            host_alloc="shm", shm_key=shm_key, model_uid=uid)

    m = make("model_a")
    assert not m.shm_warm
    payloads = {}
    for layer in range(3):
        for shard in range(2):
            for blk in range(5):
                p = bytes((layer * 31 + shard * 7 + blk * 3 + i) % 256 for i in range(96))
                m.write_block_bytes(layer, blk, p, shard)
                payloads[layer, shard, blk] = p
    m.close()
    m = make("model_a")
    assert m.shm_warm
    for (layer, shard, blk), p in payloads.items():
        assert m.read_block_bytes(layer, blk, shard) == p
    m.close()
    m = make("model_b")  # schema mismatch: re-created, zero-filled
    assert not m.shm_warm
    assert m.read_block_bytes(1, 2, 1) == b"\0" * 96
    m.close()
    # The segment starts with the 384-byte schema record.
    seg = open(f"/dev/shm/{shm_key}", "rb").read(384)
    assert seg[:8] == (0x52414944454E5348).to_bytes(8, "little")
    assert seg[12:12 + 8] == b"model_b\0"


# ---------------------------------------------------------------------------
# Store: reference cases (kv_cache_store_test.cc), product and oracle
# ---------------------------------------------------------------------------
class Recorder:
    """The reference's MockTransferManager: records calls, can fail them."""

    def __init__(self):
        self.d2h_calls = self.h2d_calls = 0
        self.last_src = self.last_dst = None
        self.fail = False

    def __call__(self, d2h, src, dst):
        if d2h:
            self.d2h_calls += 1
        else:
            self.h2d_calls += 1
        self.last_src, self.last_dst = list(src), list(dst)
        return 13 if self.fail else 0


class ProductStore:
    """Adapts the product store to the oracle's (code, value) convention."""

    def __init__(self, kvx, capacity, md_key=None, md_blocks=None, recover=True,
                 host_blocks=0):
        self.kvx = kvx
        self.rec = Recorder()
        self.rid = kvx.RaidenId("test_job", "0", "test_cache", 0)
        self.s = kvx.KVCacheStore(capacity, raiden_id=self.rid, num_shards=1,
                                  store_server_ip="127.0.0.1",
                                  metadata_shm_key=md_key or "", model_uid="m",
                                  recover_at_create=recover, host_blocks=host_blocks)
        self.s.set_transfer_fn(self.rec)
        self.md_key, self.md_blocks = md_key, md_blocks

    def slices(self, specs):
        K = self.kvx
        return [K.RaidenBlockId(self.rid if st != O.REMOTE else K.RaidenId(*sp.get("rid", ("peer", "0", "kv", 0))),
                                sp["host"], sp["dev"], K.BlockStatus(st))
                for sp in specs for st in [sp["status"]]]

    def lookup(self, hashes, pin_found):
        out = self.s.lookup([h.encode() for h in hashes], pin_found=pin_found)
        return [(h.decode(), {"host": b.host_block_id, "dev": b.device_block_id,
                              "status": int(b.status)}) for h, b in out]

    def insert(self, hashes, specs):
        try:
            ok = self.s.insert([h.encode() for h in hashes], self.slices(specs), True)
        except ValueError:
            return O.INVALID_ARGUMENT
        return O.OK if ok else O.RESOURCE_EXHAUSTED

    def release(self, hashes):
        self.s.release([h.encode() for h in hashes])

    def evict(self, hashes):
        return self.s.evict([h.encode() for h in hashes])

    def _code(self, ok):
        return O.OK if ok else self.s._last_code

    def save(self, hashes):
        return self._code(self.s.save([h.encode() for h in hashes]))

    def load(self, hashes, dev):
        return self._code(self.s.load([h.encode() for h in hashes], dev))

    def load_slices(self, hashes, specs, dev):
        return self._code(self.s.load([h.encode() for h in hashes], dev, self.slices(specs)))

    def poll_save_status(self):
        return tuple([h.decode() for h in lst] for lst in self.s.poll_save_status())

    def poll_load_status(self):
        return tuple([h.decode() for h in lst] for lst in self.s.poll_load_status())

    def pin_count(self, h):
        return self.s.get_pin_count(h.encode())

    def candidates(self):
        return [k.decode() for k in self.s.candidate_keys()]

    def evictable(self):
        return [k.decode() for k in self.s.evictable_keys(10 ** 6)]

    def lbm_counts(self):
        b = self.s.host_block_manager()
        return {"free": b.num_free_blocks, "locked": b.num_locked_blocks,
                "allocated": b.num_allocated_blocks}

    def recover(self):
        try:
            return O.OK, self.s.recover_from_local_manifest()
        except self.kvx.KvxError as e:
            return e.code, None

    def metadata_entries(self):
        r = self.kvx.KVCacheMetadataShmRegion(self.md_key, self.md_blocks, "m")
        out = [(b, h, s) for b, h, s in r.metadata().valid_entries()]
        r.close()
        return [(b, h.decode(), s) for b, h, s in out]


class OracleStore(O.Store):
    def __init__(self, capacity, md_blocks=None):
        self.rec = Recorder()
        super().__init__(capacity, metadata_blocks=md_blocks, transfer=self.rec)

    def candidates(self):
        return self.lru.candidate_keys()

    def evictable(self):
        return self.lru.evictable_keys(10 ** 6)

    def lbm_counts(self):
        c = self.lbm.counts()
        return {"free": c["free"], "locked": c["locked"], "allocated": c["allocated"]}

    def pin_count(self, h):
        return self.lru.pin_count(h)

    def insert(self, hashes, specs):
        return super().insert(hashes, [dict(s) for s in specs])

    def load_slices(self, hashes, specs, dev):
        return super().load_slices(hashes, [dict(s) for s in specs], dev)

    def metadata_entries(self):
        return [(b, h, s) for b, h, s in super().metadata_entries()]


def S(host=-1, dev=-1, status=O.HBM, rid=None):
    d = {"host": host, "dev": dev, "status": status}
    if rid is not None:
        d["rid"] = rid
    return d


def insert_resident(st, hashes, specs):
    assert st.insert(hashes, specs) == O.OK
    st.release(hashes)


def store_impls(kvx):
    return [("oracle", lambda cap, **kw: OracleStore(cap, kw.get("md_blocks"))),
            ("product", lambda cap, **kw: ProductStore(kvx, cap, **kw))]


def test_store_reference_cases(kvx, shm_key):
    for name, make in store_impls(kvx):
        # EvictionTracking (kv_cache_store_test.cc:196-245)
        st = make(2)
        assert st.insert(["101", "102"], [S(status=O.INIT), S(status=O.INIT)]) == O.OK
        assert st.insert(["103"], [S(status=O.INIT)]) == O.RESOURCE_EXHAUSTED, name
        assert st.pin_count("101") == 1 and st.pin_count("102") == 1
        st.release(["101", "102"])
        assert st.insert(["103"], [S(status=O.INIT)]) == O.OK
        assert st.candidates() == ["102"], name
        assert st.lookup(["102"], False) == []
        assert len(st.lookup(["101"], False)) == 1 and len(st.lookup(["103"], False)) == 1

        # LookupCapLimit (:621-639)
        st = make(2)
        insert_resident(st, ["101", "102"], [S(status=O.INIT)] * 2)
        assert [h for h, _ in st.lookup(["101", "102", "103"], False)] == ["101", "102"]

        # LookupAvailableSpaceLimit (:758-785)
        st = make(3)
        insert_resident(st, ["101", "102", "103"], [S(status=O.INIT)] * 3)
        assert len(st.lookup(["101"], True)) == 1
        assert [h for h, _ in st.lookup(["101", "102", "103", "104"], False)] == \
            ["101", "102", "103"]
        st.release(["101"])

        # InsertPinsExistingAndNewAlike (:787-817)
        st = make(2)
        insert_resident(st, ["local_1"], [S(status=O.INIT)])
        assert st.insert(["local_1", "remote_1"], [S(status=O.INIT)] * 2) == O.OK
        assert st.pin_count("local_1") == 1 and st.pin_count("remote_1") == 1
        assert st.insert(["remote_2"], [S(host=2, status=O.HOST)]) == O.RESOURCE_EXHAUSTED

        # InsertRejectsRemoteSlices (:819-839)
        st = make(4)
        insert_resident(st, ["h1"], [S(host=1, status=O.HOST)])
        assert st.insert(["h1", "h2"], [S(host=1, status=O.HOST),
                                        S(host=42, status=O.REMOTE)]) == O.INVALID_ARGUMENT
        assert st.pin_count("h1") == 0 and st.lookup(["h2"], False) == []

        # EvictRaceCondition (:841-868): a pinned entry is not evicted.
        st = make(3)
        insert_resident(st, ["local_1"], [S(host=-1, status=O.HOST)])
        assert len(st.lookup(["local_1"], True)) == 1
        assert st.evict(["local_1"]) == 0 and st.pin_count("local_1") == 1
        assert len(st.lookup(["local_1"], False)) == 1

        # SaveSuccess (:1086-1151)
        st = make(10)
        insert_resident(st, ["hash_1", "hash_2"], [S(dev=0), S(dev=1)])
        assert len(st.lookup(["hash_1", "hash_2"], True)) == 2
        assert st.save(["hash_1", "hash_2"]) == O.OK
        done, failed, pending, existing, unreg = st.poll_save_status()
        assert sorted(done) == ["hash_1", "hash_2"] and not failed and not existing \
            and not unreg
        assert (st.rec.d2h_calls, st.rec.h2d_calls) == (1, 0)
        assert st.rec.last_src == [0, 1] and st.rec.last_dst == [0, 1]
        got = st.lookup(["hash_1", "hash_2"], False)
        assert [(b["status"], b["host"], b["dev"]) for _, b in got] == \
            [(O.HOST_AND_HBM, 0, 0), (O.HOST_AND_HBM, 1, 1)], name
        assert st.pin_count("hash_1") == 0  # LocalSaveConsumesTheCallerPin (:1326)

        # LoadSuccess (:1153-1213) and LocalLoadConsumesTheCallerPin (:1379)
        st = make(10)
        insert_resident(st, ["hash_1", "hash_2"], [S(host=0, status=O.HOST),
                                                   S(host=1, status=O.HOST)])
        assert len(st.lookup(["hash_1", "hash_2"], True)) == 2
        assert st.load(["hash_1", "hash_2"], [2, 3]) == O.OK
        done, failed, _ = st.poll_load_status()
        assert sorted(done) == ["hash_1", "hash_2"] and not failed
        assert (st.rec.d2h_calls, st.rec.h2d_calls) == (0, 1)
        assert st.rec.last_src == [0, 1] and st.rec.last_dst == [2, 3]
        got = st.lookup(["hash_1", "hash_2"], False)
        assert [(b["status"], b["host"], b["dev"]) for _, b in got] == \
            [(O.HOST_AND_HBM, 0, 2), (O.HOST_AND_HBM, 1, 3)]
        assert st.pin_count("hash_1") == 0

        # LoadWithSlicesSuccess (:1215-1258)
        st = make(10)
        sl = [S(host=0, status=O.HOST), S(host=1, status=O.HOST)]
        insert_resident(st, ["hash_1", "hash_2"], sl)
        st.lookup(["hash_1", "hash_2"], True)
        assert st.load_slices(["hash_1", "hash_2"], sl, [2, 3]) == O.OK
        assert sorted(st.poll_load_status()[0]) == ["hash_1", "hash_2"]
        assert st.rec.last_src == [0, 1] and st.rec.last_dst == [2, 3]

        # LoadWithSlicesSizeMismatch (:1260-1279)
        st = make(10)
        assert st.load_slices(["hash_1", "hash_2"], [S(host=0, status=O.HOST)], [2, 3]) \
            == O.INVALID_ARGUMENT

        # LoadWithSlicesUnpinnedFails (:1281-1324)
        st = make(10)
        sl = [S(host=0, status=O.HOST)]
        insert_resident(st, ["hash_1"], sl)
        assert st.load_slices(["hash_1"], sl, [2]) == O.FAILED_PRECONDITION
        st.lookup(["hash_1"], True)
        assert st.load_slices(["hash_1"], sl, [2]) == O.OK
        assert st.poll_load_status()[0] == ["hash_1"] and st.pin_count("hash_1") == 0

        # FailedLocalLoadKeepsTheCallerPin (:1423-1470)
        st = make(10)
        st.rec.fail = True
        insert_resident(st, ["hash_1"], [S(host=0, status=O.HOST)])
        st.lookup(["hash_1"], True)
        assert st.load(["hash_1"], [2]) == O.OK
        done, failed, _ = st.poll_load_status()
        assert done == [] and failed == ["hash_1"] and st.pin_count("hash_1") == 1
        assert st.lookup(["hash_1"], False)[0][1]["status"] == O.HOST
        st.release(["hash_1"])
        assert st.pin_count("hash_1") == 0

        # FailedLocalSaveKeepsPinAndFreesHostBlocks (:1472-1524)
        st = make(10)
        st.rec.fail = True
        insert_resident(st, ["hash_1"], [S(dev=3)])
        st.lookup(["hash_1"], True)
        free_before = st.lbm_counts()["free"]
        assert st.save(["hash_1"]) == O.OK
        done, failed = st.poll_save_status()[:2]
        assert done == [] and failed == ["hash_1"] and st.pin_count("hash_1") == 1
        assert st.lbm_counts()["free"] == free_before
        assert st.lookup(["hash_1"], False)[0][1]["status"] == O.HBM

        # UnpinnedLoadIsRefused / UnpinnedSaveIsRefused / SaveRequiresHbmResidency
        st = make(10)
        insert_resident(st, ["hash_1"], [S(host=0, status=O.HOST)])
        assert st.load(["hash_1"], [2]) == O.FAILED_PRECONDITION
        st = make(10)
        insert_resident(st, ["hash_1"], [S(dev=3)])
        assert st.save(["hash_1"]) == O.FAILED_PRECONDITION
        st = make(10)
        assert st.insert(["hash_1"], [S(host=0, status=O.HOST)]) == O.OK
        assert st.save(["hash_1"]) == O.FAILED_PRECONDITION
        assert st.pin_count("hash_1") == 1

        # LoadWithSlicesTwoPeersFails (:1595-1614)
        st = make(10)
        assert st.load_slices(["hash_1", "hash_2"],
                              [S(host=7, status=O.REMOTE, rid=("peer_a", "0", "kv", 0)),
                               S(host=9, status=O.REMOTE, rid=("peer_b", "0", "kv", 0))],
                              [2, 3]) == O.INVALID_ARGUMENT
        # LoadWithSlicesAlreadyLoadingFails (:1616-1638)
        st = make(10)
        sl = [S(host=0, status=O.HOST)]
        insert_resident(st, ["hash_1"], sl)
        st.lookup(["hash_1"], True)
        assert st.load_slices(["hash_1"], sl, [2]) == O.OK
        assert st.load_slices(["hash_1"], sl, [3]) == O.FAILED_PRECONDITION

        # SaveReusesFreedBlocksAfterEvict (:1029-1084)
        st = make(2)
        insert_resident(st, ["hash_1", "hash_2"], [S(dev=0), S(dev=1)])
        st.lookup(["hash_1", "hash_2"], True)
        assert st.save(["hash_1", "hash_2"]) == O.OK and st.poll_save_status()[0]
        assert st.lbm_counts()["locked"] == 2
        assert st.evict(["hash_1", "hash_2"]) == 2
        assert st.lbm_counts()["free"] == 2 and st.lbm_counts()["locked"] == 0
        insert_resident(st, ["hash_3"], [S(dev=0)])
        st.lookup(["hash_3"], True)
        assert st.save(["hash_3"]) == O.OK and st.poll_save_status()[0] == ["hash_3"]
        assert st.lbm_counts()["locked"] == 1

        # ProactiveEvictionWithCandidates (:2316-2429)
        st = make(2)
        insert_resident(st, ["hash_A", "hash_B"], [S(dev=0), S(dev=1)])
        st.lookup(["hash_A", "hash_B"], True)
        assert st.save(["hash_A", "hash_B"]) == O.OK and st.poll_save_status()[0]
        got = st.lookup(["hash_B", "hash_A"], False)
        assert [b["status"] for _, b in got] == [O.HOST_AND_HBM] * 2
        insert_resident(st, ["hash_C"], [S(dev=2)])
        assert st.candidates() == ["hash_B"], (name, st.candidates())
        insert_resident(st, ["hash_D"], [S(dev=3)])
        assert st.candidates() == ["hash_B", "hash_A"]
        st.lookup(["hash_D"], True)
        assert st.save(["hash_D"]) == O.OK and st.poll_save_status()[0] == ["hash_D"]
        assert st.lookup(["hash_B"], False) == []
        got = st.lookup(["hash_D"], False)
        assert got[0][1]["status"] == O.HOST_AND_HBM and got[0][1]["host"] != -1
        assert st.candidates() == ["hash_A"]


def test_store_evict_on_save(kvx):
    """EvictOnSave (kv_cache_store_test.cc:2230-2314) without the registry:
    a 3-entry store over a 2-block controller."""
    for name in ("oracle", "product"):
        if name == "oracle":
            st = OracleStore(3)
            st.lbm = O.LogicalBlockManager(2)
            code, ids = st.lbm.allocate(2, lock=True)
        else:
            st = ProductStore(kvx, 3, host_blocks=2)
            ids = st.s.host_block_manager().allocate(2, lock=True)
        insert_resident(st, ["block_A", "block_B"], [S(host=ids[0], status=O.HOST),
                                                     S(host=ids[1], status=O.HOST)])
        insert_resident(st, ["block_C"], [S(dev=0)])
        st.lookup(["block_C"], True)
        assert st.lbm_counts()["free"] == 0
        assert st.save(["block_C"]) == O.OK
        assert st.poll_save_status()[0] == ["block_C"]
        assert st.lookup(["block_B"], False) == []
        assert len(st.lookup(["block_A"], False)) == 1
        b = st.lookup(["block_C"], False)[0][1]
        assert (b["status"], b["host"], b["dev"]) == (O.HOST_AND_HBM, ids[1], 0)


def test_store_metadata_and_recovery_cases(kvx, shm_key):
    for name in ("oracle", "product"):
        key = f"{shm_key}_{name}"

        def make(cap, md_blocks, recover=False):
            # The table and the controller both cover md_blocks host blocks.
            if name == "oracle":
                st = OracleStore(cap, md_blocks)
                st.lbm = O.LogicalBlockManager(md_blocks)
                return st
            return ProductStore(kvx, cap, md_key=key, md_blocks=md_blocks, recover=recover,
                                host_blocks=md_blocks)

        def seed(entries, blocks):
            # Writes a table as a previous process would have left it.
            if name == "oracle":
                return {bid: (h, seq) for bid, h, seq in entries}
            r = kvx.KVCacheMetadataShmRegion(key, blocks, "m")
            r.reformat()
            for bid, h, seq in entries:
                r.metadata().set(bid, h.encode(), seq)
            r.close()
            return None

        try:
            # MetadataKeepsEvictionCandidates (kv_cache_store_test.cc:901-944)
            seed([], 2)
            st = make(2, 2)
            insert_resident(st, ["host_1", "host_2"], [S(host=0, status=O.HOST),
                                                       S(host=1, status=O.HOST)])
            insert_resident(st, ["host_3"], [S(host=2, status=O.HOST)])
            assert st.candidates() == ["host_2"]
            # The table holds 2 blocks here, so host_3 (block 2) is out of its
            # range; the reference case uses a 4-block table.
            st = None
            seed([], 4)
            st = make(2, 4)
            insert_resident(st, ["host_1", "host_2"], [S(host=0, status=O.HOST),
                                                       S(host=1, status=O.HOST)])
            insert_resident(st, ["host_3"], [S(host=2, status=O.HOST)])
            assert st.metadata_entries() == [(0, "host_1", 1), (1, "host_2", 0),
                                             (2, "host_3", 2)], name
            insert_resident(st, ["host_2"], [S(host=3, status=O.HOST)])
            assert st.candidates() == []
            assert st.metadata_entries() == [(0, "host_1", 1), (2, "host_3", 2),
                                             (3, "host_2", 3)]
            # EvictClearsMetadataEntries (:946-965)
            st = None
            seed([], 2)
            st = make(2, 2)
            insert_resident(st, ["host_1", "host_2"], [S(host=0, status=O.HOST),
                                                       S(host=1, status=O.HOST)])
            assert len(st.metadata_entries()) == 2
            assert st.evict(["host_1"]) == 1
            assert st.metadata_entries() == [(1, "host_2", 0)]

            # RecoverFromLocalManifestRebuildsLruCache (:3211-3255)
            st = None
            table = [(5, "hash_b", 3), (7, "hash_a", 4), (9, "hash_c", 8)]
            md = seed(table, 10)
            st = make(10, 10)
            if md is not None:
                st.md = md
            assert st.recover() == (O.OK, 3)
            got = st.lookup(["hash_a", "hash_b", "hash_c"], False)
            assert [b["host"] for _, b in got] == [7, 5, 9]
            assert all(b["status"] == O.HOST for _, b in got)
            insert_resident(st, ["hash_d"], [S(host=0, status=O.HOST)])
            assert st.metadata_entries() == [(0, "hash_d", 9), (5, "hash_b", 3),
                                             (7, "hash_a", 4), (9, "hash_c", 8)]
            # RecoverFromLocalManifestRebuildsLruOrder (:3257-3280)
            st = None
            md = seed(table, 10)
            st = make(2, 10)
            if md is not None:
                st.md = md
            assert st.recover() == (O.OK, 3)
            assert st.candidates() == ["hash_b"]
            assert len(st.metadata_entries()) == 3
            # RecoverFromLocalManifestKeepsNewestDuplicate (:3282-3316)
            st = None
            md = seed([(2, "dup_hash", 1), (4, "other", 3), (6, "dup_hash", 5)], 10)
            st = make(10, 10)
            if md is not None:
                st.md = md
            assert st.recover() == (O.OK, 2)
            assert st.lookup(["dup_hash"], False)[0][1]["host"] == 6
            assert st.metadata_entries() == [(4, "other", 3), (6, "dup_hash", 5)]
            # RecoverFromLocalManifestFailsOnAllocatorConflict (:3318-3337)
            st = None
            md = seed([(0, "rh1", 0)], 10)
            st = make(10, 10)
            if md is not None:
                st.md = md
            if name == "oracle":
                st.lbm.allocate(1, lock=True)
            else:
                st.s.host_block_manager().allocate(1, lock=True)
            assert st.recover()[0] == O.FAILED_PRECONDITION
            assert st.lookup(["rh1"], False) == []
            assert len(st.metadata_entries()) == 1
            # RecoverFromLocalManifestPreconditions (:3339-3378)
            st = None
            seed([], 10)
            st = make(10, 10)
            insert_resident(st, ["hash_a"], [S(host=0, status=O.HOST)])
            assert st.recover()[0] == O.FAILED_PRECONDITION
            st = None
            seed([], 10)
            st = make(10, 10)
            assert st.recover() == (O.OK, 0)
        finally:
            st = None
            try:
                os.unlink(f"/dev/shm/{key}")
            except FileNotFoundError:
                pass
    # No table at all.
    st = ProductStore(kvx, 10)
    assert st.recover()[0] == O.FAILED_PRECONDITION


def test_store_recovers_at_creation_from_a_surviving_table(kvx, shm_key):
    """kv_cache_store_wrapper.cc:170-185: a warm table is recovered inside
    construction; a failed recovery reformats (cold start)."""
    r = kvx.KVCacheMetadataShmRegion(shm_key + "_metadata", 8, "uid")
    r.metadata().set(3, b"h3", 5)
    r.metadata().set(1, b"h1", 2)
    r.close()
    s = kvx.KVCacheStore(8, num_shards=1, store_server_ip="127.0.0.1",
                         metadata_shm_key=shm_key + "_metadata", model_uid="uid")
    assert s.metadata_warm and s.recovered_blocks == 2
    got = s.lookup([b"h1", b"h3"], pin_found=False)
    assert [(b.host_block_id, b.status) for _, b in got] == \
        [(1, kvx.BlockStatus.HOST), (3, kvx.BlockStatus.HOST)]
    s.close()
    # Another model: the table is re-created empty.
    s = kvx.KVCacheStore(8, num_shards=1, store_server_ip="127.0.0.1",
                         metadata_shm_key=shm_key + "_metadata", model_uid="other")
    assert not s.metadata_warm and s.recovered_blocks == 0
    assert s.lookup([b"h1"], pin_found=False) == []
    s.close()


def test_store_differential_random(kvx):
    """Random local flows: the product and the oracle agree on every answer,
    pin count, evictable order and allocator count."""
    rng = random.Random(11)
    for trial in range(12):
        cap = rng.randint(2, 7)
        a = OracleStore(cap)
        b = ProductStore(kvx, cap)
        keys = [f"k{i}" for i in range(rng.randint(3, 12))]
        for step in range(250):
            op = rng.choice(["insert", "insert", "lookup", "lookup", "release", "save",
                             "load", "poll_save", "poll_load", "evict", "fail"])
            hs = rng.sample(keys, rng.randint(1, min(3, len(keys))))
            if op == "insert":
                specs = []
                for _ in hs:
                    st = rng.choice([O.HBM, O.HBM, O.HOST, O.INIT])
                    specs.append(S(host=rng.randint(0, cap - 1) if st == O.HOST else -1,
                                   dev=rng.randint(0, 50) if st == O.HBM else -1,
                                   status=st))
                ra, rb = a.insert(hs, specs), b.insert(hs, specs)
            elif op == "lookup":
                pin = rng.random() < 0.5
                ra, rb = a.lookup(hs, pin), b.lookup(hs, pin)
            elif op == "release":
                a.release(hs)
                b.release(hs)
                ra = rb = None
            elif op == "save":
                ra, rb = a.save(hs), b.save(hs)
            elif op == "load":
                dev = [rng.randint(0, 50) for _ in hs]
                ra, rb = a.load(hs, dev), b.load(hs, dev)
            elif op == "poll_save":
                ra, rb = a.poll_save_status(), b.poll_save_status()
            elif op == "poll_load":
                ra, rb = a.poll_load_status(), b.poll_load_status()
            elif op == "evict":
                ra, rb = a.evict(hs), b.evict(hs)
            else:
                flag = rng.random() < 0.3
                a.rec.fail = b.rec.fail = flag
                ra = rb = None
            assert ra == rb, (trial, step, op, hs, ra, rb)
            for k in keys:
                assert a.pin_count(k) == b.pin_count(k), (trial, step, op, k)
            assert a.candidates() == b.candidates(), (trial, step, op)
            assert a.evictable() == b.evictable(), (trial, step, op)
            assert a.lbm_counts() == b.lbm_counts(), (trial, step, op)
            assert (a.rec.d2h_calls, a.rec.h2d_calls, a.rec.last_src, a.rec.last_dst) == \
                (b.rec.d2h_calls, b.rec.h2d_calls, b.rec.last_src, b.rec.last_dst)


def test_store_construction_rules(kvx):
    """kv_cache_store_test.cc:5077-5105 and the capacity rule of
    HostOffloadBackend::Create (host_offload_backend.cc:113-117)."""
    for kw in (dict(store_server_ip=""), dict(store_server_ip="0.0.0.0"),
               dict(store_server_ip="::"), dict(store_server_ip="127.0.0.1", num_shards=0)):
        args = dict(num_shards=1)
        args.update(kw)
        with pytest.raises(ValueError):
            kvx.KVCacheStore(4, **args)
    with pytest.raises(ValueError):
        kvx.KVCacheStore(0, num_shards=1, store_server_ip="127.0.0.1")
    s = kvx.KVCacheStore(4, num_shards=1, store_server_ip="localhost",
                         raiden_controller_port=45123)
    assert s.raiden_controller_address == "localhost:45123"
    with pytest.raises(RuntimeError):
        kvx.KVCacheStore(4, num_shards=1, store_server_ip="localhost",
                         raiden_controller_port=45123)
    s.close()


def test_store_lists_cross_whole(kvx):
    """Lists fetched with one library call each (kvx_slices_flat,
    kvx_strings_flat) give every hash and slice as fetching them one by one
    does: slices of two owners interleaved (each with its own RaidenId),
    empty and long hashes, statuses, and a poll's string lists."""
    s = kvx.KVCacheStore(64, num_shards=1, store_server_ip="127.0.0.1")
    a = kvx.RaidenId("job-a", "0", "cache", 0)
    b = kvx.RaidenId("job-b", "3", "other", 2)
    hashes = [b"", b"x" * 111] + [b"h%03d" % i for i in range(30)]
    slices = [kvx.RaidenBlockId(a if i % 3 else b, -1, 100 + i, kvx.BlockStatus.HBM)
              for i in range(len(hashes))]
    assert s.insert(hashes, slices, on_host=False)
    found = s.lookup(hashes, pin_found=False)
    assert [h for h, _ in found] == hashes
    assert [x for _, x in found] == slices
    assert all(x.raiden_id == (a if i % 3 else b) for i, (_, x) in enumerate(found))
    lib = kvx._capi.load()
    import ctypes
    buf, offs, n = kvx._capi.pack_bytes(hashes)
    out = ctypes.c_void_p()
    assert lib.kvx_store_lookup(s._h, buf, offs, n, 0, ctypes.byref(out)) == 0
    h, hl, bs = ctypes.c_void_p(), ctypes.c_int64(), kvx._capi.BlockSlice()
    for i, (hash_, x) in enumerate(found):
        assert lib.kvx_slices_get(out, i, ctypes.byref(h), ctypes.byref(hl), ctypes.byref(bs)) == 0
        assert ctypes.string_at(h, hl.value) == hash_
        assert (bs.job_name.decode(), bs.job_replica_id.decode(), bs.data_name.decode(),
                bs.data_replica_idx) == (x.job_name, x.job_replica_id, x.data_name,
                                         x.data_replica_idx)
        assert (bs.device_block_id, bs.status) == (x.device_block_id, int(x.status))
    lib.kvx_slices_release(out)
    assert lib.kvx_slices_flat(None, None, None, None) == 3
    assert lib.kvx_strings_flat(None, None, None) == 3
    # Saves through no worker fail in the poll: the failed list comes whole.
    assert s.save(hashes[:5])
    done, failed = s.poll_save_status()[:2]
    assert done == [] and sorted(failed) == sorted(hashes[:5])
    s.close()


def test_manager_joins_the_store_controller(kvx):
    """A manager created with the store's controller address becomes its
    worker; an unknown address is an error."""
    s = kvx.KVCacheStore(4, num_shards=1, store_server_ip="127.0.0.1")
    m = kvx.KVCacheManager.create_host_only_for_testing(num_layers=1, slice_byte_size=64,
                                                        host_blocks=4)
    lib = kvx._capi.load()
    assert lib.kvx_manager_register_with_controller(
        m._h, s.raiden_controller_address.encode()) == 0
    assert lib.kvx_manager_register_with_controller(m._h, b"127.0.0.1:1") == 14
    # The CPU-only worker cannot D2h: the save fails in the poll and frees its
    # host block, exactly like a failed transfer.
    rid = kvx.RaidenId("j", "0", "d", 0)
    assert s.insert([b"a"], [kvx.RaidenBlockId(rid, -1, 0, kvx.BlockStatus.HBM)], False)
    assert s.save([b"a"])
    done, failed = s.poll_save_status()[:2]
    assert done == [] and failed == [b"a"]
    assert s.host_block_manager().num_free_blocks == 4
    m.close()
    s.close()


def test_crash_recovery_across_processes(kvx, shm_key, tmp_path):
    """kv_cache_store_recovery_e2e_test.py restated on the CPU: phase A
    writes host blocks into a shared-memory pool, records them in the store
    and dies by SIGKILL; phase B recovers the index and reads the bytes back.
    A model_uid change forces a cold start."""
    script = tmp_path / "phase.py"
    script.write_text(_RECOVERY_SCRIPT)
    env = dict(os.environ, RAIDEN_SHM_KEY=shm_key, RAIDEN_SHM_MODEL_UID="recovery_model",
               PYTHONPATH=ROOT)
    a = subprocess.run([sys.executable, str(script), "a"], env=env, capture_output=True,
                       text=True, timeout=120)
    assert a.returncode == -9, a.stderr
    assert "PHASE_A_SAVED" in a.stdout
    b = subprocess.run([sys.executable, str(script), "b"], env=env, capture_output=True,
                       text=True, timeout=120)
    assert b.returncode == 0, b.stderr
    assert "PHASE_B_RECOVERED" in b.stdout and "PHASE_B_BYTES" in b.stdout
    env["RAIDEN_SHM_MODEL_UID"] = "another_model"
    c = subprocess.run([sys.executable, str(script), "cold"], env=env, capture_output=True,
                       text=True, timeout=120)
    assert c.returncode == 0, c.stderr
    assert "PHASE_B_COLD" in c.stdout
    for suffix in ("_metadata",):
        try:
            os.unlink(f"/dev/shm/{shm_key}{suffix}")
        except FileNotFoundError:
            pass


_RECOVERY_SCRIPT = r'''
import os, signal, sys
import __graft_entry__
kvx = __graft_entry__.load_package()
N, BB = 4, 256
HASHES = [b"hash_%d" % i for i in range(N)]

def stack():
    store = kvx.KVCacheStore(N, raiden_id=kvx.RaidenId("rec", "0", "cache", 0),
                             num_shards=1, store_server_ip="127.0.0.1")
    mgr = kvx.KVCacheManager.create_host_only_for_testing(
        num_layers=2, slice_byte_size=BB, host_blocks=N, host_alloc="shm")
    return store, mgr

def payload(layer, i):
    return bytes((layer * 97 + i * 13 + j) % 256 for j in range(BB))

phase = sys.argv[1]
store, mgr = stack()
rid = store.raiden_id
if phase == "a":
    assert not mgr.shm_warm
    for i in range(N):
        for layer in range(2):
            mgr.write_block_bytes(layer, i, payload(layer, i))
    slices = [kvx.RaidenBlockId(rid, i, -1, kvx.BlockStatus.HOST) for i in range(N)]
    assert store.insert(HASHES, slices, True)
    store.release(HASHES)
    print("PHASE_A_SAVED", flush=True)
    os.kill(os.getpid(), signal.SIGKILL)
elif phase == "b":
    assert mgr.shm_warm and store.metadata_warm
    got = store.lookup(HASHES)
    assert len(got) == N, got
    for i, (h, b) in enumerate(got):
        assert h == HASHES[i] and b.status == kvx.BlockStatus.HOST and b.host_block_id == i
    print("PHASE_B_RECOVERED", flush=True)
    for i in range(N):
        for layer in range(2):
            assert mgr.read_block_bytes(layer, i) == payload(layer, i)
    store.release(HASHES)
    print("PHASE_B_BYTES", flush=True)
else:
    assert not mgr.shm_warm and not store.metadata_warm
    got = store.lookup(HASHES)
    assert got == [], got
    print("PHASE_B_COLD", flush=True)
'''
