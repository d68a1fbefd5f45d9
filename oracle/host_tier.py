"""ORACLE -- test infrastructure only.

Pure-Python restatements of the reference's host-tier bookkeeping, written
the way the reference computes it (full scans and sorts, plain lists), to
check the product's data structures by differential testing on random
operation sequences. Only tests/ import this module.

  LogicalBlockManager  tpu_sync/kv_cache/logical_block_manager.cc:31-235
  LRUCache             tpu_sync/kv_cache/lru_cache.h:41-369
  metadata byte format tpu_sync/kv_cache/kv_cache_metadata.h:34-70,
                       kv_cache_metadata.cc:117-183
  Store (local flows)  tpu_sync/kv_cache/kv_cache_store.cc:837-1226,
                       1453-1551, 1743-1811, 2113-2253 over
                       tpu_sync/kv_cache/host_offload_backend.cc:154-690

Parity status: each class is pinned by the reference tests' known answers
restated in tests/golden/ (LRU: lru_cache_test.cc; metadata:
kv_cache_metadata_test.cc; store: kv_cache_store_test.cc local cases), run
against both this oracle and the product, plus the struct-definition byte
layout for the metadata table.
"""

OK, INVALID_ARGUMENT, RESOURCE_EXHAUSTED, FAILED_PRECONDITION = 0, 3, 8, 9


class LogicalBlockManager:
    """Scan-and-sort allocator; returns (code, value) pairs instead of raising."""

    def __init__(self, n):
        self.total = max(n, 0)
        self.counter = 0
        self.alloc = [False] * self.total
        self.locked = [False] * self.total
        self.last = [0] * self.total

    def allocate(self, k, lock=False):
        if k <= 0 or k > self.total:
            return INVALID_ARGUMENT, None
        free = [i for i in range(self.total) if not self.alloc[i]]
        evictable = [i for i in range(self.total) if self.alloc[i] and not self.locked[i]]
        if len(free) + len(evictable) < k:
            return RESOURCE_EXHAUSTED, None
        ids = free[:k]
        need = k - len(ids)
        if need > 0:
            evictable.sort(key=lambda i: (self.last[i], i))
            ids += evictable[:need]
        self.counter += 1
        for i in ids:
            self.alloc[i] = True
            self.locked[i] = bool(lock)
            self.last[i] = self.counter
        return OK, ids

    def allocate_target(self, ids):
        seen = set()
        for i in ids:
            if i < 0 or i >= self.total:
                return INVALID_ARGUMENT
            if self.alloc[i]:
                return FAILED_PRECONDITION
            if i in seen:
                return INVALID_ARGUMENT
            seen.add(i)
        self.counter += 1
        for i in ids:
            self.alloc[i] = True
            self.locked[i] = True
            self.last[i] = self.counter
        return OK

    def unlock(self, ids):
        for i in ids:
            if i < 0 or i >= self.total or not self.alloc[i]:
                return INVALID_ARGUMENT
        for i in ids:
            self.locked[i] = False
        return OK

    def deallocate(self, ids):
        for i in ids:
            if i < 0 or i >= self.total or not self.alloc[i]:
                return INVALID_ARGUMENT
        for i in ids:
            self.alloc[i] = False
            self.locked[i] = False
        return OK

    def access(self, i):
        if i < 0 or i >= self.total or not self.alloc[i]:
            return INVALID_ARGUMENT
        self.counter += 1
        self.last[i] = self.counter
        return OK

    def counts(self):
        return {"total": self.total,
                "free": sum(1 for a in self.alloc if not a),
                "allocated": sum(1 for a in self.alloc if a),
                "locked": sum(1 for x in self.locked if x)}


# ---------------------------------------------------------------------------
# LRUCache: tpu_sync/kv_cache/lru_cache.h:41-369, restated with three Python
# lists. ``lru`` and ``pinned`` hold keys with index 0 = front (MRU);
# ``cand`` holds eviction candidates with index 0 = front (oldest).
# ---------------------------------------------------------------------------
LRU, PINNED, CAND = "lru", "pinned", "cand"


class LRUCache:
    def __init__(self, capacity):
        self.capacity = capacity
        self.lists = {LRU: [], PINNED: [], CAND: []}
        self.entries = {}  # key -> [value, pins, location]

    # sizes (lru_cache.h:57-70)
    def size(self):
        return len(self.entries)

    def active_size(self):
        return len(self.lists[LRU]) + len(self.lists[PINNED])

    def available_space(self):
        p = len(self.lists[PINNED])
        return self.capacity - p if self.capacity > p else 0

    def contains(self, k):
        return k in self.entries and self.entries[k][2] != CAND

    def _move(self, k, where, front):
        e = self.entries[k]
        self.lists[e[2]].remove(k)
        if front:
            self.lists[where].insert(0, k)
        else:
            self.lists[where].append(k)
        e[2] = where

    def _promote(self, k, front=True):  # Promote / PromoteBack (:320-352)
        e = self.entries[k]
        self._move(k, PINNED if e[1] > 0 else LRU, front)

    def put(self, k, v):  # :99-122
        if k in self.entries:
            self.entries[k][0] = v
            self._promote(k)
            return None
        evicted = None
        if self.active_size() >= self.capacity:
            evicted = self.evict()
            if evicted is None:
                return None
        self.entries[k] = [v, 0, LRU]
        self.lists[LRU].insert(0, k)
        return evicted

    def put_back(self, k, v):  # :124-140
        if k in self.entries:
            self.entries[k][0] = v
            self._promote(k, front=False)
            return
        if self.active_size() >= self.capacity:
            self.evict()
        self.entries[k] = [v, 0, LRU]
        self.lists[LRU].append(k)

    def get(self, k):  # :142-152
        if k not in self.entries:
            return None
        self._promote(k)
        return self.entries[k][0]

    def peek(self, k):  # :154-164
        e = self.entries.get(k)
        return None if e is None or e[2] == CAND else e[0]

    def peek_including_candidates(self, k):
        e = self.entries.get(k)
        return None if e is None else e[0]

    def get_and_pin(self, k):  # :197-216
        e = self.entries.get(k)
        if e is None:
            return None
        if e[1] == 0:
            self._move(k, PINNED, True)
        e[1] += 1
        return e[0]

    def pin(self, k):
        return self.get_and_pin(k) is not None

    def unpin(self, k):  # :227-243
        e = self.entries.get(k)
        if e is None:
            return False
        if e[1] > 0:
            e[1] -= 1
            if e[1] == 0:
                self._move(k, LRU, True)
        return True

    def pin_count(self, k):
        e = self.entries.get(k)
        return 0 if e is None else e[1]

    def evictable_keys(self, count):  # :260-280
        keys = list(self.lists[CAND][:count])
        for k in reversed(self.lists[LRU]):
            if len(keys) >= count:
                break
            keys.append(k)
        return keys

    def erase(self, k):  # :282-296
        e = self.entries.get(k)
        if e is None or e[1] > 0:
            return False
        self.lists[e[2]].remove(k)
        del self.entries[k]
        return True

    def evict(self):  # :298-307
        if not self.lists[LRU]:
            return None
        k = self.lists[LRU][-1]
        self._move(k, CAND, False)
        return (k, self.entries[k][0])

    def candidate_keys(self):
        return list(self.lists[CAND])

    def clear(self):
        self.__init__(self.capacity)


# ---------------------------------------------------------------------------
# KVCacheMetadata byte format: tpu_sync/kv_cache/kv_cache_metadata.h:34-70.
# ---------------------------------------------------------------------------
import struct as _struct

METADATA_MAGIC = 0x52414944454E4B4D  # "RAIDENKM"
METADATA_HEADER = 128
METADATA_ENTRY = 128
MAX_HASH = 112


def metadata_header(num_blocks, model_uid=b""):
    """The 128 header bytes Format writes."""
    return (_struct.pack("<QIII", METADATA_MAGIC, 1, num_blocks, METADATA_ENTRY)
            + model_uid.ljust(64, b"\0") + b"\0" * (128 - 84))


def metadata_entry(seq, block_hash, valid=1):
    """The 128 entry bytes of a committed Set (reserved bytes zero)."""
    return (_struct.pack("<QHB", seq, len(block_hash), valid) + b"\0" * 5
            + block_hash.ljust(MAX_HASH, b"\0"))


def metadata_valid_entries(region, num_blocks):
    """ValidEntries (kv_cache_metadata.cc:166-183) parsed from raw bytes."""
    out = []
    for i in range(num_blocks):
        off = METADATA_HEADER + i * METADATA_ENTRY
        seq, hlen, valid = _struct.unpack_from("<QHB", region, off)
        if valid == 0 or hlen == 0 or hlen > MAX_HASH:
            continue
        out.append((i, bytes(region[off + 16:off + 16 + hlen]), seq))
    return out


# ---------------------------------------------------------------------------
# KVCacheStore local flows over HostOffloadBackend:
#   tpu_sync/kv_cache/kv_cache_store.cc:837-1226, 1453-1551, 1743-1811,
#   2113-2253; tpu_sync/kv_cache/host_offload_backend.cc:154-620, 656-690.
# Transfers complete synchronously through ``transfer(d2h, src, dst)`` which
# returns a status code; a save or load finishes in the next poll, as a ready
# future does in the reference.
# ---------------------------------------------------------------------------
INIT, REMOTE, HBM, HOST, HOST_AND_HBM = 0, 1, 2, 3, 4
NOT_FOUND = 5


def _on_host(b):
    return b["status"] in (HOST, HOST_AND_HBM)


class Store:
    def __init__(self, capacity, metadata_blocks=None, transfer=None):
        self.capacity = capacity
        self.lru = LRUCache(capacity)
        self.lbm = LogicalBlockManager(capacity)
        # metadata table: block id -> (hash, seq) for valid entries
        self.md = {} if metadata_blocks is not None else None
        self.md_blocks = metadata_blocks
        self.next_seq = 0
        self.saving, self.loading = set(), set()
        self.active_saves, self.active_loads = [], []
        self.done_saves, self.failed_saves = [], []
        self.done_loads, self.failed_loads = [], []
        self.transfer = transfer

    # metadata mirror (host_offload_backend.cc:1224-1254)
    def _md_set(self, h, b):
        if self.md is None or not _on_host(b):
            return
        bid = b["host"]
        seq = self.next_seq
        self.next_seq += 1
        if 0 <= bid < self.md_blocks and 0 < len(h) <= MAX_HASH:
            self.md[bid] = (h, seq)

    def _md_clear(self, b):
        if self.md is None or not _on_host(b):
            return
        self.md.pop(b["host"], None)

    def metadata_entries(self):
        return sorted((bid, h, s) for bid, (h, s) in (self.md or {}).items())

    # backend
    def _lookup(self, hashes, pin_found):
        hit = []
        for h in hashes:
            found = self.lru.peek(h) is not None
            if found and pin_found:
                self.lru.pin(h)
            hit.append(found)
        out = []
        for i, h in enumerate(hashes):
            if not hit[i] or self.lru.peek(h) is None:
                break
            out.append((h, dict(self.lru.peek(h))))
        if pin_found:
            for i in range(len(out), len(hashes)):
                if hit[i]:
                    self.lru.unpin(hashes[i])
        return out

    def _update(self, hashes, slices):
        for i, h in enumerate(hashes):
            if self.lru.contains(h):
                if i < len(slices):
                    self.lru.entries[h][0] = dict(slices[i])
                    self._md_set(h, slices[i])
                continue
            stale = self.lru.peek_including_candidates(h)
            if stale is not None:
                self._md_clear(stale)
            if i < len(slices):
                self.lru.put(h, dict(slices[i]))
                self._md_set(h, slices[i])
            else:
                self.lru.put(h, {"host": -1, "dev": -1, "status": INIT})

    def _insert_and_lock(self, hashes, slices):
        have = [i for i, h in enumerate(hashes) if self.lru.contains(h)]
        fresh = [i for i, h in enumerate(hashes) if not self.lru.contains(h)]
        for k, i in enumerate(have):
            if not self.lru.pin(hashes[i]):
                for j in have[:k]:
                    self.lru.unpin(hashes[j])
                return False
            if i < len(slices):
                cur = self.lru.peek(hashes[i])
                if cur is not None and cur["status"] == HBM:
                    self._md_clear(cur)
                    self.lru.entries[hashes[i]][0] = dict(slices[i])
                    self._md_set(hashes[i], slices[i])
        if self.lru.available_space() < len(fresh):
            for i in have:
                self.lru.unpin(hashes[i])
            return False
        for i in reversed(fresh):
            stale = self.lru.peek_including_candidates(hashes[i])
            if stale is not None:
                self._md_clear(stale)
            if i < len(slices):
                self.lru.put(hashes[i], dict(slices[i]))
                self._md_set(hashes[i], slices[i])
            else:
                self.lru.put(hashes[i], {"host": -1, "dev": -1, "status": INIT})
        for k, i in enumerate(fresh):
            if not self.lru.pin(hashes[i]):
                for j in fresh[:k]:
                    self.lru.unpin(hashes[j])
                for j in have:
                    self.lru.unpin(hashes[j])
                for j in fresh:
                    v = self.lru.peek_including_candidates(hashes[j])
                    if v is not None:
                        self._md_clear(v)
                    self.lru.erase(hashes[j])
                return False
        return True

    def _release(self, hashes):
        for h in reversed(hashes):
            self.lru.unpin(h)

    def _evict_backend(self, hashes):
        ids = []
        for h in hashes:
            b = self.lru.peek_including_candidates(h)
            if b is not None and self.lru.pin_count(h) == 0 and _on_host(b):
                ids.append(b["host"])
                self._md_clear(b)
                self.lru.erase(h)
        return ids

    # store
    def lookup(self, hashes, pin_found):
        out = self._lookup(hashes, pin_found)
        if self.capacity > 0 and len(out) > self.capacity:
            if pin_found:
                self._release([h for h, _ in out[self.capacity:]])
            out = out[:self.capacity]
        return out

    def insert(self, hashes, slices):
        if any(s["status"] == REMOTE for s in slices):
            return INVALID_ARGUMENT
        return OK if self._insert_and_lock(hashes, slices) else RESOURCE_EXHAUSTED

    def release(self, hashes):
        self._release(hashes)

    def evict(self, hashes):
        ids = self._evict_backend(hashes)
        if ids:
            self.lbm.deallocate(ids)
        return len(ids)

    def _allocate(self, needed):
        free = self.lbm.counts()["free"]
        to_free = needed - free
        if to_free > 0:
            victims = self.lru.evictable_keys(to_free)
            if len(victims) < to_free:
                return RESOURCE_EXHAUSTED, None
            self.evict(victims)
        return self.lbm.allocate(needed, lock=True)

    def _run(self, d2h, src, dst):
        return self.transfer(d2h, src, dst) if self.transfer else FAILED_PRECONDITION

    def save(self, hashes):
        found = self._lookup(hashes, False)
        if len(found) < len(hashes):
            return NOT_FOUND
        src = []
        for i, (h, b) in enumerate(found):
            if b["status"] != HBM or b["dev"] == -1 or self.lru.pin_count(h) <= 0 \
                    or h in self.saving:
                return FAILED_PRECONDITION
            src.append(b["dev"])
        self.saving.update(hashes)
        code, host = self._allocate(len(hashes))
        if code != OK:
            self.saving.difference_update(hashes)
            return code
        self.active_saves.append((self._run(True, src, host), list(hashes), host))
        return OK

    def load(self, hashes, dev):
        if len(hashes) != len(dev):
            return INVALID_ARGUMENT
        if not hashes:
            return OK
        found = self._lookup(hashes, False)
        if len(found) < len(hashes):
            return NOT_FOUND
        for h, b in found:
            if b["status"] == REMOTE:
                return INVALID_ARGUMENT
            if self.lru.pin_count(h) <= 0 or h in self.loading or not _on_host(b) \
                    or b["host"] == -1:
                return FAILED_PRECONDITION
        self.loading.update(hashes)
        src = [b["host"] for _, b in found]
        self.active_loads.append((self._run(False, src, list(dev)), list(hashes), list(dev)))
        return OK

    def load_slices(self, hashes, slices, dev):
        if len(hashes) != len(slices) or len(slices) != len(dev):
            return INVALID_ARGUMENT
        if not hashes:
            return OK
        remote = slices[0]["status"] == REMOTE
        for h, s in zip(hashes, slices):
            if h in self.loading:
                return FAILED_PRECONDITION
            if remote:
                if s["status"] != REMOTE or s.get("rid") != slices[0].get("rid"):
                    return INVALID_ARGUMENT
            elif self.lru.pin_count(h) <= 0 or not _on_host(s) or s["host"] == -1:
                return FAILED_PRECONDITION
        self.loading.update(hashes)
        code = FAILED_PRECONDITION if remote else \
            self._run(False, [s["host"] for s in slices], list(dev))
        self.active_loads.append((code, list(hashes), list(dev)))
        return OK

    def _poll(self):
        saves, self.active_saves = self.active_saves, []
        for code, hashes, host in saves:
            if code == OK:
                found = self._lookup(hashes, False)
                upd_h, upd_s = [], []
                for i, h in enumerate(hashes):
                    if i < len(found):
                        b = dict(found[i][1])
                        b["host"], b["status"] = host[i], HOST_AND_HBM
                        upd_h.append(h)
                        upd_s.append(b)
                    self.done_saves.append(h)
                if upd_h:
                    self._update(upd_h, upd_s)
                    self._release(upd_h)
            else:
                self.lbm.deallocate(host)
                self.failed_saves.extend(hashes)
            self.saving.difference_update(hashes)
        loads, self.active_loads = self.active_loads, []
        for code, hashes, dev in loads:
            if code == OK:
                found = self._lookup(hashes, False)
                upd_h, upd_s = [], []
                for i, h in enumerate(hashes):
                    if i < len(found):
                        b = dict(found[i][1])
                        b["dev"], b["status"] = dev[i], HOST_AND_HBM
                        upd_h.append(h)
                        upd_s.append(b)
                    self.done_loads.append(h)
                if upd_h:
                    self._update(upd_h, upd_s)
                    self._release(upd_h)
            else:
                self.failed_loads.extend(hashes)
            self.loading.difference_update(hashes)

    def poll_save_status(self):
        self._poll()
        done, failed = self.done_saves, self.failed_saves
        self.done_saves, self.failed_saves = [], []
        return done, failed, [], [], []

    def poll_load_status(self):
        self._poll()
        done, failed = self.done_loads, self.failed_loads
        self.done_loads, self.failed_loads = [], []
        return done, failed, []

    def recover(self):
        """RecoverFromLocalManifest (host_offload_backend.cc:559-620)."""
        if self.lru.size() > 0:
            return FAILED_PRECONDITION, None
        if self.md is None:
            return FAILED_PRECONDITION, None
        entries = self.metadata_entries()
        if not entries:
            return OK, 0
        newest = {}
        for bid, h, seq in entries:
            if h not in newest or seq > newest[h][2]:
                newest[h] = (bid, h, seq)
        keep = sorted(newest.values(), key=lambda e: (e[2], e[0]))
        code = self.lbm.allocate_target([e[0] for e in keep])
        if code != OK:
            return code, None
        for bid, h, seq in keep:
            self.lru.put(h, {"host": bid, "dev": -1, "status": HOST})
        self.next_seq = max(e[2] for e in keep) + 1
        for bid, h, seq in entries:
            if newest[h][0] != bid:
                self.md.pop(bid, None)
        return OK, len(keep)
