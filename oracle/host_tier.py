"""ORACLE -- test infrastructure only.

Pure-Python restatements of the reference's host-tier bookkeeping, written
the way the reference computes it (full scans and sorts), to check the
product's faster data structures by differential testing on random
operation sequences. Only tests/ import this module.

  LogicalBlockManager  tpu_sync/kv_cache/logical_block_manager.cc:31-235
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
