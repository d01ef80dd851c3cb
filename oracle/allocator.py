"""Restatement of the reference's block allocator (TEST INFRASTRUCTURE ONLY).

Follows Sources/PagedAttentionMetal/KVCacheManager.swift:
  free list           :101   Deque(reversed(0..<maxBlocks)); allocation removeLast (:241-248)
  appendTokens        :115-174 (copy-on-write of a shared partial tail, prefix-hash reuse)
  copyOnWrite         :176-194 (the block copy itself is data movement, recorded here)
  ensureExclusiveAccess :200-214
  freeSequence        :216-239 (FIFO prepend / LIFO append / best-fit size bookkeeping)
  allocateBestFit     :250-265, rebuildFreeList :267-283
  memoryStats         :353-378
  batch slab          :661-703 (BatchKVCacheManager.getBatchBlockTableBuffer / getSeqLengthsBuffer)
and the C ABI's per-call batch view (PagedAttentionCABI.swift:339-372).

Pure Python on purpose: it is the checker for libpam's C++ allocator.
"""
from __future__ import annotations

from collections import deque

FIFO, LIFO, BEST_FIT = 0, 1, 2


class OutOfMemory(Exception):
    pass


class SequenceNotFound(Exception):
    pass


class SequenceAlreadyExists(Exception):
    pass


class InvalidRequest(Exception):
    pass


class RefAllocator:
    def __init__(self, max_blocks: int, block_size: int = 16):
        self.max_blocks = max_blocks
        self.block_size = block_size
        self.free = deque(reversed(range(max_blocks)))
        self.policy = FIFO
        self.free_sizes: dict[int, int] = {}
        self.seqs: dict[int, dict] = {}
        self.prefix: dict[int, int] = {}
        self.ref = [0] * max_blocks
        self.prefix_hits = 0
        self.copies: list[tuple[int, int]] = []  # (src, dst) block copies issued by CoW

    # KVCacheManager.swift:65-67 + :267-283
    def set_policy(self, policy: int):
        self.policy = policy
        if policy in (FIFO, LIFO):
            self.free = deque(reversed(self.free))
            self.free_sizes.clear()
        else:
            for b in self.free:
                self.free_sizes.setdefault(b, self.block_size)
            self.free = deque(sorted(self.free, key=lambda b: -self.free_sizes.get(b, 0)))

    def allocate_sequence(self, sid: int):
        if sid in self.seqs:
            raise SequenceAlreadyExists()
        self.seqs[sid] = {"bt": [], "len": 0}

    def _alloc(self) -> int:
        if self.policy in (FIFO, LIFO):
            return self.free.pop()
        best_i, best_d = 0, None
        for i, b in enumerate(self.free):
            held = self.free_sizes.get(b, self.block_size)
            dd = abs(held - self.block_size)
            if best_d is None or dd < best_d:
                best_d, best_i = dd, i
        b = self.free[best_i]
        del self.free[best_i]
        self.free_sizes.pop(b, None)
        return b

    def _cow(self, seq, idx: int):
        if not self.free:
            raise OutOfMemory()
        old = seq["bt"][idx]
        new = self._alloc()
        self.copies.append((old, new))
        self.ref[old] -= 1
        self.ref[new] = 1
        seq["bt"][idx] = new

    def append_tokens(self, sid: int, count: int, hashes=None):
        if count < 0:
            raise InvalidRequest("count must be non-negative")
        if count == 0:
            return
        if sid not in self.seqs:
            raise SequenceNotFound()
        seq = {"bt": list(self.seqs[sid]["bt"]), "len": self.seqs[sid]["len"]}
        bs = self.block_size
        cur = seq["len"]
        new_len = cur + count
        now = (cur + bs - 1) // bs
        after = (new_len + bs - 1) // bs
        extra = after - now
        if now > 0 and cur % bs != 0:
            last = seq["bt"][now - 1]
            if self.ref[last] > 1:
                self._cow(seq, now - 1)
        if extra > 0:
            if len(self.free) < extra:
                # a CoW above has already moved free-list and refcount state while the
                # sequence's own table change is dropped, as in the reference
                raise OutOfMemory()
            for i in range(extra):
                if hashes is not None and i < len(hashes) and hashes[i] in self.prefix:
                    b = self.prefix[hashes[i]]
                    seq["bt"].append(b)
                    self.ref[b] += 1
                    self.prefix_hits += 1
                    continue
                b = self._alloc()
                seq["bt"].append(b)
                self.ref[b] = 1
                if hashes is not None and i < len(hashes):
                    self.prefix[hashes[i]] = b
        seq["len"] = new_len
        self.seqs[sid] = seq

    def ensure_exclusive(self, sid: int, idx: int):
        if sid not in self.seqs:
            raise SequenceNotFound()
        seq = self.seqs[sid]
        if idx >= len(seq["bt"]):
            raise InvalidRequest("block index out of range")
        if self.ref[seq["bt"][idx]] > 1:
            self._cow(seq, idx)

    def register_block_hash(self, h: int, block: int):
        self.prefix[h] = block

    def free_sequence(self, sid: int):
        seq = self.seqs.pop(sid, None)
        if seq is None:
            return
        bs = self.block_size
        total = len(seq["bt"])
        rem = seq["len"] % bs
        last_tokens = bs if rem == 0 else rem
        for i, b in enumerate(seq["bt"]):
            self.ref[b] -= 1
            if self.ref[b] <= 0:
                if self.policy == FIFO:
                    self.free.appendleft(b)
                elif self.policy == LIFO:
                    self.free.append(b)
                else:
                    self.free_sizes[b] = bs if i < total - 1 else last_tokens
                    self.free.append(b)

    def block_table(self, sid: int):
        if sid not in self.seqs:
            raise SequenceNotFound()
        return list(self.seqs[sid]["bt"])

    def seq_len(self, sid: int) -> int:
        if sid not in self.seqs:
            raise SequenceNotFound()
        return self.seqs[sid]["len"]

    @property
    def available(self) -> int:
        return len(self.free)

    def stats(self, bytes_per_block_kv: int):
        used = self.max_blocks - len(self.free)
        partial = sum(1 for s in self.seqs.values() if 0 < s["len"] % self.block_size < self.block_size)
        active = max(len(self.seqs), 1)
        return {
            "total_blocks": self.max_blocks,
            "used_blocks": used,
            "free_blocks": len(self.free),
            "active_sequences": len(self.seqs),
            "total_memory_bytes": self.max_blocks * bytes_per_block_kv,
            "used_memory_bytes": used * bytes_per_block_kv,
            "partially_filled_blocks": partial,
            "fragmentation_ratio": partial / active,
            "prefix_cache_hits": self.prefix_hits,
            "prefix_cache_entries": len(self.prefix),
            "shared_blocks": sum(1 for r in self.ref if r > 1),
        }

    def batch_view(self, ids):
        """PagedAttentionCABI.swift:339-372: zero-padded [B][maxNumBlocks] + lengths."""
        max_nb = max([1] + [len(self.seqs[i]["bt"]) for i in ids])
        bt = [[0] * max_nb for _ in ids]
        for r, i in enumerate(ids):
            for c, b in enumerate(self.seqs[i]["bt"]):
                bt[r][c] = b
        return bt, [self.seqs[i]["len"] for i in ids], max_nb
