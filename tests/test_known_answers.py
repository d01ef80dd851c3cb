"""Hand-worked known answers for the allocator's eviction policies, its memory
statistics and the scheduler's admission order (CPU only, no GPU calls).

Every expected list below was worked out by hand from the reference source and
is written literally; each case runs against BOTH the oracle restatements
(oracle/allocator.py, oracle/scheduler.py) and libpam's C++, so a slip shared
by the two (prepend vs append, ascending vs descending sort, running before
waiting) fails here. The rules each case follows:

  KVCacheManager.swift:101      free list = Deque(reversed(0..<maxBlocks))
  KVCacheManager.swift:65-67    evictionPolicy didSet -> rebuildFreeList (on every set)
  KVCacheManager.swift:216-239  freeSequence: FIFO prepend, LIFO append, best-fit append
                                recording held tokens (blockSize, lastTokens for the tail)
  KVCacheManager.swift:241-248  FIFO/LIFO allocate = removeLast
  KVCacheManager.swift:250-265  best-fit = first minimum |held - blockSize| in deque order
  KVCacheManager.swift:267-283  rebuild: FIFO/LIFO reverse (and forget sizes); best-fit
                                fills missing sizes with blockSize and sorts by held
                                size, descending (Swift's sort keeps equal keys in order)
  KVCacheManager.swift:353-378  memoryStats / fragmentationRatio
  Scheduler.swift:78-114        step: waiting (arrival order, capped at maxBatchSize),
                                then running && !isDone, then paused
  Scheduler.swift:135-152       handleMemoryPressure: pause the newest running first
"""
import ctypes as C

import pytest

from oracle.allocator import BEST_FIT, FIFO, LIFO, OutOfMemory, RefAllocator
from oracle.scheduler import PAUSED, RUNNING, WAITING, COMPLETED, RefScheduler


@pytest.fixture(scope="module")
def pam():
    from pagedattentionmetal_amd import _lib
    return _lib.load()


@pytest.fixture()
def ctx(pam):
    c = pam.pam_create_context()
    assert c
    yield c
    pam.pam_destroy_context(c)


class Both:
    """Drives libpam's host cache and the oracle allocator with the same calls and
    returns their (identical) answers."""

    def __init__(self, pam, ctx, max_blocks, bs=4, hd=32, hkv=1, dtype=0):
        self.pam, self.ctx = pam, ctx
        self.c = pam.pam_create_cache_host(ctx, max_blocks, bs, hd, hkv, dtype)
        assert self.c, pam.pam_last_error(ctx)
        self.ref = RefAllocator(max_blocks, bs)

    def close(self):
        self.pam.pam_destroy_cache(self.c)

    def policy(self, p):
        assert self.pam.pam_set_eviction_policy(self.c, p) == 0
        self.ref.set_policy(p)

    def add(self, sid, tokens, hashes=None):
        """reserve + append; returns the block table both sides agree on."""
        assert self.pam.pam_reserve_sequence(self.ctx, self.c, sid) == 0
        self.ref.allocate_sequence(sid)
        return self.append(sid, tokens, hashes)

    def append(self, sid, tokens, hashes=None):
        if hashes is None:
            rc = self.pam.pam_append_tokens(self.ctx, self.c, sid, tokens)
        else:
            arr = (C.c_uint64 * len(hashes))(*hashes)
            rc = self.pam.pam_append_tokens_hashed(self.ctx, self.c, sid, tokens, arr, len(hashes))
        try:
            self.ref.append_tokens(sid, tokens, hashes)
            ok = True
        except OutOfMemory:
            ok = False
        assert (rc == 0) == ok
        if not ok:
            assert b"outOfMemory" in self.pam.pam_last_error(self.ctx)
            return None
        return self.table(sid)

    def free(self, sid):
        self.pam.pam_free_sequence(self.c, sid)
        self.ref.free_sequence(sid)

    def table(self, sid):
        n = self.pam.pam_block_table(self.ctx, self.c, sid, None, 0)
        buf = (C.c_int32 * max(n, 1))()
        self.pam.pam_block_table(self.ctx, self.c, sid, buf, n)
        mine = list(buf[:n])
        assert mine == self.ref.block_table(sid)
        return mine

    def available(self):
        n = self.pam.pam_available_blocks(self.c)
        assert n == self.ref.available
        return n


def test_fifo_reuses_freed_blocks_last(pam, ctx):
    b = Both(pam, ctx, 8)
    assert b.add(1, 8) == [0, 1]          # removeLast of [7..0]
    assert b.add(2, 4) == [2]
    b.free(1)                              # prepend 0, then 1: [1, 0, 7, 6, 5, 4, 3]
    assert b.add(3, 12) == [3, 4, 5]
    assert b.add(4, 20) is None            # 5 blocks needed, 4 free
    assert b.add(5, 16) == [6, 7, 0, 1]
    assert b.available() == 0
    b.close()


def test_lifo_reuses_freed_blocks_first(pam, ctx):
    b = Both(pam, ctx, 8)
    b.policy(LIFO)                         # rebuild reverses: [0, 1, ..., 7]
    assert b.add(1, 8) == [7, 6]
    assert b.add(2, 4) == [5]
    b.free(1)                              # append 7, then 6: [0, 1, 2, 3, 4, 7, 6]
    assert b.add(3, 12) == [6, 7, 4]
    b.free(2)                              # [0, 1, 2, 3, 5]
    assert b.add(4, 8) == [5, 3]
    b.close()


def test_policy_switch_reverses_the_free_list(pam, ctx):
    b = Both(pam, ctx, 8)
    assert b.add(1, 8) == [0, 1]           # free [7, 6, 5, 4, 3, 2]
    b.policy(LIFO)                         # [2, 3, 4, 5, 6, 7]
    assert b.add(2, 4) == [7]
    b.policy(FIFO)                         # [6, 5, 4, 3, 2]
    assert b.add(3, 8) == [2, 3]
    b.free(1)                              # FIFO prepend 0, 1: [1, 0, 6, 5, 4]
    b.policy(FIFO)                         # didSet rebuilds on every set: [4, 5, 6, 0, 1]
    assert b.add(4, 8) == [1, 0]
    b.close()


def test_best_fit_prefers_full_blocks_then_nearest(pam, ctx):
    b = Both(pam, ctx, 8)
    assert b.add(1, 6) == [0, 1]           # tail holds 2 of 4
    assert b.add(2, 5) == [2, 3]           # tail holds 1 of 4
    assert b.add(3, 4) == [4]
    b.policy(BEST_FIT)                     # free [7, 6, 5], each sized 4
    b.free(1)                              # append 0 (4), 1 (2)
    b.free(2)                              # append 2 (4), 3 (1)
    # sizes: 7:4 6:4 5:4 0:4 1:2 2:4 3:1 -> delta 0 in deque order, then 1 (delta 2), then 3
    assert b.add(4, 24) == [7, 6, 5, 0, 2, 1]
    assert b.add(5, 4) == [3]
    b.close()


def test_best_fit_rebuild_sorts_by_held_size_descending(pam, ctx):
    b = Both(pam, ctx, 8)
    b.policy(BEST_FIT)                     # [7..0], every size 4
    assert b.add(1, 6) == [7, 6]
    assert b.add(2, 5) == [5, 4]
    assert b.add(3, 7) == [3, 2]           # free [1, 0]
    b.free(1)                              # [1, 0, 7, 6]          7:4 6:2
    b.free(2)                              # [.., 5, 4]            5:4 4:1
    b.free(3)                              # [.., 3, 2]            3:4 2:3
    b.policy(BEST_FIT)                     # sort by size, descending: [1, 0, 7, 5, 3, 2, 6, 4]
    b.policy(FIFO)                         # reverse:                [4, 6, 2, 3, 5, 7, 0, 1]
    # removeLast order exposes the sorted list (ascending would give 4, 6, 2, 1, ...)
    assert b.add(4, 32) == [1, 0, 7, 5, 3, 2, 6, 4]
    b.close()


def stats(b, bytes_per_block_kv):
    from pagedattentionmetal_amd import _lib
    st = _lib.MemoryStats()
    assert b.pam.pam_cache_memory_stats(b.c, C.byref(st)) == 0
    rs = b.ref.stats(bytes_per_block_kv)
    mine = {k: getattr(st, k) for k in rs}
    assert mine["fragmentation_ratio"] == pytest.approx(rs["fragmentation_ratio"], abs=1e-7)
    mine["fragmentation_ratio"] = rs["fragmentation_ratio"]
    assert mine == rs
    return rs


def test_memory_stats_worked_case(pam, ctx):
    # bs 4, head_dim 32, 1 kv head, f32: 4*1*32*4 bytes per block per pool, x2 for K and V
    b = Both(pam, ctx, 8, bs=4, hd=32, hkv=1, dtype=0)
    st = stats(b, 1024)
    assert st["fragmentation_ratio"] == 0.0      # no sequences: 0 / max(0, 1)
    assert b.add(1, 6) == [0, 1]                 # partial tail (6 % 4 = 2)
    assert b.add(2, 8) == [2, 3]                 # full
    assert b.add(3, 0) == []                     # reserved, length 0: not partial
    assert b.add(4, 4, [11]) == [4]              # registers hash 11
    assert b.add(5, 4, [11]) == [4]              # prefix hit: block 4 shared
    st = stats(b, 1024)
    assert st == {
        "total_blocks": 8, "used_blocks": 5, "free_blocks": 3, "active_sequences": 5,
        "total_memory_bytes": 8192, "used_memory_bytes": 5120, "partially_filled_blocks": 1,
        "fragmentation_ratio": pytest.approx(0.2), "prefix_cache_hits": 1, "prefix_cache_entries": 1,
        "shared_blocks": 1,
    }
    b.free(5)                                    # block 4 back to refcount 1: no longer shared
    b.append(2, 1)                               # 9 tokens: a third block, partial
    st = stats(b, 1024)
    assert (st["used_blocks"], st["partially_filled_blocks"], st["shared_blocks"]) == (6, 2, 0)
    assert st["fragmentation_ratio"] == pytest.approx(2 / 4)
    b.close()
    # f16, 2 kv heads, head_dim 64, bs 16: 16*2*64*2*2 bytes per block
    b = Both(pam, ctx, 3, bs=16, hd=64, hkv=2, dtype=1)
    b.add(1, 17)
    st = stats(b, 8192)
    assert (st["total_memory_bytes"], st["used_memory_bytes"]) == (3 * 8192, 2 * 8192)
    b.close()


class BothSched:
    def __init__(self, pam, max_batch, max_seqs=128):
        self.pam = pam
        self.s = pam.pam_scheduler_create(max_batch, max_seqs)
        self.ref = RefScheduler(max_batch, max_seqs)
        self.buf = (C.c_int32 * 256)()

    def add(self, prompt, max_new):
        sid = self.pam.pam_scheduler_add_request(self.s, prompt, max_new)
        assert sid == self.ref.add_request(prompt, max_new)
        return sid

    def step(self):
        n = self.pam.pam_scheduler_step(self.s, self.buf, 256)
        mine = list(self.buf[:n])
        assert mine == self.ref.step()
        return mine

    def do(self, op, sid):
        getattr(self.pam, "pam_scheduler_" + op)(self.s, sid)
        getattr(self.ref, {"mark_decoded": "mark_decoded", "mark_prefilled": "mark_prefilled",
                           "preempt": "preempt", "complete": "complete"}[op])(sid)

    def counts(self):
        mine = tuple(self.pam.pam_scheduler_count(self.s, st) for st in (WAITING, RUNNING, PAUSED, COMPLETED))
        assert mine == tuple(self.ref.count(st) for st in (WAITING, RUNNING, PAUSED, COMPLETED))
        return mine

    def close(self):
        self.pam.pam_scheduler_destroy(self.s)


def test_scheduler_admission_order_and_cap(pam):
    s = BothSched(pam, 3)
    assert [s.add(10, 2) for _ in range(5)] == [0, 1, 2, 3, 4]
    assert s.step() == [0, 1, 2]                 # waiting, capped at maxBatchSize
    assert s.counts() == (2, 3, 0, 0)
    assert s.step() == [3, 4, 0]                 # waiting first, then running by arrival
    s.do("preempt", 1)
    s.do("mark_decoded", 0)
    s.do("mark_decoded", 0)                      # 0 is done: skipped while running
    assert s.step() == [2, 3, 4]                 # running (not done) fill the batch; 1 stays paused
    assert s.counts() == (0, 4, 1, 0)
    s.do("complete", 2)
    s.do("complete", 3)
    assert s.step() == [4, 1]                    # then paused, resumed to running
    assert s.counts() == (0, 3, 0, 2)
    assert s.add(7, 1) == 5
    s.do("preempt", 4)
    assert s.step() == [5, 1, 4]                 # waiting, running, paused
    s.close()


def test_scheduler_memory_pressure_pauses_newest_first(pam, ctx):
    s = BothSched(pam, 4)
    for _ in range(4):
        s.add(10, 5)
    assert s.step() == [0, 1, 2, 3]
    s.do("preempt", 1)
    b = Both(pam, ctx, 8)                        # 8 free blocks, never changed by the call
    n = pam.pam_scheduler_handle_memory_pressure(s.s, 9, b.c, s.buf, 256)
    got = list(s.buf[:n])
    assert got == s.ref.handle_memory_pressure(9, lambda: 8)
    assert got == [3, 2, 0]                      # running by arrival, newest first; 1 was paused
    n = pam.pam_scheduler_handle_memory_pressure(s.s, 8, b.c, s.buf, 256)
    assert n == 0 and s.ref.handle_memory_pressure(8, lambda: 8) == []
    assert s.step() == [0, 1, 2, 3]              # all paused: resume in arrival order
    b.close()
    s.close()
