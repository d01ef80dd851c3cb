"""Serving-loop driver: the semantics of the reference's PagedAttentionInference
(Sources/PagedAttentionMetal/PagedAttentionInference.swift:119-299) over libpam.

Each ``step()`` takes the scheduler's batch (``ContinuousBatchingScheduler.step``,
Scheduler.swift:78-114) and splits it, as ``step`` does (:119-149), into
newcomers and sequences already prefilled:

* newcomers (``handlePrefill``, :172-219): blocks for the prompt are made
  available (preempting under memory pressure), the sequence is (re)allocated
  and its prompt tokens appended to the cache manager;
* prefilled sequences (``handleDecode``, :221-278): the blocks one more token
  needs are made available, and after the attention each gets one token, is
  marked decoded and is completed (its blocks freed) once done;
* ``ensureBlocksAvailable`` (:280-299): the scheduler's memory-pressure handler
  pauses running sequences, newest first, until enough blocks are free, then
  their blocks are released and they must be prefilled again later.

With one layer, the attention of a step runs as ONE ``mixed_step`` launch
set: the newcomers' prompts as causal prefill chunks and the prefilled
sequences as single-token decode rows, with synthetic new K/V appended at their
positions (the reference issues a prefill per newcomer and then one batched
decode, on uninitialised Q buffers and without writing K/V).

With several layers (``layer`` a list of specs over the one shared pool, the
reference's ``layerSpecs``), the step makes the reference's calls: per
newcomer, its prompt's synthetic K/V appended and ``prefill_layers`` over its
rows (handlePrefill, :172-219); then, for the prefilled sequences, their new
tokens' K/V appended (one slot-mapped append) and one ``decode_layers`` over
the batch (handleDecode, :221-278), every layer with its own Q and output.  Sequences the step
preempts are left out of its launch (the reference would still decode them
from freed blocks).  Q and the new K/V are synthetic: there is no model.

With a sliding window W, a prompt longer than W has one window start,
len - W, for all its rows (the reference's prefill window), so its first
len - W rows attend to no key and come out 0/0 (NaN), as the reference's do.
"""
from __future__ import annotations

import math

import numpy as np

from .api import KVCacheManager, ContinuousBatchingScheduler, PagedAttentionEngine, PagedAttentionError, \
    PagedLayerSpec


class OutOfBlocks(PagedAttentionError):
    """KVCacheError.outOfMemory raised by ensureBlocksAvailable (PagedAttentionInference.swift:295-297)."""


class PagedAttentionInference:
    def __init__(self, engine: PagedAttentionEngine, cache: KVCacheManager, scheduler: ContinuousBatchingScheduler,
                 layer: PagedLayerSpec, attend: bool = True, seed: int = 0):
        """`attend=False` keeps the bookkeeping only (no GPU work), for host tests."""
        self.engine = engine
        self.cache = cache
        self.scheduler = scheduler
        self.layers = list(layer) if isinstance(layer, (list, tuple)) else [layer]
        self.layer = self.layers[0]
        self.attend = attend
        self.prefilled: set[int] = set()
        self.step_count = 0
        self.total_tokens_generated = 0  # prompt tokens prefilled + decoded tokens, as the reference counts
        self.decoded_tokens = 0
        self.prefill_tokens = 0
        self.preemptions = 0
        self._seed = int(seed)
        self._fills = 0  # synthetic-data streams used so far (workloads.device_normals)
        self._buf_rows = 0
        self._max_new: dict[int, int] = {}
        # host mirrors of per-sequence state the step reads every time, kept in
        # step with the library's: the prompt, the scheduler's generated count
        # (changed only by mark_decoded) and the cache's length (the prompt at
        # prefill, one more per decode append)
        self._prompt: dict[int, int] = {}
        self._generated: dict[int, int] = {}
        self._length: dict[int, int] = {}
        self.last_launch = None  # (context lengths, query lengths) of the last mixed_step, rows in that order
        self.attended_pairs = 0  # unmasked (query row, key) pairs per head launched so far

    # --- requests (PagedAttentionInference.swift:100-113)
    def add_request(self, prompt_token_count: int, max_new_tokens: int) -> int:
        """-1 when the scheduler holds max_sequences sequences (Scheduler.swift:59-70)."""
        sid = self.scheduler.add_request(prompt_token_count, max_new_tokens)
        if sid >= 0:
            self._max_new[sid] = max_new_tokens
            self._prompt[sid] = prompt_token_count
            self._generated[sid] = 0
        return sid

    def complete_sequence(self, sid: int):
        self.scheduler.complete_sequence(sid)
        self.cache.free_sequence(sid)
        self.prefilled.discard(sid)
        self._length.pop(sid, None)

    @property
    def waiting_count(self):
        return self.scheduler.waiting_count

    @property
    def running_count(self):
        return self.scheduler.running_count

    @property
    def completed_count(self):
        return self.scheduler.completed_count

    # --- one step (PagedAttentionInference.swift:119-149)
    def step(self):
        batch = self.scheduler.step()
        if not batch:
            return []
        newcomers = [s for s in batch if s not in self.prefilled]
        decoding = [s for s in batch if s in self.prefilled]
        bs = self.cache.block_size
        dropped: set[int] = set()

        prompts = {}
        for sid in newcomers:  # handlePrefill's block work (:172-186)
            prompt = self._prompt[sid]
            dropped |= self._ensure_blocks((prompt + bs - 1) // bs)
            if sid in dropped:  # paused by this or an earlier newcomer's memory pressure: no blocks for it
                continue
            try:
                self.cache.allocate_sequence(sid)
            except PagedAttentionError:
                self.cache.free_sequence(sid)
                self.cache.allocate_sequence(sid)
            self.cache.append_tokens(sid, prompt)
            self._length[sid] = prompt
            prompts[sid] = prompt

        decoding = [s for s in decoding if s not in dropped]
        lens = {sid: self._length[sid] for sid in decoding}
        extras = sum((L + 1 + bs - 1) // bs - (L + bs - 1) // bs for L in lens.values())
        if extras > 0:  # handleDecode (:225-233)
            dropped |= self._ensure_blocks(extras)
        newcomers = [s for s in newcomers if s not in dropped]
        decoding = [s for s in decoding if s not in dropped]
        for sid in decoding:
            self.cache.append_tokens(sid, 1)  # the new token's slot, written by the step
            self._length[sid] += 1

        if self.attend and (newcomers or decoding):
            if len(self.layers) > 1:
                self._launch_layers(newcomers, decoding, prompts, lens)
            else:
                self._launch(newcomers, decoding, prompts, lens)

        for sid in newcomers:  # :205-217
            self.scheduler.mark_prefilled(sid)
            self.prefilled.add(sid)
            self.total_tokens_generated += prompts[sid]
            self.prefill_tokens += prompts[sid]
        for sid in decoding:  # :260-276
            self.scheduler.mark_decoded(sid)
            self._generated[sid] += 1
            self.total_tokens_generated += 1
            self.decoded_tokens += 1
            if self._generated[sid] >= self._max_new[sid]:  # SchedulerSequence.isDone
                self.complete_sequence(sid)
        self.step_count += 1
        return batch

    def run_all(self, max_steps: int = 1 << 30):
        """runAll (:151-157): steps while some sequence is waiting or running, so
        it returns when only paused (preempted) sequences are left, as the
        reference's does."""
        while (self.waiting_count > 0 or self.running_count > 0) and max_steps > 0:
            if not self.step():
                break
            max_steps -= 1

    # --- internals
    def _ensure_blocks(self, needed: int) -> set:
        """ensureBlocksAvailable (:280-299): returns the sequences it preempted."""
        if self.cache.available_blocks >= needed:
            return set()
        victims = self.scheduler.handle_memory_pressure(needed, self.cache)
        for pid in victims:
            self.cache.free_sequence(pid)
            self.prefilled.discard(pid)
        self.preemptions += len(victims)
        if self.cache.available_blocks < needed:
            raise OutOfBlocks(f"{needed} blocks needed, {self.cache.available_blocks} available")
        return set(victims)

    def _pairs(self, ctx, ql) -> int:
        """Unmasked (query row, key) pairs per head of a mixed step: a chunk's rows
        see keys from its one window start max(0, ctx + T - W) up to their own
        position; a decode row sees its last min(L + 1, W) keys."""
        W = self.layer.window_size
        c = np.asarray(ctx, np.int64)
        kv = c + np.asarray(ql, np.int64)
        ws = np.maximum(0, kv - W) if W > 0 else np.zeros_like(kv)
        a, b = np.maximum(0, kv - ws), np.maximum(0, c - ws)
        return int(((a * (a + 1) - b * (b + 1)) // 2).sum())

    def _normals(self, shape, dtype, std):
        """Synthetic Q / K / V rows: the counter-based normals of this driver's seed,
        a fresh stream per buffer (streams from 16 on; the workloads use 0-8)."""
        from . import workloads
        self._fills += 1
        return workloads.device_normals(shape, dtype, self._seed, 15 + self._fills, std)

    def _buffers(self, rows):
        import torch
        L = self.layer
        if rows > self._buf_rows:
            n = max(rows, 2 * self._buf_rows, 4096)
            self._q = self._normals((n, L.num_heads, L.head_dim), torch.float16, 1.0)
            self._out = torch.empty_like(self._q)
            self._nk = self._normals((n, L.num_kv_heads, L.head_dim), torch.float16, 0.5)
            self._nv = self._normals((n, L.num_kv_heads, L.head_dim), torch.float16, 0.5)
            self._buf_rows = n
        return self._q[:rows], self._out[:rows], self._nk[:rows], self._nv[:rows]

    def _launch(self, newcomers, decoding, prompts, lens):
        import torch
        ids = newcomers + decoding
        ctx = np.array([0] * len(newcomers) + [lens[s] for s in decoding], np.int32)
        ql = np.array([prompts[s] for s in newcomers] + [1] * len(decoding), np.int32)
        bs = self.cache.block_size
        width = int(((ctx + ql + bs - 1) // bs).max())
        # batch_view writes every entry (the table zero-padded)
        bt = torch.empty((len(ids), width), dtype=torch.int32, device="cuda")
        sl = torch.empty(len(ids), dtype=torch.int32, device="cuda")
        self.cache.batch_view(ids, bt, sl, width)
        rows = int(ql.sum())
        self.last_launch = (ctx, ql)
        self.attended_pairs += self._pairs(ctx, ql)
        q, out, nk, nv = self._buffers(rows)
        c = self.cache
        self.engine.mixed_step(q, out, c.k_pool(), c.v_pool(), bt, ctx, ql, self.layer, new_keys=nk, new_values=nv,
                               k_scale=c.k_scale(), v_scale=c.v_scale())


    def _layer_buffers(self, rows):
        """Per-layer synthetic Q and outputs (rows x H x d), and the step's new K/V."""
        import torch
        if rows > getattr(self, "_lbuf_rows", 0):
            n = max(rows, 2 * getattr(self, "_lbuf_rows", 0), 1024)
            dt = torch.float32 if self.layer.data_type == 0 else torch.float16
            self._lq = [self._normals((n, l.num_heads, l.head_dim), dt, 1.0) for l in self.layers]
            self._lout = [torch.empty_like(q) for q in self._lq]
            L = self.layer
            self._lk = self._normals((n, L.num_kv_heads, L.head_dim), dt, 0.5)
            self._lv = self._normals((n, L.num_kv_heads, L.head_dim), dt, 0.5)
            self._lbuf_rows = n
        return ([q[:rows] for q in self._lq], [o[:rows] for o in self._lout], self._lk[:rows], self._lv[:rows])

    def _launch_layers(self, newcomers, decoding, prompts, lens):
        """The reference's per-step calls over all layers (PagedAttentionInference.swift:172-278)."""
        import torch
        c, eng, L = self.cache, self.engine, self.layer
        bs = c.block_size
        fp8 = L.data_type == 2
        scales = dict(k_scale=c.k_scale(), v_scale=c.v_scale()) if fp8 else {}
        self.last_launch = None
        for sid in newcomers:  # handlePrefill: one prefillLayers per newcomer
            T = prompts[sid]
            bt = torch.tensor(c.get_block_table(sid), dtype=torch.int32, device="cuda")
            qs, outs, nk, nv = self._layer_buffers(T)
            eng.append_to_cache(nk, nv, c.k_pool(), c.v_pool(), bt, 0, T, L, **scales)
            eng.prefill_layers(qs, c.k_pool(), c.v_pool(), bt, outs, T, self.layers, causal=True, **scales)
            self.attended_pairs += self._pairs(np.array([0]), np.array([T])) * len(self.layers)
        if not decoding:
            return
        # handleDecode: the new tokens' K/V at their positions, then one decodeLayers
        B = len(decoding)
        qs, outs, nk, nv = self._layer_buffers(B)
        if fp8:  # FP8 appends take a block table (per-block scale rule)
            for i, sid in enumerate(decoding):
                bt = torch.tensor(c.get_block_table(sid), dtype=torch.int32, device="cuda")
                eng.append_to_cache(nk[i:i + 1], nv[i:i + 1], c.k_pool(), c.v_pool(), bt, lens[sid], 1, L, **scales)
        else:
            slots = []
            for sid in decoding:
                t = c.get_block_table(sid)
                pos = lens[sid]
                slots.append(t[pos // bs] * bs + pos % bs)
            sm = torch.tensor(slots, dtype=torch.int64, device="cuda")
            eng.append_to_cache(nk, nv, c.k_pool(), c.v_pool(), None, 0, B, L, slot_mapping=sm)
        width = max((lens[s] + 1 + bs - 1) // bs for s in decoding)
        bt = torch.empty((B, width), dtype=torch.int32, device="cuda")  # batch_view writes every entry
        sl = torch.empty(B, dtype=torch.int32, device="cuda")
        c.batch_view(decoding, bt, sl, width)
        eng.decode_layers(qs, c.k_pool(), c.v_pool(), bt, sl, outs, B, width, self.layers, **scales)
        ctx = np.array([lens[s] for s in decoding], np.int32)
        self.attended_pairs += self._pairs(ctx, np.ones(B, np.int32)) * len(self.layers)
        self.last_launch = (ctx, np.ones(B, np.int32))


def poisson_trace(inference: PagedAttentionInference, steps: int, rate: float, prompt_range, output_range,
                  seed: int, on_step=None):
    """The BASELINE c5 driver: `steps` scheduler steps with Poisson(`rate`) arrivals
    before each, prompts and output lengths uniform over the given inclusive
    ranges.  Returns the number of requests admitted.  Draws: SplitMix64 stream 0
    of `seed` (workloads.uniforms), one uniform per step for its arrival count
    (Poisson by inversion), then two per arrival for its prompt and output length."""
    from .workloads import uniforms
    admitted = 0
    pos = 0

    block = np.zeros(0)

    def draw():  # output pos of the stream, generated 4096 at a time
        nonlocal pos, block
        if pos % 4096 == 0:
            block = uniforms(seed, 0, 4096, pos)
        pos += 1
        return float(block[(pos - 1) % 4096])

    def poisson():
        u, k = draw(), 0
        p = math.exp(-rate)
        F = p
        while u > F and k < 10_000:
            k += 1
            p *= rate / k
            F += p
        return k

    for i in range(steps):
        for _ in range(poisson()):
            prompt = prompt_range[0] + int(draw() * (prompt_range[1] - prompt_range[0] + 1))
            out = output_range[0] + int(draw() * (output_range[1] - output_range[0] + 1))
            if inference.add_request(prompt, out) >= 0:
                admitted += 1
        inference.step()
        if on_step is not None:
            on_step(i)
    return admitted
