"""Synthetic workloads for the five configurations the path is measured on.

Every draw comes from one counter-based generator, SplitMix64 (output k of the
generator seeded with S is mix(S + (k + 1) * 0x9E3779B97F4A7C15)), so the data
does not depend on the numpy, torch or ROCm version.  Seed of configuration k is
``0x5EED0000 + k``.  Draws are split into streams of 2^40 outputs, one per
purpose, in the draw order contexts (0) -> block-table permutation (1) -> Q (2)
-> K (3) -> V (4) -> outliers of K (5) and V (6) -> new keys (7) and values (8).
Metadata is drawn on the host here; pool and query contents are drawn on the
device by libpam's ``pam_synth_normal`` (the same generator, one element per
thread), so a multi-GiB pool never passes through host memory.

  c1  B=4 decode, L~U[17,200], MHA 8/8, d=128, bs=16, fp32, 1024-block pool
  c2  B=64 decode, L~U[128,4096], GQA 32/8, fp16, 32768-block shuffled pool,
      sequences 0..31 share a 512-token (32-block) prefix, K/V ~ N(0, 0.5^2)
  c3  mixed step: 8 prefill chunks of 512 tokens after c~U[0,3584] cached tokens
      + 56 decodes with L~U[256,4096], GQA 32/8, fp16
  c4  B=256 decode, L = clamp(round(lognormal(ln 1024, 1)), 16, 8192), GQA 32/8,
      e4m3 KV quantised on append (1% of K/V entries x8), f16 Q
  c5  B=32 decode, L~U[16384,131072], GQA 64/8, fp16, window 4096
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

SEED_BASE = 0x5EED0000


@dataclass
class DecodeWorkload:
    name: str
    batch: int
    num_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    data_type: int            # 0 f32, 1 f16, 2 fp8
    pool_blocks: int
    seq_lens: np.ndarray      # uint32 [B]
    block_tables: np.ndarray  # int32 [B][max_nb], zero padded
    window: int = 0
    kv_std: float = 1.0
    outlier_frac: float = 0.0
    seed: int = 0
    shared_prefix_blocks: int = 0
    extra: dict = field(default_factory=dict)

    @property
    def max_num_blocks(self):
        return self.block_tables.shape[1]

    def kv_bytes(self) -> int:
        """Algorithmic KV bytes of one decode: sum_b min(L_b, W) * Hkv * d * 2 * elem
        (+ 2 half scales per touched block for FP8)."""
        L = self.seq_lens.astype(np.int64)
        eff = np.minimum(L, self.window) if self.window > 0 else L
        eb = {0: 4, 1: 2, 2: 1}[self.data_type]
        total = int(eff.sum()) * self.num_kv_heads * self.head_dim * 2 * eb
        if self.data_type == 2:
            lo = L - eff
            blocks = (L + self.block_size - 1) // self.block_size - lo // self.block_size
            total += int(blocks.sum()) * 2 * 2
        return total


S_CONTEXTS, S_PERM, S_Q, S_K, S_V, S_K_OUTLIERS, S_V_OUTLIERS, S_NEW_K, S_NEW_V = range(9)
_GAMMA = np.uint64(0x9E3779B97F4A7C15)


def splitmix(seed: int, stream: int, idx) -> np.ndarray:
    """SplitMix64 outputs at positions (stream << 40) + idx of the generator seeded with `seed`."""
    k = (np.uint64(stream) << np.uint64(40)) + np.asarray(idx, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed & ((1 << 64) - 1)) + (k + np.uint64(1)) * _GAMMA
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def uniforms(seed: int, stream: int, n: int, start: int = 0) -> np.ndarray:
    """u in [0, 1) from the top 53 bits of outputs start .. start + n - 1."""
    z = splitmix(seed, stream, np.arange(start, start + n, dtype=np.uint64))
    return (z >> np.uint64(11)).astype(np.float64) * 2.0 ** -53


def normals(seed: int, stream: int, n: int, start: int = 0) -> np.ndarray:
    """Standard normals i = start .. start + n - 1 (Box-Muller cosine branch on
    outputs 2i and 2i + 1, binary64), as pam_synth_normal computes them."""
    u = uniforms(seed, stream, 2 * n, 2 * start)
    return np.sqrt(-2.0 * np.log(1.0 - u[0::2])) * np.cos(6.283185307179586 * u[1::2])


class _Draws:
    """Consecutive integer draws from one stream (contexts), in call order."""

    def __init__(self, seed: int, stream: int):
        self.seed, self.stream, self.pos = seed, stream, 0

    def integers(self, lo: int, hi_excl: int, n: int) -> np.ndarray:
        u = uniforms(self.seed, self.stream, n, self.pos)
        self.pos += n
        return lo + np.floor(u * (hi_excl - lo)).astype(np.int64)

    def normals(self, n: int) -> np.ndarray:
        # pairs of outputs from the current (even) position
        self.pos += self.pos & 1
        v = normals(self.seed, self.stream, n, self.pos // 2)
        self.pos += 2 * n
        return v


def permutation(seed: int, n: int) -> np.ndarray:
    """Fisher-Yates over 0..n-1: swap k (k = 0 .. n-2) exchanges i = n-1-k with
    j = floor(u_k (i + 1)), u_k from stream S_PERM."""
    perm = np.arange(n, dtype=np.int64)
    if n < 2:
        return perm
    u = uniforms(seed, S_PERM, n - 1)
    i = np.arange(n - 1, 0, -1)
    j = np.floor(u * (i + 1)).astype(np.int64)
    for a, b in zip(i.tolist(), j.tolist()):
        perm[a], perm[b] = perm[b], perm[a]
    return perm


def _tables(seed, lens, bs, pool_blocks, shared_prefix_blocks=0, sharers=0):
    """Block tables over a shuffled pool; the first `sharers` sequences start with
    the same `shared_prefix_blocks` physical blocks (ref-counted prefix)."""
    perm = permutation(seed, pool_blocks).astype(np.int32)
    nblocks = (lens.astype(np.int64) + bs - 1) // bs
    max_nb = int(max(1, nblocks.max()))
    bt = np.zeros((len(lens), max_nb), np.int32)
    cursor = 0
    prefix = perm[:shared_prefix_blocks]
    cursor += shared_prefix_blocks
    for b, n in enumerate(nblocks):
        start = 0
        if b < sharers:
            bt[b, :shared_prefix_blocks] = prefix
            start = shared_prefix_blocks
        take = int(n) - start
        if cursor + take > pool_blocks:
            raise ValueError("pool too small for workload")
        bt[b, start:n] = perm[cursor:cursor + take]
        cursor += take
    return bt


def config(k: int, batch_scale: float = 1.0) -> DecodeWorkload:
    """Decode workloads c1, c2, c4, c5 (c3 is `mixed_config`)."""
    seed = SEED_BASE + k
    rng = _Draws(seed, S_CONTEXTS)
    if k == 1:
        B = 4
        lens = rng.integers(17, 201, B).astype(np.uint32)
        bt = _tables(seed, lens, 16, 1024)
        return DecodeWorkload("c1", B, 8, 8, 128, 16, 0, 1024, lens, bt, seed=SEED_BASE + k)
    if k == 2:
        B = max(2, int(64 * batch_scale))
        sharers = B // 2
        lens = rng.integers(128, 4097, B).astype(np.int64)
        lens[:sharers] = rng.integers(513, 4097, sharers)
        lens = lens.astype(np.uint32)
        bt = _tables(seed, lens, 16, 32768, shared_prefix_blocks=32, sharers=sharers)
        return DecodeWorkload("c2", B, 32, 8, 128, 16, 1, 32768, lens, bt, kv_std=0.5, seed=SEED_BASE + k,
                              shared_prefix_blocks=32, extra={"sharers": sharers})
    if k == 4:
        B = max(2, int(256 * batch_scale))
        lens = np.clip(np.round(np.exp(np.log(1024.0) + rng.normals(B))), 16, 8192).astype(np.uint32)
        need = int(((lens.astype(np.int64) + 15) // 16).sum())
        pool = max(need + 64, 1024)
        bt = _tables(seed, lens, 16, pool)
        return DecodeWorkload("c4", B, 32, 8, 128, 16, 2, pool, lens, bt, outlier_frac=0.01, seed=SEED_BASE + k)
    if k == 5:
        B = max(2, int(32 * batch_scale))
        lens = rng.integers(16384, 131073, B).astype(np.uint32)
        need = int(((lens.astype(np.int64) + 15) // 16).sum())
        bt = _tables(seed, lens, 16, need + 64)
        return DecodeWorkload("c5", B, 64, 8, 128, 16, 1, need + 64, lens, bt, window=4096, seed=SEED_BASE + k)
    raise ValueError(f"no decode workload c{k}")


@dataclass
class MixedWorkload:
    name: str
    num_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    context_lens: np.ndarray  # int32 [S]: cached tokens before the step
    query_lens: np.ndarray    # int32 [S]: new tokens this step (1 = decode)
    block_tables: np.ndarray  # int32 [S][max_nb] covering context + new tokens
    pool_blocks: int
    seed: int

    @property
    def total_rows(self):
        return int(self.query_lens.sum())

    def prefill_flops(self) -> int:
        """4 * d * H * sum over chunk rows of (c + i + 1), unmasked pairs only."""
        f = 0
        for c, t in zip(self.context_lens, self.query_lens):
            if t > 1:
                f += int(t) * int(c) + int(t) * (int(t) + 1) // 2
        return 4 * self.head_dim * self.num_heads * f

    def decode_kv_bytes(self) -> int:
        tot = sum(int(c) + 1 for c, t in zip(self.context_lens, self.query_lens) if t == 1)
        return tot * self.num_kv_heads * self.head_dim * 2 * 2


def mixed_config(n_chunks=8, chunk=512, n_decodes=56) -> MixedWorkload:
    seed = SEED_BASE + 3
    rng = _Draws(seed, S_CONTEXTS)
    ctx = np.concatenate([rng.integers(0, 3585, n_chunks), rng.integers(256, 4097, n_decodes) - 1]).astype(np.int32)
    ql = np.concatenate([np.full(n_chunks, chunk), np.ones(n_decodes)]).astype(np.int32)
    total = (ctx.astype(np.int64) + ql)
    need = int(((total + 15) // 16).sum())
    bt = _tables(seed, total.astype(np.uint32), 16, need + 64)
    return MixedWorkload("c3", 32, 8, 128, 16, ctx, ql, bt, need + 64, SEED_BASE + 3)


_synth = None


def device_normals(shape, dtype, seed: int, stream: int, std: float = 1.0, outlier_stream: int = -1,
                   outlier_frac: float = 0.0, device="cuda"):
    """A device tensor of the counter-based normals of (seed, stream) in row-major
    element order, drawn by pam_synth_normal (float32 or float16)."""
    import torch

    from . import api
    global _synth
    if _synth is None:
        _synth = api.PagedAttentionEngine()
    t = torch.empty(shape, dtype=dtype, device=device)
    _synth.synth_normal(t, seed, stream, std, outlier_stream, outlier_frac)
    return t


def device_pools(w: DecodeWorkload, device="cuda"):
    """Q and the K/V pools (f32/f16), or the f16 source values of an FP8 pool."""
    import torch
    shape = (w.pool_blocks, w.block_size, w.num_kv_heads, w.head_dim)
    dt = torch.float32 if w.data_type == 0 else torch.float16
    ko, vo = (S_K_OUTLIERS, S_V_OUTLIERS) if w.outlier_frac > 0 else (-1, -1)
    q = device_normals((w.batch, w.num_heads, w.head_dim), dt, w.seed, S_Q, device=device)
    k = device_normals(shape, dt, w.seed, S_K, w.kv_std, ko, w.outlier_frac, device)
    v = device_normals(shape, dt, w.seed, S_V, w.kv_std, vo, w.outlier_frac, device)
    return q, k, v


def mixed_pools(w: MixedWorkload, device="cuda"):
    """f16 K/V pools (N(0, 0.5^2)), Q (N(0, 1)) and the step's new keys and values
    (N(0, 0.5^2)) of a mixed step."""
    import torch
    shape = (w.pool_blocks, w.block_size, w.num_kv_heads, w.head_dim)
    rows = w.total_rows
    kp = device_normals(shape, torch.float16, w.seed, S_K, 0.5, device=device)
    vp = device_normals(shape, torch.float16, w.seed, S_V, 0.5, device=device)
    q = device_normals((rows, w.num_heads, w.head_dim), torch.float16, w.seed, S_Q, device=device)
    nk = device_normals((rows, w.num_kv_heads, w.head_dim), torch.float16, w.seed, S_NEW_K, 0.5, device=device)
    nv = device_normals((rows, w.num_kv_heads, w.head_dim), torch.float16, w.seed, S_NEW_V, 0.5, device=device)
    return kp, vp, q, nk, nv
