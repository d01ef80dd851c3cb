"""Synthetic workloads for the five configurations the path is measured on.

Metadata (context lengths, block tables, chunk layouts) comes from a seeded
numpy generator; pool and query contents are drawn on the device with a seeded
torch generator, so a multi-GiB pool never passes through host memory.  Seed of
configuration k is ``0x5EED0000 + k``.

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


def _tables(rng, lens, bs, pool_blocks, shared_prefix_blocks=0, sharers=0):
    """Block tables over a shuffled pool; the first `sharers` sequences start with
    the same `shared_prefix_blocks` physical blocks (ref-counted prefix)."""
    perm = rng.permutation(pool_blocks).astype(np.int32)
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
    rng = np.random.default_rng(SEED_BASE + k)
    if k == 1:
        B = 4
        lens = rng.integers(17, 201, B).astype(np.uint32)
        bt = _tables(rng, lens, 16, 1024)
        return DecodeWorkload("c1", B, 8, 8, 128, 16, 0, 1024, lens, bt, seed=SEED_BASE + k)
    if k == 2:
        B = max(2, int(64 * batch_scale))
        sharers = B // 2
        lens = rng.integers(128, 4097, B).astype(np.int64)
        lens[:sharers] = rng.integers(513, 4097, sharers)
        lens = lens.astype(np.uint32)
        bt = _tables(rng, lens, 16, 32768, shared_prefix_blocks=32, sharers=sharers)
        return DecodeWorkload("c2", B, 32, 8, 128, 16, 1, 32768, lens, bt, kv_std=0.5, seed=SEED_BASE + k,
                              shared_prefix_blocks=32, extra={"sharers": sharers})
    if k == 4:
        B = max(2, int(256 * batch_scale))
        lens = np.clip(np.round(np.exp(rng.normal(np.log(1024.0), 1.0, B))), 16, 8192).astype(np.uint32)
        need = int(((lens.astype(np.int64) + 15) // 16).sum())
        pool = max(need + 64, 1024)
        bt = _tables(rng, lens, 16, pool)
        return DecodeWorkload("c4", B, 32, 8, 128, 16, 2, pool, lens, bt, outlier_frac=0.01, seed=SEED_BASE + k)
    if k == 5:
        B = max(2, int(32 * batch_scale))
        lens = rng.integers(16384, 131073, B).astype(np.uint32)
        need = int(((lens.astype(np.int64) + 15) // 16).sum())
        bt = _tables(rng, lens, 16, need + 64)
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
    rng = np.random.default_rng(SEED_BASE + 3)
    ctx = np.concatenate([rng.integers(0, 3585, n_chunks), rng.integers(256, 4097, n_decodes) - 1]).astype(np.int32)
    ql = np.concatenate([np.full(n_chunks, chunk), np.ones(n_decodes)]).astype(np.int32)
    total = (ctx.astype(np.int64) + ql)
    need = int(((total + 15) // 16).sum())
    bt = _tables(rng, total.astype(np.uint32), 16, need + 64)
    return MixedWorkload("c3", 32, 8, 128, 16, ctx, ql, bt, need + 64, SEED_BASE + 3)


def device_pools(w: DecodeWorkload, device="cuda"):
    """K/V pools (f32/f16) or the f16 source values for an FP8 pool, drawn on the device."""
    import torch
    g = torch.Generator(device=device)
    g.manual_seed(w.seed)
    shape = (w.pool_blocks, w.block_size, w.num_kv_heads, w.head_dim)
    dt = torch.float32 if w.data_type == 0 else torch.float16
    k = torch.randn(shape, generator=g, device=device, dtype=torch.float32).mul_(w.kv_std)
    v = torch.randn(shape, generator=g, device=device, dtype=torch.float32).mul_(w.kv_std)
    if w.outlier_frac > 0:
        for t in (k, v):
            m = torch.rand(shape, generator=g, device=device) < w.outlier_frac
            t[m] *= 8.0
    q = torch.randn((w.batch, w.num_heads, w.head_dim), generator=g, device=device, dtype=torch.float32)
    return q.to(dt), k.to(dt), v.to(dt)
