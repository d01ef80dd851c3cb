"""Shared test helpers: seeded paged workloads, tolerance checks, device copies."""
from __future__ import annotations

import numpy as np

# tolerances stated by the path's contract: per output row (b, h),
# max|a - ref| / max(max|ref|, 1e-6) <= TOL[dtype]
TOL = {0: 1e-5, 1: 2e-3, 2: 2e-3}


def row_rel_err(out, ref):
    out = np.asarray(out, np.float64).reshape(-1, ref.shape[-1])
    ref = np.asarray(ref, np.float64).reshape(-1, ref.shape[-1])
    # a row without keys is 0/0 = NaN in the reference; NaN must meet NaN
    both = np.isnan(out) & np.isnan(ref)
    diff = np.where(both, 0.0, np.abs(out - ref))
    diff = np.where(np.isnan(diff), np.inf, diff)
    num = diff.max(axis=1)
    den = np.maximum(np.nan_to_num(np.abs(ref), nan=0.0).max(axis=1), 1e-6)
    return float((num / den).max())


def worst_rows(out, ref, rows_of=None, k=5):
    """Indices (of [..., H, d] rows flattened to [N, H]) with the largest relative errors."""
    h, d = ref.shape[-2], ref.shape[-1]
    out = np.asarray(out, np.float64).reshape(-1, h, d)
    ref = np.asarray(ref, np.float64).reshape(-1, h, d)
    e = np.abs(out - ref).max(axis=2) / np.maximum(np.abs(ref).max(axis=2), 1e-6)
    idx = np.argsort(e, axis=None)[::-1][:k]
    return [(int(i // h), int(i % h), float(e.flat[i])) for i in idx]


def np_dtype(dtype):
    return {0: np.float32, 1: np.float16, 2: np.float16}[dtype]


def make_case(rng, B, H, hkv, d, bs, dtype, lens, pool_blocks=None, std=1.0):
    """Random pools/Q, block tables over a shuffled pool, zero padded."""
    lens = np.asarray(lens, np.uint32)
    nblk = (lens.astype(np.int64) + bs - 1) // bs
    max_nb = int(max(1, nblk.max()))
    need = int(nblk.sum())
    nb = pool_blocks or max(need + 3, 8)
    perm = rng.permutation(nb).astype(np.int32)
    bt = np.zeros((B, max_nb), np.int32)
    c = 0
    for b in range(B):
        bt[b, :nblk[b]] = perm[c:c + nblk[b]]
        c += int(nblk[b])
    dt = np_dtype(dtype)
    k = (rng.standard_normal((nb, bs, hkv, d)) * std).astype(dt)
    v = (rng.standard_normal((nb, bs, hkv, d)) * std).astype(dt)
    q = rng.standard_normal((B, H, d)).astype(dt)
    return q, k, v, bt, lens


def dense_attention(q, keys, vals, scale):
    """softmax(q K^T * scale) V in fp64 for one row (the sim's own check, sim:204-236)."""
    s = keys.astype(np.float64) @ q.astype(np.float64) * scale
    s = np.exp(s - s.max())
    return (s[:, None] * vals.astype(np.float64)).sum(0) / s.sum()


def to_dev(a):
    import torch
    a = np.ascontiguousarray(a)
    # torch has no general unsigned 16/32-bit support: move the same bytes as signed
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    elif a.dtype == np.uint32:
        a = a.view(np.int32)
    return torch.from_numpy(a).cuda()


def to_host(t):
    return t.detach().cpu().numpy()
