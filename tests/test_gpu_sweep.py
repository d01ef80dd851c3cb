"""Seeded random parity sweep: decode and prefill over drawn shapes, against the oracle.

The fixed cases in test_gpu_kernels.py pin each code path with a chosen shape;
this sweep draws its shapes from one seeded generator, so that combinations no
one chose get run too: dtype (f32 / f16 / e4m3), group sizes 1 to 16 with head
counts that are not powers of two, head sizes 32 to 256, block sizes from 4 to
128 (non powers of two go to the row kernel), windows, empty and single-token
rows, long contexts, chunks with cached context.  Every row is compared with the
oracle at the contract tolerance, so a kernel that is wrong only for some
combination of shape parameters fails here.
"""
import numpy as np
import pytest

import oracle
from helpers import TOL, make_case, row_rel_err, to_dev, to_host, worst_rows
from test_gpu_kernels import build_fp8, layer

pytestmark = pytest.mark.gpu

HEADS = [(8, 8), (16, 4), (32, 8), (64, 8), (8, 1), (4, 4), (12, 4), (40, 8), (6, 2), (16, 16), (128, 8), (32, 2)]


def _draw_shape(rng, dtype):
    H, hkv = HEADS[rng.integers(len(HEADS))]
    if dtype == 0:
        d = int(rng.choice([32, 64, 80, 96, 128, 256]))
    else:
        d = int(rng.choice([64, 128, 128, 128, 256, 96]))
    bs = int(rng.choice([16, 16, 32, 8, 64, 4, 12, 128]))
    return H, hkv, d, bs


def _decode_cases(n=32, seed=20251):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        dtype = int(rng.choice([0, 1, 1, 2, 2]))
        H, hkv, d, bs = _draw_shape(rng, dtype)
        B = int(rng.integers(1, 13))
        lens = []
        for _ in range(B):
            u = rng.random()
            lens.append(0 if u < 0.06 else 1 if u < 0.12 else int(rng.integers(2, 12000 if u > 0.9 else 3000)))
        window = 0 if rng.random() < 0.7 else int(rng.integers(1, 2000))
        # bound the pools (host draws) and the oracle's work
        scale = min(1.0, 2.5e7 / max(1, sum(lens) * hkv * d), 4e9 / max(1, sum(lens) * H * d))
        lens = [max(min(x, 1), int(x * scale)) for x in lens]
        cases.append((i, B, H, hkv, d, bs, dtype, lens, window))
    return cases


def _prefill_cases(n=28, seed=30251):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        dtype = int(rng.choice([0, 1, 1, 1, 2, 2]))
        H, hkv, d, bs = _draw_shape(rng, dtype)
        if rng.random() < 0.5:  # the dense kernel's shapes
            d, bs = 128, int(rng.choice([8, 16, 32]))
        T = int(rng.integers(1, 600))
        off = 0 if rng.random() < 0.3 else int(rng.integers(1, 3000))
        causal = bool(rng.random() < 0.8)
        window = 0 if rng.random() < 0.75 else int(rng.integers(1, 1500))
        # bound the oracle's work (T x keys x H x d)
        while T > 1 and T * (off + T) * H * d > 6e9:
            T, off = max(1, T // 2), off // 2
        cases.append((i, T, off, H, hkv, d, bs, dtype, causal, window))
    return cases


DECODE_SWEEP = _decode_cases()
PREFILL_SWEEP = _prefill_cases()


@pytest.fixture(scope="module")
def engine():
    from pagedattentionmetal_amd import PagedAttentionEngine
    e = PagedAttentionEngine()
    e.set_graceful_degradation(False)
    return e


def _pools(engine, rng, dtype, k, v, bt, lens, hkv, d, bs):
    if dtype == 2:
        kd, vd, ksd, vsd, kp, vp, ks, vs = build_fp8(engine, rng, k, v, bt, lens, hkv, d, bs)
        return kd, vd, ksd, vsd, kp, vp, ks.view(np.uint16), vs.view(np.uint16)
    return to_dev(k), to_dev(v), None, None, k, v, None, None


@pytest.mark.parametrize("case", DECODE_SWEEP,
                         ids=[f"d{c[0]}-{['f32', 'f16', 'e4m3'][c[6]]}-H{c[2]}x{c[3]}-d{c[4]}-bs{c[5]}-w{c[8]}"
                              for c in DECODE_SWEEP])
def test_decode_sweep(engine, case):
    import torch
    i, B, H, hkv, d, bs, dtype, lens, window = case
    print(f"decode sweep case {case}", flush=True)
    rng = np.random.default_rng(5000 + i)
    q, k, v, bt, lens = make_case(rng, B, H, hkv, d, bs, dtype, lens)
    kd, vd, ksd, vsd, kp, vp, ks, vs = _pools(engine, rng, dtype, k, v, bt, lens, hkv, d, bs)
    out = torch.zeros((B, H, d), dtype=torch.float32 if dtype == 0 else torch.float16, device="cuda")
    engine.decode(to_dev(q), kd, vd, to_dev(bt), to_dev(lens), out, B, bt.shape[1],
                  layer(H, hkv, d, bs, dtype, window), k_scale=ksd, v_scale=vsd)
    ref = oracle.decode(dtype, q, kp, vp, bt, lens, H, window=window, k_scale=ks, v_scale=vs, n_threads=8)
    o = to_host(out)
    err = row_rel_err(o, ref)
    assert err <= TOL[dtype], f"rel err {err:.3e}; worst (row, head, err): {worst_rows(o, ref)}"


@pytest.mark.parametrize("case", PREFILL_SWEEP,
                         ids=[f"p{c[0]}-{['f32', 'f16', 'e4m3'][c[7]]}-T{c[1]}+{c[2]}-H{c[3]}x{c[4]}-d{c[5]}-bs{c[6]}"
                              f"-{'c' if c[8] else 'n'}-w{c[9]}" for c in PREFILL_SWEEP])
def test_prefill_sweep(engine, case):
    import torch
    i, T, off, H, hkv, d, bs, dtype, causal, window = case
    print(f"prefill sweep case {case}", flush=True)
    rng = np.random.default_rng(6000 + i)
    kv_len = off + T
    _, k, v, bt, _ = make_case(rng, 1, H, hkv, d, bs, dtype, [kv_len])
    q = rng.standard_normal((T, H, d)).astype(np.float32 if dtype == 0 else np.float16)
    kd, vd, ksd, vsd, kp, vp, ks, vs = _pools(engine, rng, dtype, k, v, bt, [kv_len], hkv, d, bs)
    out = torch.zeros((T, H, d), dtype=torch.float32 if dtype == 0 else torch.float16, device="cuda")
    engine.prefill(to_dev(q), kd, vd, to_dev(bt[0]), out, T, layer(H, hkv, d, bs, dtype, window), causal=causal,
                   q_offset=off, k_scale=ksd, v_scale=vsd)
    ref = oracle.prefill(dtype, q, kp, vp, bt[0], off, causal=causal, window=window, k_scale=ks, v_scale=vs,
                         n_threads=8)
    o = to_host(out).astype(np.float64)
    fin = np.isfinite(ref).all(axis=-1)
    assert np.isnan(o[~fin]).all(), "rows with no key in range are 0/0"
    err = row_rel_err(o[fin], ref[fin]) if fin.any() else 0.0
    assert err <= TOL[dtype], f"rel err {err:.3e}"
