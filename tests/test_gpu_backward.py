"""GPU parity of the backward kernels (backward.hip) against the oracle's fp64
restatement, which is itself pinned by finite differences (test_oracle.py).

Per row (dQ: (row, head); dK/dV: (token, kv head)): max|a - ref| / max|ref| <=
1e-5 (f32) or 2e-3 (f16), the path's tolerances.  The gradient pools are
accumulated into, as the reference's atomic adds do; keys before the window
start stay untouched.
"""
import numpy as np
import pytest

import oracle
from helpers import TOL, row_rel_err, to_dev, to_host

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype,T,H,hkv,d,bs,W", [
    (0, 40, 8, 2, 64, 16, 0),
    (0, 33, 4, 4, 128, 8, 20),     # window: keys 0..12 get no gradient
    (1, 64, 16, 4, 128, 16, 0),
    (1, 50, 8, 8, 64, 16, 0),
    (0, 17, 2, 1, 256, 16, 0),     # d = 256, MQA
    # f16, d = 128: the MFMA kernels (ragged row and key tiles, windows, G = 1..8)
    (1, 300, 32, 4, 128, 16, 0),
    (1, 257, 8, 8, 128, 32, 100),
    (1, 131, 16, 2, 128, 16, 0),
    (1, 96, 64, 8, 128, 16, 45),
    (1, 2100, 4, 4, 128, 1, 0),    # 2100 one-token blocks: the dQ kernel's large block-table form
])
def test_backward_parity(dtype, T, H, hkv, d, bs, W):
    import torch
    from pagedattentionmetal_amd import PagedAttentionEngine, PagedLayerSpec
    eng = PagedAttentionEngine()
    eng.set_graceful_degradation(False)
    rng = np.random.default_rng(300 + T + d)
    io = np.float32 if dtype == 0 else np.float16
    nbl = (T + bs - 1) // bs
    nb = nbl + 3
    bt = rng.permutation(nb)[:nbl].astype(np.int32)
    kp = rng.standard_normal((nb, bs, hkv, d)).astype(io)
    vp = rng.standard_normal((nb, bs, hkv, d)).astype(io)
    q = rng.standard_normal((T, H, d)).astype(io)
    go = rng.standard_normal((T, H, d)).astype(io)
    m, l, _ = oracle.forward_stats(q, kp, vp, bt, window=W)
    dq_r, dk_r, dv_r = oracle.backward(q, kp, vp, bt, go, m, l, window=W)
    init = np.zeros((nb, bs, hkv, d), io) if dtype == 1 else (0.1 * rng.standard_normal((nb, bs, hkv, d))).astype(io)
    dkp, dvp = to_dev(init.copy()), to_dev(init.copy())
    dq = torch.zeros((T, H, d), dtype=torch.float32 if dtype == 0 else torch.float16, device="cuda")
    lay = PagedLayerSpec(d, H, hkv, bs, dtype, W)
    eng.backward(to_dev(q), to_dev(kp), to_dev(vp), to_dev(bt), to_dev(go), to_dev(m.astype(np.float32)),
                 to_dev(l.astype(np.float32)), dq, dkp, dvp, T, lay)
    assert eng.last_stats["operation"] == 7
    assert row_rel_err(to_host(dq), dq_r) <= TOL[dtype]
    j = np.arange(T)
    slots = (bt[j // bs], j % bs)
    base = init[slots].astype(np.float64)
    got_k = to_host(dkp)[slots].astype(np.float64)
    got_v = to_host(dvp)[slots].astype(np.float64)
    ws = max(0, T - W) if W else 0
    assert row_rel_err(got_k[ws:], base[ws:] + dk_r[ws:]) <= TOL[dtype]
    assert row_rel_err(got_v[ws:], base[ws:] + dv_r[ws:]) <= TOL[dtype]
    assert np.array_equal(got_k[:ws], base[:ws]) and np.array_equal(got_v[:ws], base[:ws])
    # blocks the sequence does not use are untouched
    unused = np.setdiff1d(np.arange(nb), bt)
    assert np.array_equal(to_host(dkp)[unused], init[unused])


def test_backward_refuses_fp8(torch_mod=None):
    from pagedattentionmetal_amd import PagedAttentionEngine, PagedAttentionError, PagedLayerSpec
    import torch
    eng = PagedAttentionEngine()
    eng.set_graceful_degradation(False)
    x = torch.zeros(64, device="cuda")
    with pytest.raises(PagedAttentionError, match="f32 or f16"):
        eng.backward(x, x, x, x, x, x, x, x, x, x, 4, PagedLayerSpec(16, 2, 2, 16, 2))
