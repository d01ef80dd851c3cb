"""Multi-layer engine calls and the engine's configuration surface on the GPU.

decodeLayers / prefillLayers / appendLayers (PagedAttentionEngine.swift:1433-1895)
run every layer's Q (or keys / values) over the one shared pool; each layer is
checked against the oracle, and the fused decode (layers of one spec sharing a
launch) against single-layer decodes bit for bit.  The flat overloads
(:713-760, :1012-1046) resolve the window from their argument or
defaultWindowSize, and the prefill's chunk loop gives the unchunked result.
"""
import numpy as np
import pytest

import oracle
from helpers import TOL, make_case, row_rel_err, to_dev, to_host

pytestmark = pytest.mark.gpu


@pytest.fixture()
def engine():
    from pagedattentionmetal_amd import PagedAttentionEngine
    e = PagedAttentionEngine()
    e.set_graceful_degradation(False)
    yield e
    e.close()


def _spec(H, hkv, d, bs, dtype, window=0):
    from pagedattentionmetal_amd import PagedLayerSpec
    return PagedLayerSpec(d, H, hkv, bs, dtype, window)


def _fp8_pools(rng, nb, bs, hkv, d):
    """e4m3 code pools (no 0x7F / 0xFF, which the quantiser never writes) and half scales."""
    mag = rng.integers(0, 0x7F, size=(nb, bs, hkv, d), dtype=np.uint8)
    sign = (rng.random((nb, bs, hkv, d)) < 0.5).astype(np.uint8) << 7
    k = mag | sign
    mag = rng.integers(0, 0x7F, size=(nb, bs, hkv, d), dtype=np.uint8)
    v = mag | ((rng.random((nb, bs, hkv, d)) < 0.5).astype(np.uint8) << 7)
    ks = (rng.uniform(0.002, 0.02, nb)).astype(np.float16).view(np.uint16)
    vs = (rng.uniform(0.002, 0.02, nb)).astype(np.float16).view(np.uint16)
    return k, v, ks, vs


@pytest.mark.parametrize("dtype,n_layers,window", [(1, 3, 0), (1, 6, 0), (1, 4, 700), (2, 3, 0)])
def test_decode_layers_matches_each_layer(engine, dtype, n_layers, window):
    import torch
    rng = np.random.default_rng(900 + 7 * n_layers + dtype)
    H, hkv, d, bs = 32, 8, 128, 16
    lens = [3000, 17, 1200, 1, 4097]
    q0, k, v, bt, lens_u = make_case(rng, len(lens), H, hkv, d, bs, 1, lens)
    ks = vs = None
    if dtype == 2:
        k, v, ks, vs = _fp8_pools(rng, k.shape[0], bs, hkv, d)
    B, nb = len(lens), bt.shape[1]
    kd, vd, btd, ld = to_dev(k), to_dev(v), to_dev(bt), to_dev(lens_u)
    ksd = to_dev(ks) if ks is not None else None
    vsd = to_dev(vs) if vs is not None else None
    qs = [rng.standard_normal((B, H, d)).astype(np.float16) for _ in range(n_layers)]
    outs = [torch.full((B, H, d), 5.0, dtype=torch.float16, device="cuda") for _ in range(n_layers)]
    layers = [_spec(H, hkv, d, bs, dtype) for _ in range(n_layers)]
    engine.decode_layers([to_dev(q) for q in qs], kd, vd, btd, ld, outs, B, nb, layers, window_size=window,
                         k_scale=ksd, v_scale=vsd)
    for i in range(n_layers):
        ref = oracle.decode(dtype, qs[i], k, v, bt, lens_u, H, window=window, k_scale=ks, v_scale=vs, n_threads=8)
        got = to_host(outs[i])
        assert row_rel_err(got.astype(np.float64), ref) <= TOL[dtype], f"layer {i}"
        # the same layer alone (its window in the spec): the same bits
        one = torch.zeros_like(outs[i])
        engine.decode(to_dev(qs[i]), kd, vd, btd, ld, one, B, nb, _spec(H, hkv, d, bs, dtype, window),
                      k_scale=ksd, v_scale=vsd)
        assert np.array_equal(to_host(one).view(np.uint16), got.view(np.uint16)), f"layer {i} differs from decode"


def test_decode_layers_mixed_specs(engine):
    """Layers of different group sizes in one call: the MFMA layers fuse, the MHA
    layer between them runs alone (VALU kernel), each against the oracle."""
    import torch
    rng = np.random.default_rng(77)
    hkv, d, bs = 4, 128, 16
    lens = [500, 2100, 33]
    _, k, v, bt, lens_u = make_case(rng, len(lens), 16, hkv, d, bs, 1, lens)
    B, nb = len(lens), bt.shape[1]
    heads = [16, 16, 4, 16]
    qs = [rng.standard_normal((B, H, d)).astype(np.float16) for H in heads]
    outs = [torch.zeros((B, H, d), dtype=torch.float16, device="cuda") for H in heads]
    layers = [_spec(H, hkv, d, bs, 1) for H in heads]
    engine.decode_layers([to_dev(q) for q in qs], to_dev(k), to_dev(v), to_dev(bt), to_dev(lens_u), outs, B, nb,
                         layers)
    for i, H in enumerate(heads):
        ref = oracle.decode(1, qs[i], k, v, bt, lens_u, H, n_threads=8)
        assert row_rel_err(to_host(outs[i]).astype(np.float64), ref) <= TOL[1], f"layer {i}"


def test_prefill_layers(engine):
    import torch
    rng = np.random.default_rng(31)
    H, hkv, d, bs, T = 32, 8, 128, 16, 300
    _, k, v, bt, _ = make_case(rng, 1, H, hkv, d, bs, 1, [T])
    qs = [rng.standard_normal((T, H, d)).astype(np.float16) for _ in range(3)]
    outs = [torch.zeros((T, H, d), dtype=torch.float16, device="cuda") for _ in range(3)]
    layers = [_spec(H, hkv, d, bs, 1) for _ in range(3)]
    for window in (0, 128):
        engine.prefill_layers([to_dev(q) for q in qs], to_dev(k), to_dev(v), to_dev(bt[0]), outs, T, layers,
                              causal=True, window_size=window)
        for i in range(3):
            ref = oracle.prefill(1, qs[i], k, v, bt[0], 0, causal=True, window=window, n_threads=8)
            got = to_host(outs[i]).astype(np.float64)
            fin = np.isfinite(ref).all(-1)
            assert np.isnan(got[~fin]).all()
            assert row_rel_err(got[fin], ref[fin]) <= TOL[1], f"window {window} layer {i}"


@pytest.mark.parametrize("dtype", [1, 2])
def test_append_layers_equals_appends_in_order(engine, dtype):
    """appendLayers writes every layer at the same positions of the one pool, in
    layer order: pools (and FP8 scales) equal three appendToCache calls."""
    import torch
    rng = np.random.default_rng(61 + dtype)
    hkv, d, bs, nb, T, off = 4, 64, 16, 12, 40, 10
    bt = torch.from_numpy(rng.permutation(nb)[:4].astype(np.int32)).cuda()
    kt = torch.uint8 if dtype == 2 else torch.float16
    pools = [torch.zeros((nb, bs, hkv, d), dtype=kt, device="cuda") for _ in range(4)]
    scales = [torch.zeros(nb, dtype=torch.float16, device="cuda") for _ in range(4)]
    keys = [torch.from_numpy((rng.standard_normal((T, hkv, d)) * (i + 1)).astype(np.float16)).cuda()
            for i in range(3)]
    vals = [torch.from_numpy(rng.standard_normal((T, hkv, d)).astype(np.float16)).cuda() for i in range(3)]
    layers = [_spec(hkv, hkv, d, bs, dtype) for _ in range(3)]
    fp8 = dtype == 2
    engine.append_layers(keys, vals, pools[0], pools[1], bt, off, T, layers,
                         k_scale_buffers=[scales[0]] * 3 if fp8 else None,
                         v_scale_buffers=[scales[1]] * 3 if fp8 else None)
    for i in range(3):
        engine.append_to_cache(keys[i], vals[i], pools[2], pools[3], bt, off, T, layers[i],
                               k_scale=scales[2] if fp8 else None, v_scale=scales[3] if fp8 else None)
    torch.cuda.synchronize()
    view = (lambda t: to_host(t)) if fp8 else (lambda t: to_host(t).view(np.uint16))
    assert np.array_equal(view(pools[0]), view(pools[2]))
    assert np.array_equal(view(pools[1]), view(pools[3]))
    if fp8:
        assert np.array_equal(to_host(scales[0]).view(np.uint16), to_host(scales[2]).view(np.uint16))
        assert np.array_equal(to_host(scales[1]).view(np.uint16), to_host(scales[3]).view(np.uint16))


def test_flat_prefill_chunk_loop_and_windows(engine):
    """prefill(q:...:windowSize:chunkSize:): the chunk loop's result is the
    unchunked prefill; the window comes from the argument or defaultWindowSize."""
    import torch
    rng = np.random.default_rng(12)
    H, hkv, d, bs, T = 32, 8, 128, 16, 1000
    q, k, v, bt, _ = make_case(rng, 1, H, hkv, d, bs, 1, [T])
    q = rng.standard_normal((T, H, d)).astype(np.float16)
    qd, kd, vd, btd = to_dev(q), to_dev(k), to_dev(v), to_dev(bt[0])
    ref = oracle.prefill(1, q, k, v, bt[0], 0, causal=True, n_threads=8)
    out = torch.zeros((T, H, d), dtype=torch.float16, device="cuda")
    engine.prefill_flat(qd, kd, vd, btd, T, d, H, hkv, bs, out, causal=True, chunk_size=256)
    assert engine.last_stats["chunks"] == 4
    assert row_rel_err(to_host(out).astype(np.float64), ref) <= TOL[1]
    # defaultChunkSize applies when the argument is 0
    engine.default_chunk_size = 300
    out2 = torch.zeros_like(out)
    engine.prefill_flat(qd, kd, vd, btd, T, d, H, hkv, bs, out2, causal=True)
    assert engine.last_stats["chunks"] == 4
    assert row_rel_err(to_host(out2).astype(np.float64), ref) <= TOL[1]
    engine.default_chunk_size = 0
    # a window (argument, then defaultWindowSize): one pass, the windowed prefill
    for use_default in (False, True):
        refw = oracle.prefill(1, q, k, v, bt[0], 0, causal=True, window=200, n_threads=8)
        outw = torch.zeros_like(out)
        if use_default:
            engine.default_window_size = 200
            engine.prefill_flat(qd, kd, vd, btd, T, d, H, hkv, bs, outw, causal=True, chunk_size=256)
            engine.default_window_size = 0
        else:
            engine.prefill_flat(qd, kd, vd, btd, T, d, H, hkv, bs, outw, causal=True, window_size=200,
                                chunk_size=256)
        got = to_host(outw).astype(np.float64)
        fin = np.isfinite(refw).all(-1)
        assert np.isnan(got[~fin]).all()
        assert row_rel_err(got[fin], refw[fin]) <= TOL[1]


def test_flat_decode_window(engine):
    import torch
    rng = np.random.default_rng(5)
    H, hkv, d, bs = 32, 8, 128, 16
    q, k, v, bt, lens = make_case(rng, 3, H, hkv, d, bs, 1, [2000, 90, 1500])
    args = (to_dev(q), to_dev(k), to_dev(v), to_dev(bt), to_dev(lens))
    for window, default in ((512, 0), (0, 300), (0, 0)):
        engine.default_window_size = default
        out = torch.zeros((3, H, d), dtype=torch.float16, device="cuda")
        engine.decode_flat(*args, 3, bt.shape[1], d, H, hkv, bs, out, window_size=window)
        w = window or default
        ref = oracle.decode(1, q, k, v, bt, lens, H, window=w, n_threads=8)
        assert row_rel_err(to_host(out).astype(np.float64), ref) <= TOL[1], (window, default)
    engine.default_window_size = 0
