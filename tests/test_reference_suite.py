"""The reference's own test suite, scenario by scenario, against libpam.

Each test below carries the name of one test in
Tests/PagedAttentionMetalTests/PagedAttentionMetalTests.swift (line cited) and
runs the same scenario through this package: the same shapes, dtypes, block
sizes and call sequence, with the same assertions and tolerances.  Where the
reference checks only "no NaN / not all zero", the test here also compares with
the oracle.  The reference fills its pools through shared CPU memory; here the
pools live in HBM and are filled by a device copy of the same
[block][slot][kv head][d] layout.  Inputs are seeded normals or uniforms (the
reference draws Float.random(in: -1...1) unseeded).

Cache-only scenarios run on the CPU against a host-bookkeeping cache; the rest
need a GPU and carry the gpu marker.
"""
import numpy as np
import pytest

import oracle
from helpers import TOL, row_rel_err, to_dev, to_host

OP_PREFILL_SINGLE_PASS, OP_PREFILL_MMA, OP_PREFILL_FLASH, OP_PREFILL_TILED_PASS, OP_DECODE = 1, 2, 3, 4, 5


def _uniform(rng, shape):
    return rng.uniform(-1.0, 1.0, shape).astype(np.float32)


def _cpu_attention(q, k, v, causal):
    """The reference's cpuAttention / inline loops (PagedAttentionMetalTests.swift:36-63,
    125-147) in fp64: q [T][H][d], k/v [T][Hkv][d] -> [T][H][d]."""
    T, H, d = q.shape
    G = H // k.shape[1]
    out = np.zeros((T, H, d))
    for h in range(H):
        kh, vh = k[:, h // G].astype(np.float64), v[:, h // G].astype(np.float64)
        s = q[:, h].astype(np.float64) @ kh.T / np.sqrt(d)
        if causal:
            s = np.where(np.tril(np.ones((T, T), bool)), s, -np.inf)
        p = np.exp(s - s.max(axis=1, keepdims=True))
        out[:, h] = (p / p.sum(axis=1, keepdims=True)) @ vh
    return out


def _engine():
    from pagedattentionmetal_amd import PagedAttentionEngine
    eng = PagedAttentionEngine()
    eng.set_graceful_degradation(False)
    return eng


def _fill_sequence(cache, sid, keys, values):
    """Write token rows [T][Hkv][d] of sequence `sid` into the cache's pools, slot
    by slot through its block table (the reference's kPtr/vPtr loops)."""
    import torch
    bt = cache.get_block_table(sid)
    kp, vp = cache.k_pool(), cache.v_pool()
    bs = cache.block_size
    i = np.arange(keys.shape[0])
    blk = torch.from_numpy(np.asarray(bt, np.int64)[i // bs]).cuda()
    slot = torch.from_numpy(i % bs).cuda()
    kp[blk, slot] = torch.from_numpy(np.ascontiguousarray(keys)).to("cuda", kp.dtype)
    vp[blk, slot] = torch.from_numpy(np.ascontiguousarray(values)).to("cuda", vp.dtype)
    torch.cuda.synchronize()


def _prefill(eng, cache, sid, q, T, layer, causal, out_dtype):
    import torch
    out = torch.zeros((T, layer.num_heads, layer.head_dim), dtype=out_dtype, device="cuda")
    bt = to_dev(np.array(cache.get_block_table(sid), np.int32))
    eng.prefill(to_dev(q), cache.k_pool(), cache.v_pool(), bt, out, T, layer, causal=causal)
    return out


# ----------------------------------------------------------------- GPU scenarios

@pytest.mark.gpu
def test_correctnessVsCPU():
    """PagedAttentionMetalTests.swift:70-114: f32, seqLen 16, headDim 64, one head,
    block 16, non-causal prefill; max |gpu - cpu| < 1e-3."""
    import torch
    from pagedattentionmetal_amd import KVCacheManager, PagedLayerSpec
    eng = _engine()
    rng = np.random.default_rng(70)
    T, d = 16, 64
    q, k, v = (_uniform(rng, (T, 1, d)) for _ in range(3))
    cache = KVCacheManager(eng, 4, 16, d, 1, 0)
    cache.allocate_sequence(1)
    cache.append_tokens(1, T)
    _fill_sequence(cache, 1, k, v)
    out = _prefill(eng, cache, 1, q, T, PagedLayerSpec(d, 1, 1, 16, 0), False, torch.float32)
    assert np.abs(to_host(out) - _cpu_attention(q, k, v, False)).max() < 1e-3


@pytest.mark.gpu
def test_mmaCorrectness():
    """PagedAttentionMetalTests.swift:117-205: the f16 (MMA) prefill against the CPU
    loops, max error < 0.1; then the same inputs in f32.  The reference prints the
    f32 error without a bound; here it must meet the f32 tolerance too."""
    import torch
    from pagedattentionmetal_amd import KVCacheManager, PagedLayerSpec
    eng = _engine()
    rng = np.random.default_rng(117)
    T, d = 16, 64
    q, k, v = (_uniform(rng, (T, 1, d)) for _ in range(3))
    ref = _cpu_attention(q, k, v, False)
    cache = KVCacheManager(eng, 8, 16, d, 1, 1)
    cache.allocate_sequence(1)
    cache.append_tokens(1, T)
    _fill_sequence(cache, 1, k, v)
    out = _prefill(eng, cache, 1, q.astype(np.float16), T, PagedLayerSpec(d, 1, 1, 16, 1), False, torch.float16)
    assert np.abs(to_host(out).astype(np.float64) - ref).max() < 0.1
    assert eng.last_stats["operation"] == OP_PREFILL_MMA

    cache32 = KVCacheManager(eng, 8, 16, d, 1, 0)
    cache32.allocate_sequence(2)
    cache32.append_tokens(2, T)
    _fill_sequence(cache32, 2, k, v)
    out32 = _prefill(eng, cache32, 2, q, T, PagedLayerSpec(d, 1, 1, 16, 0), False, torch.float32)
    assert np.abs(to_host(out32) - ref).max() < 1e-3


@pytest.mark.gpu
def test_causalMasking():
    """PagedAttentionMetalTests.swift:208-253: f32, seqLen 8, headDim 32, causal;
    max error < 1e-3."""
    import torch
    from pagedattentionmetal_amd import KVCacheManager, PagedLayerSpec
    eng = _engine()
    rng = np.random.default_rng(208)
    T, d = 8, 32
    q, k, v = (_uniform(rng, (T, 1, d)) for _ in range(3))
    cache = KVCacheManager(eng, 2, 16, d, 1, 0)
    cache.allocate_sequence(1)
    cache.append_tokens(1, T)
    _fill_sequence(cache, 1, k, v)
    out = _prefill(eng, cache, 1, q, T, PagedLayerSpec(d, 1, 1, 16, 0), True, torch.float32)
    assert np.abs(to_host(out) - _cpu_attention(q, k, v, True)).max() < 1e-3


@pytest.mark.gpu
def test_gqa():
    """PagedAttentionMetalTests.swift:257-303: 8 query heads over 2 KV heads, f32,
    seqLen 16, headDim 64: no NaN, not all zero, |x| < 10; and equal to the CPU
    attention with each query head reading KV head h / 4."""
    import torch
    from pagedattentionmetal_amd import KVCacheManager, PagedLayerSpec
    eng = _engine()
    rng = np.random.default_rng(257)
    T, d, H, hkv = 16, 64, 8, 2
    q = _uniform(rng, (T, H, d))
    k, v = _uniform(rng, (T, hkv, d)), _uniform(rng, (T, hkv, d))
    cache = KVCacheManager(eng, 4, 16, d, hkv, 0)
    cache.allocate_sequence(1)
    cache.append_tokens(1, T)
    _fill_sequence(cache, 1, k, v)
    out = to_host(_prefill(eng, cache, 1, q, T, PagedLayerSpec(d, H, hkv, 16, 0), False, torch.float32))
    assert not np.isnan(out).any()
    assert not np.all(out == 0)
    assert np.all(np.abs(out) < 10)
    assert np.abs(out - _cpu_attention(q, k, v, False)).max() < 1e-3


@pytest.mark.gpu
def test_fp16Performance():
    """PagedAttentionMetalTests.swift:307-396: seqLen 512, headDim 128, 8 heads over
    2 KV heads, 50 prefills each in f32 and f16: f16 within 0.15 of f32 and its
    pools exactly half the bytes.  Times are printed, not asserted, as there."""
    import time

    import torch
    from pagedattentionmetal_amd import KVCacheManager, PagedLayerSpec
    eng = _engine()
    rng = np.random.default_rng(307)
    T, d, H, hkv, bs, iters = 512, 128, 8, 2, 16, 50
    q = _uniform(rng, (T, H, d))
    k, v = _uniform(rng, (T, hkv, d)), _uniform(rng, (T, hkv, d))
    outs, times, pool_bytes = {}, {}, {}
    for dt, tdt in ((0, torch.float32), (1, torch.float16)):
        cache = KVCacheManager(eng, 64, bs, d, hkv, dt)
        cache.allocate_sequence(1)
        cache.append_tokens(1, T)
        _fill_sequence(cache, 1, k, v)
        layer = PagedLayerSpec(d, H, hkv, bs, dt)
        qd = to_dev(q.astype(np.float32 if dt == 0 else np.float16))
        bt = to_dev(np.array(cache.get_block_table(1), np.int32))
        out = torch.zeros((T, H, d), dtype=tdt, device="cuda")
        t0 = time.perf_counter()
        for _ in range(iters):
            eng.prefill(qd, cache.k_pool(), cache.v_pool(), bt, out, T, layer, causal=False)
        times[dt] = (time.perf_counter() - t0) * 1e3 / iters
        outs[dt] = to_host(out).astype(np.float64)
        pool_bytes[dt] = cache.k_pool().nbytes + cache.v_pool().nbytes
    print(f"f32 {times[0]:.3f} ms, f16 {times[1]:.3f} ms per prefill (host clock, synchronous calls)")
    assert np.abs(outs[0] - outs[1]).max() < 0.15
    assert abs(pool_bytes[0] / pool_bytes[1] - 2.0) < 0.01


@pytest.mark.gpu
def test_batchDecode():
    """PagedAttentionMetalTests.swift:400-432: a batch cache of 4 sequences of 32,
    48, 64 and 80 tokens, f32, headDim 64, 4 heads over 2 KV heads, decoded with a
    16-column block-table slab: no NaN, and equal to the oracle over the pools."""
    import torch
    from pagedattentionmetal_amd import KVCacheManager, PagedLayerSpec
    eng = _engine()
    rng = np.random.default_rng(400)
    B, d, H, hkv, bs, lens = 4, 64, 4, 2, 16, [32, 48, 64, 80]
    cache = KVCacheManager(eng, 64, bs, d, hkv, 0)
    for i, L in enumerate(lens):
        cache.allocate_sequence(i)
        cache.append_tokens(i, L)
        _fill_sequence(cache, i, _uniform(rng, (L, hkv, d)), _uniform(rng, (L, hkv, d)))
    bts = torch.zeros((B, 16), dtype=torch.int32, device="cuda")
    sls = torch.zeros((B,), dtype=torch.int32, device="cuda")
    cache.batch_view(list(range(B)), bts, sls, 16)
    q = _uniform(rng, (B, H, d))
    out = torch.zeros((B, H, d), dtype=torch.float32, device="cuda")
    eng.decode(to_dev(q), cache.k_pool(), cache.v_pool(), bts, sls, out, B, 16, PagedLayerSpec(d, H, hkv, bs, 0))
    o = to_host(out)
    assert not np.isnan(o).any()
    assert list(to_host(sls)) == lens
    ref = oracle.decode(0, q, to_host(cache.k_pool()), to_host(cache.v_pool()), to_host(bts),
                        np.array(lens, np.uint32), H)
    assert row_rel_err(o, ref) <= TOL[0]


@pytest.mark.gpu
def test_variableBlockSizes():
    """PagedAttentionMetalTests.swift:436-486: the same f32 prefill (seqLen 32,
    headDim 64, 2 heads) with block sizes 8, 16 and 32.  The reference allows 0.5
    between them; the block size changes only the paging, so here they agree to
    the f32 tolerance."""
    import torch
    from pagedattentionmetal_amd import KVCacheManager, PagedLayerSpec
    eng = _engine()
    rng = np.random.default_rng(436)
    T, d, H = 32, 64, 2
    q, k, v = _uniform(rng, (T, H, d)), _uniform(rng, (T, H, d)), _uniform(rng, (T, H, d))
    outs = []
    for bs in (8, 16, 32):
        cache = KVCacheManager(eng, 8, bs, d, H, 0)
        cache.allocate_sequence(1)
        cache.append_tokens(1, T)
        _fill_sequence(cache, 1, k, v)
        outs.append(to_host(_prefill(eng, cache, 1, q, T, PagedLayerSpec(d, H, H, bs, 0), False, torch.float32)))
    for o in outs[1:]:
        assert np.abs(o - outs[0]).max() < 0.5
        assert row_rel_err(o, outs[0].astype(np.float64)) <= TOL[0]


@pytest.mark.gpu
def test_checkedAPIValidationAndStats():
    """PagedAttentionMetalTests.swift:490-532: a one-float output buffer is refused
    with bufferTooSmall naming "output"; the same call with a full buffer succeeds
    and lastStats reports prefillFlash over sequenceLength 8."""
    import torch
    from pagedattentionmetal_amd import KVCacheManager, PagedAttentionError, PagedLayerSpec
    eng = _engine()
    T, d = 8, 32
    layer = PagedLayerSpec(d, 1, 1, 8, 0)
    cache = KVCacheManager(eng, 4, 8, d, 1, 0)
    cache.allocate_sequence(1)
    cache.append_tokens(1, T)
    q = torch.full((T, 1, d), 0.25, dtype=torch.float32, device="cuda")
    bt = to_dev(np.array(cache.get_block_table(1), np.int32))
    small = torch.zeros((1,), dtype=torch.float32, device="cuda")
    with pytest.raises(PagedAttentionError, match=r"^output buffer is too small"):
        eng.prefill(q, cache.k_pool(), cache.v_pool(), bt, small, T, layer, causal=True)
    out = torch.zeros((T, 1, d), dtype=torch.float32, device="cuda")
    eng.prefill(q, cache.k_pool(), cache.v_pool(), bt, out, T, layer, causal=True)
    st = eng.last_stats
    assert st["operation"] == OP_PREFILL_FLASH
    assert st["sequence_length"] == T


@pytest.mark.gpu
def test_prefillFallsBackToSplitWhenSinglePassThreadgroupIsTooLarge():
    """PagedAttentionMetalTests.swift:535-583: headDim 256, 8 heads over 2 KV heads,
    f32, seqLen 32, K/V appended through appendToCache from the reference's
    patterned inputs, causal prefill: lastStats reports prefillTiledPass; values
    finite and not all zero; and equal to the oracle."""
    import torch
    from pagedattentionmetal_amd import KVCacheManager, PagedLayerSpec
    eng = _engine()
    T = 32
    layer = PagedLayerSpec(256, 8, 2, 16, 0)
    cache = KVCacheManager(eng, 8, 16, 256, 2, 0)
    cache.allocate_sequence(1)
    cache.append_tokens(1, T)
    nq, nkv = T * layer.q_elements_per_token, T * layer.kv_elements_per_token
    q = ((np.arange(nq) % 17 + 1) / 17.0).astype(np.float32).reshape(T, 8, 256)
    k = ((np.arange(nkv) % 11 + 1) / 19.0).astype(np.float32).reshape(T, 2, 256)
    v = ((np.arange(nkv) % 13 + 1) / 23.0).astype(np.float32).reshape(T, 2, 256)
    bt = to_dev(np.array(cache.get_block_table(1), np.int32))
    eng.append_to_cache(to_dev(k), to_dev(v), cache.k_pool(), cache.v_pool(), bt, 0, T, layer)
    out = torch.zeros((T, 8, 256), dtype=torch.float32, device="cuda")
    eng.prefill(to_dev(q), cache.k_pool(), cache.v_pool(), bt, out, T, layer, causal=True)
    assert eng.last_stats["operation"] == OP_PREFILL_TILED_PASS
    o = to_host(out)
    assert np.isfinite(o).all()
    assert not np.all(o == 0)
    ref = oracle.prefill(0, q, to_host(cache.k_pool()), to_host(cache.v_pool()), to_host(bt), 0, causal=True)
    assert row_rel_err(o, ref) <= TOL[0]


@pytest.mark.gpu
def test_mlxSupportCacheConstruction():
    """PagedAttentionMetalTests.swift:608-620: the framework cache for sequence 7
    (headDim 64, 8 heads over 2 KV heads, block 16, f16, 32 blocks) starts at
    offset 0 with all 32 blocks free and keeps its layer."""
    from pagedattentionmetal_amd import PagedLayerSpec
    from pagedattentionmetal_amd.adapter import PagedTorchKVCache
    layer = PagedLayerSpec(64, 8, 2, 16, 1)
    cache = PagedTorchKVCache(7, layer, 32, engine=_engine())
    assert cache.offset == 0
    assert cache.cache_manager.available_blocks == 32
    assert cache.layer == layer


@pytest.mark.gpu
def test_fp8Quantization():
    """PagedAttentionMetalTests.swift:623-711: an f16 prefill (seqLen 16, headDim 64,
    4 heads over 2 KV heads) against the same K/V appended into FP8 pools with
    zeroed per-block scales, through the f16 cache's block table: the FP8 output
    has no NaN and is not all zero (the reference's checks), is within the f16
    tolerance of the oracle over the FP8 pools, and stays close to the f16 output.
    The reference hands the append a head-major copy of K/V; here both caches get
    the same token-major rows, so the two outputs are comparable."""
    import torch
    from pagedattentionmetal_amd import KVCacheManager, PagedLayerSpec
    eng = _engine()
    rng = np.random.default_rng(623)
    T, d, H, hkv, bs = 16, 64, 4, 2, 16
    nb = (T + bs - 1) // bs
    q = _uniform(rng, (T, H, d)).astype(np.float16)
    k = _uniform(rng, (T, hkv, d)).astype(np.float16)
    v = _uniform(rng, (T, hkv, d)).astype(np.float16)
    cache16 = KVCacheManager(eng, nb, bs, d, hkv, 1)
    cache16.allocate_sequence(1)
    cache16.append_tokens(1, T)
    _fill_sequence(cache16, 1, k, v)
    out16 = to_host(_prefill(eng, cache16, 1, q, T, PagedLayerSpec(d, H, hkv, bs, 1), False, torch.float16))

    kp8 = torch.zeros((nb, bs, hkv, d), dtype=torch.uint8, device="cuda")
    vp8 = torch.zeros_like(kp8)
    ks = torch.zeros((nb,), dtype=torch.float16, device="cuda")
    vs = torch.zeros_like(ks)
    bt = to_dev(np.array(cache16.get_block_table(1), np.int32))
    layer8 = PagedLayerSpec(d, hkv, hkv, bs, 2)
    eng.append_to_cache(to_dev(k), to_dev(v), kp8, vp8, bt, 0, T, layer8, k_scale=ks, v_scale=vs)
    out8 = torch.zeros((T, H, d), dtype=torch.float16, device="cuda")
    eng.prefill(to_dev(q), kp8, vp8, bt, out8, T, PagedLayerSpec(d, H, hkv, bs, 2), causal=False,
                k_scale=ks, v_scale=vs)
    o8 = to_host(out8)
    print(f"FP8 max error vs FP16: {np.abs(o8.astype(np.float64) - out16).max():.4f}")
    assert not np.isnan(o8).any()
    assert not np.all(o8 == 0)
    ref = oracle.prefill(2, q, to_host(kp8), to_host(vp8), to_host(bt), 0, causal=False,
                         k_scale=to_host(ks).view(np.uint16), v_scale=to_host(vs).view(np.uint16))
    assert row_rel_err(o8, ref) <= TOL[2]
    assert np.abs(o8.astype(np.float64) - out16.astype(np.float64)).max() < 0.1


@pytest.mark.gpu
def test_emptySequencePrefill():
    """PagedAttentionMetalTests.swift:715-733: a prefill with seqLen 0 either
    returns or raises a library error (the reference accepts both); it does not
    crash, and the engine serves the next call."""
    import torch
    from pagedattentionmetal_amd import KVCacheManager, PagedAttentionError, PagedLayerSpec
    eng = _engine()
    cache = KVCacheManager(eng, 4, 16, 32, 1, 0)
    cache.allocate_sequence(1)
    cache.append_tokens(1, 8)
    layer = PagedLayerSpec(32, 1, 1, 16, 0)
    q = torch.zeros((16,), dtype=torch.float32, device="cuda")
    out = torch.full((16,), 3.0, dtype=torch.float32, device="cuda")
    bt = to_dev(np.array(cache.get_block_table(1), np.int32))
    try:
        eng.prefill(q, cache.k_pool(), cache.v_pool(), bt, out, 0, layer, causal=False)
    except PagedAttentionError as e:
        print(f"empty seq prefill raised: {e}")
    torch.cuda.synchronize()
    assert np.all(to_host(out) == 3.0), "no rows, nothing written"
    rng = np.random.default_rng(715)
    q8 = _uniform(rng, (8, 1, 32))
    k8, v8 = _uniform(rng, (8, 1, 32)), _uniform(rng, (8, 1, 32))
    _fill_sequence(cache, 1, k8, v8)
    o = _prefill(eng, cache, 1, q8, 8, layer, False, torch.float32)
    assert np.abs(to_host(o) - _cpu_attention(q8, k8, v8, False)).max() < 1e-3


@pytest.mark.gpu
def test_batchDecodeEmpty():
    """PagedAttentionMetalTests.swift:774-791: a decode with batchSize 0 either
    returns or raises a library error; no crash, and the engine serves the next
    call."""
    import torch
    from pagedattentionmetal_amd import PagedAttentionError, PagedLayerSpec
    eng = _engine()
    buf = lambda: torch.zeros((16,), dtype=torch.float32, device="cuda")  # noqa: E731
    layer = PagedLayerSpec(32, 1, 1, 16, 0)
    out = torch.full((16,), 3.0, dtype=torch.float32, device="cuda")
    try:
        eng.decode(buf(), buf(), buf(), buf().view(torch.int32), buf().view(torch.int32), out, 0, 1, layer)
    except PagedAttentionError as e:
        print(f"empty batch decode raised: {e}")
    torch.cuda.synchronize()
    assert np.all(to_host(out) == 3.0)
    rng = np.random.default_rng(774)
    k = rng.standard_normal((2, 16, 1, 32)).astype(np.float32)
    v = rng.standard_normal((2, 16, 1, 32)).astype(np.float32)
    q = rng.standard_normal((1, 1, 32)).astype(np.float32)
    bt, sl = np.array([[1, 0]], np.int32), np.array([20], np.uint32)
    o = torch.zeros((1, 1, 32), dtype=torch.float32, device="cuda")
    eng.decode(to_dev(q), to_dev(k), to_dev(v), to_dev(bt), to_dev(sl), o, 1, 2, layer)
    assert row_rel_err(to_host(o), oracle.decode(0, q, k, v, bt, sl, 1)) <= TOL[0]


@pytest.mark.gpu
def test_sequentialAndRepeatedPrefills():
    """PagedAttentionMetalTests.swift:811-871: five cycles on one sequence (f32,
    headDim 32, 2 heads over 1 KV head, block 16), each appending 8 tokens: a
    prefill over the first 8, then a decode with q = 0.5 over the growing
    context (16 .. 40 tokens).  No NaN, length 40, and every result equal to the
    oracle.  The reference's first-cycle q has 8 rows for seqLen 8; the decode
    cycles read the whole block table as one batch row."""
    import torch
    from pagedattentionmetal_amd import KVCacheManager, PagedLayerSpec
    eng = _engine()
    rng = np.random.default_rng(811)
    d, H, hkv, bs = 32, 2, 1, 16
    layer = PagedLayerSpec(d, H, hkv, bs, 0)
    cache = KVCacheManager(eng, 16, bs, d, hkv, 0)
    cache.allocate_sequence(1)
    keys, vals = np.zeros((0, hkv, d), np.float32), np.zeros((0, hkv, d), np.float32)
    for cycle in range(5):
        q = _uniform(rng, (8, H, d))
        keys = np.concatenate([keys, _uniform(rng, (8, hkv, d))])
        vals = np.concatenate([vals, _uniform(rng, (8, hkv, d))])
        cache.append_tokens(1, 8)
        _fill_sequence(cache, 1, keys, vals)
        total = keys.shape[0]
        if cycle == 0:
            o = to_host(_prefill(eng, cache, 1, q, total, layer, False, torch.float32))
            assert not np.isnan(o).any()
            assert np.abs(o - _cpu_attention(q, keys, vals, False)).max() < 1e-3
        else:
            qd = np.full((1, H, d), 0.5, np.float32)
            bt = np.array([cache.get_block_table(1)], np.int32)
            sl = np.array([total], np.uint32)
            o = torch.zeros((1, H, d), dtype=torch.float32, device="cuda")
            eng.decode(to_dev(qd), cache.k_pool(), cache.v_pool(), to_dev(bt), to_dev(sl), o, 1, bt.shape[1], layer)
            o = to_host(o)
            assert not np.isnan(o).any()
            ref = oracle.decode(0, qd, to_host(cache.k_pool()), to_host(cache.v_pool()), bt, sl, H)
            assert row_rel_err(o, ref) <= TOL[0]
    assert cache.get_sequence_length(1) == 40


@pytest.mark.gpu
def test_simultaneousPrefillDecode():
    """PagedAttentionMetalTests.swift:874-923: a 16-token f32 sequence (headDim 32,
    2 heads over 1 KV head): a prefill, then a decode with q = 0.5 over the same
    cache; neither has NaN, and both equal the CPU attention."""
    import torch
    from pagedattentionmetal_amd import KVCacheManager, PagedLayerSpec
    eng = _engine()
    rng = np.random.default_rng(874)
    d, H, hkv, bs = 32, 2, 1, 16
    layer = PagedLayerSpec(d, H, hkv, bs, 0)
    cache = KVCacheManager(eng, 16, bs, d, hkv, 0)
    cache.allocate_sequence(1)
    cache.append_tokens(1, 16)
    k, v = _uniform(rng, (16, hkv, d)), _uniform(rng, (16, hkv, d))
    _fill_sequence(cache, 1, k, v)
    q1 = _uniform(rng, (16, H, d))
    o1 = to_host(_prefill(eng, cache, 1, q1, 16, layer, False, torch.float32))
    q2 = np.full((1, H, d), 0.5, np.float32)
    bt = np.array([cache.get_block_table(1)], np.int32)
    o2 = torch.zeros((1, H, d), dtype=torch.float32, device="cuda")
    eng.decode(to_dev(q2), cache.k_pool(), cache.v_pool(), to_dev(bt), to_dev(np.array([16], np.uint32)), o2, 1,
               bt.shape[1], layer)
    o2 = to_host(o2)
    assert not np.isnan(o1).any() and not np.isnan(o2).any()
    assert np.abs(o1 - _cpu_attention(q1, k, v, False)).max() < 1e-3
    # one query row at the end of the context: the non-causal CPU attention of that row
    assert np.abs(o2[0] - _cpu_attention(q2, k, v, False)[0]).max() < 1e-3


@pytest.mark.gpu
def test_fusedPrefill():
    """PagedAttentionMetalTests.swift:927-1037: fusedPrefill (f32, seqLen 16,
    headDim 64, 4 heads over 2 KV heads) against appending the same rows by hand
    and prefilling: outputs within 1e-3, K and V pools within 1e-6 (here equal)."""
    import torch
    from pagedattentionmetal_amd import KVCacheManager, PagedLayerSpec
    eng = _engine()
    rng = np.random.default_rng(927)
    T, d, H, hkv, bs = 16, 64, 4, 2, 16
    layer = PagedLayerSpec(d, H, hkv, bs, 0)
    q = _uniform(rng, (T, H, d))
    k, v = _uniform(rng, (T, hkv, d)), _uniform(rng, (T, hkv, d))
    fused = KVCacheManager(eng, 1, bs, d, hkv, 0)
    fused.allocate_sequence(1)
    fused.append_tokens(1, T)
    bt_f = to_dev(np.array(fused.get_block_table(1), np.int32))
    out_f = torch.zeros((T, H, d), dtype=torch.float32, device="cuda")
    eng.fused_prefill(to_dev(q), to_dev(k), to_dev(v), bt_f, fused.k_pool(), fused.v_pool(), out_f, T, layer,
                      causal=False)
    sep = KVCacheManager(eng, 1, bs, d, hkv, 0)
    sep.allocate_sequence(1)
    sep.append_tokens(1, T)
    _fill_sequence(sep, 1, k, v)
    out_s = _prefill(eng, sep, 1, q, T, layer, False, torch.float32)
    assert np.abs(to_host(out_f) - to_host(out_s)).max() < 1e-3
    pf, ps = fused.get_block_table(1)[0], sep.get_block_table(1)[0]
    assert np.array_equal(to_host(fused.k_pool())[pf, :T], to_host(sep.k_pool())[ps, :T])
    assert np.array_equal(to_host(fused.v_pool())[pf, :T], to_host(sep.v_pool())[ps, :T])


@pytest.mark.gpu
def test_gpuRecoveryOnTransientError():
    """PagedAttentionMetalTests.swift:1040-1087: with graceful degradation on, a
    prefill (f32, seqLen 8, headDim 32) completes with no NaN; with it off the
    same call completes or raises a library error; then it is switched back on.
    Here the degraded branch is also forced: a launch made to fail returns with a
    zero-filled output instead of an error."""
    import torch
    from pagedattentionmetal_amd import KVCacheManager, PagedAttentionError, PagedLayerSpec
    eng = _engine()
    rng = np.random.default_rng(1040)
    T, d = 8, 32
    layer = PagedLayerSpec(d, 1, 1, 16, 0)
    cache = KVCacheManager(eng, 4, 16, d, 1, 0)
    cache.allocate_sequence(1)
    cache.append_tokens(1, T)
    k, v = _uniform(rng, (T, 1, d)), _uniform(rng, (T, 1, d))
    _fill_sequence(cache, 1, k, v)
    q = np.full((T, 1, d), 0.5, np.float32)
    eng.set_graceful_degradation(True)
    out = to_host(_prefill(eng, cache, 1, q, T, layer, False, torch.float32))
    assert not np.isnan(out).any()
    assert np.abs(out - _cpu_attention(q, k, v, False)).max() < 1e-3
    eng.set_max_retries(1)
    eng.debug_fail_next_launches(5)
    degraded = to_host(_prefill(eng, cache, 1, q, T, layer, False, torch.float32))
    assert np.all(degraded == 0)
    eng.debug_fail_next_launches(0)
    eng.set_graceful_degradation(False)
    try:
        _prefill(eng, cache, 1, q, T, layer, False, torch.float32)
    except PagedAttentionError as e:
        print(f"prefill without degradation raised: {e}")
    eng.set_graceful_degradation(True)


# ----------------------------------------------------------------- cache-only scenarios

def _host_cache(max_blocks, bs, d, hkv, dtype):
    """A cache with block bookkeeping only (no pools): needs no GPU."""
    from pagedattentionmetal_amd import KVCacheManager, PagedAttentionEngine
    return KVCacheManager(PagedAttentionEngine(), max_blocks, bs, d, hkv, dtype, device=False)


def test_cabiLifecycle():
    """PagedAttentionMetalTests.swift:586-605: through the flat C ABI, a cache of 8
    blocks of 4 tokens: reserve 42, append 5 tokens, length 5, 6 blocks free,
    free it, 8 free."""
    from pagedattentionmetal_amd import api
    lib = api.lib()
    ctx = lib.pam_create_context()
    cache = lib.pam_create_cache_host(ctx, 8, 4, 16, 1, 0)
    try:
        assert lib.pam_reserve_sequence(ctx, cache, 42) == 0
        assert lib.pam_append_tokens(ctx, cache, 42, 5) == 0
        assert lib.pam_sequence_length(ctx, cache, 42) == 5
        assert lib.pam_available_blocks(cache) == 6
        lib.pam_free_sequence(cache, 42)
        assert lib.pam_available_blocks(cache) == 8
    finally:
        lib.pam_destroy_cache(cache)
        lib.pam_destroy_context(ctx)


def test_prefillWithZeroBlocks():
    """PagedAttentionMetalTests.swift:736-752: one block of 16: 16 tokens use it up,
    the 17th raises KVCacheError.outOfMemory."""
    from pagedattentionmetal_amd import PagedAttentionError
    cache = _host_cache(1, 16, 32, 1, 0)
    assert cache.available_blocks == 1
    cache.allocate_sequence(1)
    cache.append_tokens(1, 16)
    assert cache.available_blocks == 0
    with pytest.raises(PagedAttentionError, match="outOfMemory"):
        cache.append_tokens(1, 1)


def test_allocateThenImmediateFree():
    """PagedAttentionMetalTests.swift:755-771: allocate, free, and the recycled
    blocks serve the next sequence (2 blocks for 32 tokens)."""
    cache = _host_cache(4, 16, 32, 1, 0)
    assert cache.available_blocks == 4
    cache.allocate_sequence(1)
    cache.append_tokens(1, 16)
    assert cache.available_blocks == 3
    cache.free_sequence(1)
    assert cache.available_blocks == 4
    cache.allocate_sequence(2)
    cache.append_tokens(2, 32)
    assert len(cache.get_block_table(2)) == 2


def test_appendBeyondBlockBoundary():
    """PagedAttentionMetalTests.swift:794-808: 3 * 16 + 7 tokens take 4 blocks; 32
    more take 6, length 87."""
    cache = _host_cache(16, 16, 32, 1, 0)
    cache.allocate_sequence(1)
    cache.append_tokens(1, 16 * 3 + 7)
    assert len(cache.get_block_table(1)) == 4
    assert cache.get_sequence_length(1) == 16 * 3 + 7
    cache.append_tokens(1, 32)
    assert len(cache.get_block_table(1)) == 6
    assert cache.get_sequence_length(1) == 16 * 5 + 7
