"""GPU tests of the reference's flat C ABI end to end (PagedAttentionCABI.swift:71-372)
and of the engine behaviour around it.

They run on a device cache: pam_reserve_sequence, pam_append_tokens, pam_append_kv,
pam_prefill and pam_decode, all called through ctypes with device pointers, and
checked against the oracle on the cache's own pools.  They also cover
copy-on-write of a shared prefix block in HBM (KVCacheManager.swift:176-214,
FP8 scales included), and graceful degradation and retries
(PagedAttentionEngine.swift:375-418).
"""
import ctypes as C

import numpy as np
import pytest

import oracle
from helpers import TOL, row_rel_err, to_dev, to_host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch
    return torch


def _p(t):
    return C.c_void_p(t.data_ptr())


def _lib():
    from pagedattentionmetal_amd import _lib
    return _lib.load()


@pytest.mark.parametrize("dtype", [0, 1, 2])
def test_cabi_append_prefill_decode_on_device(torch, dtype):
    from pagedattentionmetal_amd import KVCacheManager, PagedAttentionEngine
    lib = _lib()
    eng = PagedAttentionEngine()
    eng.set_graceful_degradation(False)
    hkv, H, d, bs = 4, 16, 128, 16
    cache = KVCacheManager(eng, 64, bs, d, hkv, dtype)
    rng = np.random.default_rng(40 + dtype)
    io = np.float32 if dtype == 0 else np.float16
    tdt = torch.float32 if dtype == 0 else torch.float16
    lens = {7: 100, 9: 37}
    for sid, L in lens.items():
        cache.allocate_sequence(sid)
        cache.append_tokens(sid, L)
        keys = to_dev(rng.standard_normal((L, hkv, d)).astype(io))
        vals = to_dev(rng.standard_normal((L, hkv, d)).astype(io))
        assert lib.pam_append_kv(eng.handle, cache.handle, sid, _p(keys), _p(vals), 0, L, hkv) == 0, \
            lib.pam_last_error(eng.handle)
    torch.cuda.synchronize()
    kh, vh = to_host(cache.k_pool()), to_host(cache.v_pool())
    ks = vs = None
    if dtype == 2:
        ks, vs = to_host(cache.k_scale()).view(np.uint16), to_host(cache.v_scale()).view(np.uint16)

    # pam_prefill: causal attention over the whole sequence 7
    L = lens[7]
    q = rng.standard_normal((L, H, d)).astype(io)
    out = torch.zeros((L, H, d), dtype=tdt, device="cuda")
    assert lib.pam_prefill(eng.handle, cache.handle, 7, _p(to_dev(q)), _p(out), L, H, True) == 0, \
        lib.pam_last_error(eng.handle)
    bt7 = np.array(cache.get_block_table(7), np.int32)
    ref = oracle.prefill(dtype, q, kh, vh, bt7, 0, causal=True, k_scale=ks, v_scale=vs)
    err = row_rel_err(to_host(out), ref)
    assert err <= TOL[dtype], f"pam_prefill rel err {err:.3e}"

    # pam_decode over both sequences (zero-padded batch slab built by the library)
    ids = (C.c_int64 * 2)(9, 7)
    qd = rng.standard_normal((2, H, d)).astype(io)
    outd = torch.zeros((2, H, d), dtype=tdt, device="cuda")
    assert lib.pam_decode(eng.handle, cache.handle, ids, 2, _p(to_dev(qd)), _p(outd), H) == 0, \
        lib.pam_last_error(eng.handle)
    t9, t7 = cache.get_block_table(9), cache.get_block_table(7)
    slab = np.zeros((2, max(len(t9), len(t7))), np.int32)
    slab[0, :len(t9)], slab[1, :len(t7)] = t9, t7
    ref = oracle.decode(dtype, qd, kh, vh, slab, np.array([lens[9], lens[7]], np.uint32), H,
                        k_scale=ks, v_scale=vs)
    err = row_rel_err(to_host(outd), ref)
    assert err <= TOL[dtype], f"pam_decode rel err {err:.3e}"


@pytest.mark.parametrize("dtype", [1, 2])
def test_copy_on_write_copies_block_and_scales_in_hbm(torch, dtype):
    """Two sequences share a prefix block via block hashes; making one exclusive
    gives it a new physical block holding the same bytes (and FP8 scales)."""
    from pagedattentionmetal_amd import KVCacheManager, PagedAttentionEngine
    lib = _lib()
    eng = PagedAttentionEngine()
    eng.set_graceful_degradation(False)
    hkv, d, bs = 2, 64, 16
    cache = KVCacheManager(eng, 16, bs, d, hkv, dtype)
    rng = np.random.default_rng(77)
    cache.allocate_sequence(1)
    cache.append_tokens(1, 20, block_hashes=[0xABC, 0xDEF])
    keys = to_dev(rng.standard_normal((20, hkv, d)).astype(np.float16))
    vals = to_dev(rng.standard_normal((20, hkv, d)).astype(np.float16))
    assert lib.pam_append_kv(eng.handle, cache.handle, 1, _p(keys), _p(vals), 0, 20, hkv) == 0
    cache.allocate_sequence(2)
    cache.append_tokens(2, 16, block_hashes=[0xABC])  # prefix hit on the first block
    t1, t2 = cache.get_block_table(1), cache.get_block_table(2)
    assert t2[0] == t1[0], "prefix block is shared"
    cache.ensure_exclusive_access(2, 0)
    torch.cuda.synchronize()
    t2b = cache.get_block_table(2)
    assert t2b[0] != t1[0], "copy-on-write moved the writer to a new block"
    kh, vh = to_host(cache.k_pool()), to_host(cache.v_pool())
    assert np.array_equal(kh[t2b[0]].view(np.uint8), kh[t1[0]].view(np.uint8))
    assert np.array_equal(vh[t2b[0]].view(np.uint8), vh[t1[0]].view(np.uint8))
    if dtype == 2:
        ks, vs = to_host(cache.k_scale()).view(np.uint16), to_host(cache.v_scale()).view(np.uint16)
        assert ks[t2b[0]] == ks[t1[0]] and vs[t2b[0]] == vs[t1[0]] and ks[t1[0]] != 0


def test_graceful_degradation_and_retries(torch):
    """A failed launch: with graceful degradation on, the call succeeds with a
    zero-filled output; off, it returns the error; a transient failure within the
    retry budget is retried and the result is correct."""
    from pagedattentionmetal_amd import PagedAttentionEngine, PagedAttentionError, PagedLayerSpec
    eng = PagedAttentionEngine()
    rng = np.random.default_rng(3)
    H, hkv, d, bs = 8, 8, 64, 16
    lens = np.array([40, 17], np.uint32)
    nb = 8
    k = rng.standard_normal((nb, bs, hkv, d)).astype(np.float16)
    v = rng.standard_normal((nb, bs, hkv, d)).astype(np.float16)
    q = rng.standard_normal((2, H, d)).astype(np.float16)
    bt = np.array([[0, 1, 2], [3, 4, 0]], np.int32)
    args = (to_dev(q), to_dev(k), to_dev(v), to_dev(bt), to_dev(lens))
    layer = PagedLayerSpec(d, H, hkv, bs, 1)
    ref = oracle.decode(1, q, k, v, bt, lens, H)

    out = torch.full((2, H, d), 7.0, dtype=torch.float16, device="cuda")
    eng.set_graceful_degradation(True)
    eng.set_max_retries(1)
    eng.debug_fail_next_launches(5)
    eng.decode(*args, out, 2, 3, layer)
    assert np.all(to_host(out) == 0), "degraded call zero-fills its output"

    eng.set_graceful_degradation(False)
    eng.debug_fail_next_launches(5)
    with pytest.raises(PagedAttentionError):
        eng.decode(*args, out, 2, 3, layer)

    eng.debug_fail_next_launches(0)
    eng.set_max_retries(3)
    eng.debug_fail_next_launches(2)  # fails twice, the third attempt runs
    eng.decode(*args, out, 2, 3, layer)
    err = row_rel_err(to_host(out), ref)
    assert err <= TOL[1], f"rel err after retries {err:.3e}"


def test_gpu_timing_switch(torch):
    """pam_set_gpu_timing(false): no events, times read -1; the result is unchanged."""
    from pagedattentionmetal_amd import PagedAttentionEngine, PagedLayerSpec
    eng = PagedAttentionEngine()
    eng.set_graceful_degradation(False)
    rng = np.random.default_rng(5)
    H, hkv, d, bs = 32, 8, 128, 16
    lens = np.array([300, 41], np.uint32)
    k = rng.standard_normal((48, bs, hkv, d)).astype(np.float16)
    v = rng.standard_normal((48, bs, hkv, d)).astype(np.float16)
    q = rng.standard_normal((2, H, d)).astype(np.float16)
    bt = rng.permutation(48)[:38].astype(np.int32).reshape(2, 19)
    args = (to_dev(q), to_dev(k), to_dev(v), to_dev(bt), to_dev(lens))
    layer = PagedLayerSpec(d, H, hkv, bs, 1)
    ref = oracle.decode(1, q, k, v, bt, lens, H)
    for timing in (False, True):
        eng.set_gpu_timing(timing)
        out = torch.zeros((2, H, d), dtype=torch.float16, device="cuda")
        eng.decode(*args, out, 2, 19, layer)
        assert row_rel_err(to_host(out), ref) <= TOL[1]
        st = eng.last_stats
        if timing:
            assert st["kernel_ms"] > 0 and st["elapsed_ms"] > 0
        else:
            assert st["kernel_ms"] == -1 and st["elapsed_ms"] == -1


@pytest.mark.parametrize("dtype,H,hkv,d,bs,T,causal,window", [
    (0, 4, 2, 64, 16, 16, False, 0),     # the reference's fusedPrefill test shape (Tests/...:927-1030)
    (0, 8, 8, 32, 16, 40, True, 0),
    (1, 32, 8, 128, 16, 300, True, 0),   # f16, d = 128: dense MFMA prefill kernel
    (1, 32, 8, 128, 16, 200, True, 64),  # fixed window start
    (1, 32, 16, 128, 32, 1000, True, 0),  # one-kernel fused path, items split over workgroups
    (1, 8, 8, 128, 16, 150, False, 0),   # one-kernel fused path, G = 1, full attention
    (1, 16, 4, 64, 8, 77, True, 0),      # d = 64 dense kernel, bs 8
    (1, 32, 8, 64, 16, 300, True, 0),    # d = 64 dense kernel, one-kernel fused path
    (2, 32, 8, 128, 16, 100, True, 0),   # FP8: quantise on append, dequantise in attention
])
def test_fused_prefill_equals_append_then_prefill(torch, dtype, H, hkv, d, bs, T, causal, window):
    """Pool bytes (and FP8 scales) equal a separate append; the output equals a
    separate prefill over that pool, bit for bit, and the oracle within tolerance.
    (f16 with d = 128 also runs as the one kernel that reads the new keys from
    the inputs and writes them into the pools: same bytes and output.)"""
    from pagedattentionmetal_amd import PagedAttentionEngine, PagedLayerSpec
    eng = PagedAttentionEngine()
    eng.set_graceful_degradation(False)
    rng = np.random.default_rng(60 + T + dtype)
    io = np.float32 if dtype == 0 else np.float16
    tdt = torch.float32 if dtype == 0 else torch.float16
    nbl = (T + bs - 1) // bs
    nb = nbl + 5
    bt = rng.permutation(nb)[:nbl].astype(np.int32)
    q = to_dev(rng.standard_normal((T, H, d)).astype(io))
    rk = to_dev(rng.standard_normal((T, hkv, d)).astype(io))
    rv = to_dev(rng.standard_normal((T, hkv, d)).astype(io))
    pdt = torch.uint8 if dtype == 2 else tdt
    layer = PagedLayerSpec(d, H, hkv, bs, dtype, window)
    pools = []
    for _ in range(2):
        kp = torch.zeros((nb, bs, hkv, d), dtype=pdt, device="cuda")
        vp = torch.zeros_like(kp)
        ks = vs = None
        if dtype == 2:
            ks = torch.zeros(nb, dtype=torch.float16, device="cuda")
            vs = torch.zeros_like(ks)
        pools.append((kp, vp, ks, vs))
    btd = to_dev(bt)
    out_f = torch.zeros((T, H, d), dtype=tdt, device="cuda")
    kp, vp, ks, vs = pools[0]
    eng.fused_prefill(q, rk, rv, btd, kp, vp, out_f, T, layer, causal=causal, k_scale=ks, v_scale=vs)
    assert eng.last_stats["operation"] == 1  # reported as prefillSinglePass, as the reference does
    if dtype == 1 and d == 128:
        # the one-kernel form writes the same pool bytes and output
        kp1, vp1 = torch.zeros_like(kp), torch.zeros_like(vp)
        out_1 = torch.zeros_like(out_f)
        eng.set_fused_prefill_one_kernel(True)
        eng.fused_prefill(q, rk, rv, btd, kp1, vp1, out_1, T, layer, causal=causal)
        eng.set_fused_prefill_one_kernel(False)
        torch.cuda.synchronize()
        assert np.array_equal(to_host(kp1).view(np.uint8), to_host(kp).view(np.uint8))
        assert np.array_equal(to_host(vp1).view(np.uint8), to_host(vp).view(np.uint8))
        assert np.array_equal(to_host(out_1).view(np.uint8), to_host(out_f).view(np.uint8)), "one kernel != two"

    out_s = torch.zeros_like(out_f)
    kp2, vp2, ks2, vs2 = pools[1]
    eng.append_to_cache(rk, rv, kp2, vp2, btd, 0, T, layer, k_scale=ks2, v_scale=vs2)
    eng.prefill(q, kp2, vp2, btd, out_s, T, layer, causal=causal, k_scale=ks2, v_scale=vs2)
    torch.cuda.synchronize()
    assert np.array_equal(to_host(kp).view(np.uint8), to_host(kp2).view(np.uint8))
    assert np.array_equal(to_host(vp).view(np.uint8), to_host(vp2).view(np.uint8))
    ksh = vsh = None
    if dtype == 2:
        assert np.array_equal(to_host(ks).view(np.uint16), to_host(ks2).view(np.uint16))
        assert np.array_equal(to_host(vs).view(np.uint16), to_host(vs2).view(np.uint16))
        ksh, vsh = to_host(ks).view(np.uint16), to_host(vs).view(np.uint16)
    got = to_host(out_f)
    assert np.array_equal(got.view(np.uint8), to_host(out_s).view(np.uint8)), "fused != separate"
    ref = oracle.prefill(dtype, to_host(q), to_host(kp), to_host(vp), bt, 0, causal=causal, window=window,
                         k_scale=ksh, v_scale=vsh)
    err = row_rel_err(got, ref)
    assert err <= TOL[dtype], f"rel err {err:.3e}"


def test_stream_switch_orders_work(torch):
    """Two asynchronous decodes that both need split-context partials (the shared
    workspace and stream-K counters), issued by one context on two streams: the
    switch orders the second after the first, so both are correct."""
    from pagedattentionmetal_amd import PagedAttentionEngine, PagedLayerSpec
    from helpers import make_case
    eng = PagedAttentionEngine()
    eng.set_graceful_degradation(False)
    rng = np.random.default_rng(123)
    cases = []
    for lens in ([9000, 7000, 300], [12000, 50]):
        q, k, v, bt, ln = make_case(rng, len(lens), 32, 8, 128, 16, 1, lens)
        cases.append((q, k, v, bt, ln, oracle.decode(1, q, k, v, bt, ln, 32, n_threads=8)))
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    eng.synchronous = False
    outs = []
    try:
        for (q, k, v, bt, ln, _), s in zip(cases, (s1, s2)):
            eng.set_stream(s)
            with torch.cuda.stream(s):
                args = (to_dev(q), to_dev(k), to_dev(v), to_dev(bt), to_dev(ln))
                out = torch.zeros((len(ln), 32, 128), dtype=torch.float16, device="cuda")
            s.synchronize()  # inputs in place; the decodes themselves stay asynchronous
            eng.decode(*args, out, len(ln), bt.shape[1], PagedLayerSpec(128, 32, 8, 16, 1))
            outs.append((out, args))
        torch.cuda.synchronize()
    finally:
        eng.synchronous = True
        eng.set_stream(None)
    for (out, _), case in zip(outs, cases):
        assert row_rel_err(to_host(out), case[5]) <= TOL[1]


def test_calibration_streams(torch):
    """pam_calib_stream_read / pam_calib_stream_copy: each times its stream with
    HIP events (a positive time), and the copy leaves an exact copy."""
    from pagedattentionmetal_amd import PagedAttentionEngine
    eng = PagedAttentionEngine()
    src = torch.randint(-2**31, 2**31 - 1, (16 << 20,), dtype=torch.int32, device="cuda")
    dst = torch.zeros_like(src)
    assert eng.calib_stream_read(src) > 0
    assert eng.calib_stream_copy(src, dst) > 0
    torch.cuda.synchronize()
    assert torch.equal(src, dst)


def test_calibration_mfma_loop(torch):
    """pam_calib_mfma: the MFMA-only loop's rate is positive and no more than the
    part's published dense f16 peak (2.5 PFLOP/s); bad arguments are refused."""
    from pagedattentionmetal_amd import PagedAttentionEngine
    from pagedattentionmetal_amd.api import PagedAttentionError
    eng = PagedAttentionEngine()
    t = eng.calib_mfma(500)
    assert 100.0 < t <= 2500.0, t
    with pytest.raises(PagedAttentionError, match="iters"):
        eng.calib_mfma(0)
