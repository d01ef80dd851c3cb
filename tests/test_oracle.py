"""Pins the CPU oracle (CPU only).

Each check is chosen so that a plausible slip in the restatement (a dropped
term, a wrong sign or index, a transposed operand) fails it:
  * binary16 conversion: exhaustive against numpy's float16;
  * e4m3 decode table: torch.float8_e4m3fn for every code but 0x7F/0xFF, which
    the reference decodes as +-480 (kernels.metal:553-562) and never produces;
  * quantize: nearest-code brute force, round trips, the reference's special cases;
  * attention: dense fp64 softmax(QK^T)V (the sim's own check,
    Reference/paged_attention_sim.py:204-236), closed forms (L = 1, identical keys),
    invariances (block placement, block size, split-context merge), the
    decode-as-sim reduction and causal-prefill-as-decode.
"""
import math

import numpy as np
import pytest

import oracle
from helpers import dense_attention, make_case


# ---------------------------------------------------------------- binary16

def test_f16_to_f32_exhaustive():
    lib = oracle.lib()
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([lib.pamo_f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(got[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.all(np.isnan(got[~finite & np.isnan(ref)]))


def test_f32_to_f16_matches_numpy():
    lib = oracle.lib()
    rng = np.random.default_rng(0)
    # every half, every midpoint between neighbouring halves (ties) and random floats
    h = np.arange(0x7C00, dtype=np.uint16).view(np.float16).astype(np.float32)
    mids = ((h[:-1].astype(np.float64) + h[1:].astype(np.float64)) / 2).astype(np.float32)
    x = np.concatenate([h, mids, rng.standard_normal(20000).astype(np.float32) * 1000,
                        rng.uniform(-1e-4, 1e-4, 20000).astype(np.float32), [65519.0, 65520.0, 1e-8]]).astype(np.float32)
    x = np.concatenate([x, -x])
    with np.errstate(over="ignore"):  # 65520 rounds to infinity, on purpose
        ref = x.astype(np.float16).view(np.uint16)
    got = np.array([lib.pamo_f32_to_f16(float(v)) for v in x], dtype=np.uint16)
    assert np.array_equal(got, ref)


# ---------------------------------------------------------------- FP8 codec

def test_decode_table_matches_e4m3fn():
    torch = pytest.importorskip("torch")
    codes = np.arange(256, dtype=np.uint8)
    ours = oracle.dequant_fp8(codes, np.float16(1.0)).astype(np.float32)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).to(torch.float32).numpy()
    normal = (codes & 0x7F) != 0x7F
    assert np.array_equal(ours[normal], ref[normal])
    assert ours[0x7F] == 480.0 and ours[0xFF] == -480.0
    assert ours[0x80] == 0.0 and not np.signbit(ours[0x80])  # -0 decodes to +0


def test_dequant_is_two_half_products():
    """(+-scale * m) * 2^e rounded in half twice, e.g. a subnormal result."""
    s = np.float16(1.0009765625)  # 1 + 2^-10
    got = oracle.dequant_fp8(np.array([0x3F, 0x01], np.uint8), s)
    m1 = np.float16(s * np.float16(1.875))  # 0x3F: e=7, m=7
    assert got[0] == m1
    sub = np.float16(np.float16(s * np.float16(0.125)) * np.float16(0.015625))
    assert got[1] == sub


def _all_codes_values():
    codes = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], np.uint8)
    return codes, oracle.dequant_fp8(codes, np.float16(1.0)).astype(np.float64)


def test_quantize_is_nearest_code():
    codes, vals = _all_codes_values()
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(4000) * 50, rng.uniform(-0.05, 0.05, 4000)]).astype(np.float16)
    q = oracle.quantize_fp8(x, np.float16(1.0))
    qv = oracle.dequant_fp8(q, np.float16(1.0)).astype(np.float64)
    xv = np.clip(x.astype(np.float64), -448, 448)
    best = np.abs(xv[:, None] - vals[None, :]).min(axis=1)
    # kernels.metal:580-584: in [7.5 * 2^-9, 2^-6) the subnormal mantissa rounds
    # to 8 and is clamped to 7 instead of becoming the normal code 0x08
    quirk = (np.abs(xv) >= 7.5 * 2.0 ** -9) & (np.abs(xv) < 2.0 ** -6)
    assert quirk.sum() > 0
    assert np.all((q[quirk] & 0x7F) == 0x07)
    assert np.allclose(np.abs(qv - xv)[~quirk], best[~quirk], rtol=0, atol=1e-12)


def test_quantize_round_trip_and_special_cases():
    codes, vals = _all_codes_values()
    back = oracle.quantize_fp8(vals.astype(np.float16), np.float16(1.0))
    expect = codes.copy()
    expect[expect == 0x80] = 0x00  # -0 quantizes to +0
    assert np.array_equal(back, expect)
    one = np.float16(1.0)
    q = lambda v: int(oracle.quantize_fp8(np.array([v], np.float16), one)[0])
    assert q(0.0) == 0 and q(-0.0) == 0
    assert q(464.0) == 0x7E and q(1e4) == 0x7E and q(-1e4) == 0xFE and q(65504.0) == 0x7E
    assert q(0.0155) == 0x07  # subnormal mantissa rounds to 8 and clamps to 7
    assert q(2.0 ** -6) == 0x08
    assert q(0.5 * 2.0 ** -9) == 0x01  # half-way rounds away from zero (MSL round)
    assert q(2.5) == 0x42 and q(2.625) == 0x42 + 1  # 2.5 exact, 2.625 exact


def test_scale_rule():
    assert float(oracle.fp8_scale(0.0, np.float16(0.0))) == 1.0
    assert oracle.fp8_scale(448.0, np.float16(0.0)) == np.float16(1.0)
    # sticky growth: the old scale's range is kept
    assert oracle.fp8_scale(1.0, np.float16(2.0)) == np.float16(2.0)
    assert oracle.fp8_scale(3 * 448.0, np.float16(2.0)) == np.float16(3.0)
    # a block written once with all-zero data gets scale 1 and keeps it for small data
    assert oracle.fp8_scale(0.5, np.float16(1.0)) == np.float16(1.0)
    assert oracle.fp8_scale(100.0, np.float16(0.0)) == np.float16(np.float32(100.0) / np.float32(448.0))


# ---------------------------------------------------------------- append

def test_slot_mapping_enumeration():
    bt = np.array([7, 2, 9, 4], np.int32)
    for bs in (1, 4, 16):
        for pos in range(len(bt) * bs):
            assert oracle.slot(bt, pos, bs) == bt[pos // bs] * bs + pos % bs


def test_append_f32_scatter():
    rng = np.random.default_rng(2)
    nb, bs, hkv, d = 6, 4, 2, 8
    kp = np.zeros((nb, bs, hkv, d), np.float32)
    vp = np.zeros_like(kp)
    bt = np.array([5, 1, 3], np.int32)
    keys = rng.standard_normal((7, hkv, d)).astype(np.float32)
    vals = rng.standard_normal((7, hkv, d)).astype(np.float32)
    oracle.append(0, keys, vals, kp, vp, bt, 3)
    for t in range(7):
        pos = 3 + t
        assert np.array_equal(kp[bt[pos // bs], pos % bs], keys[t])
        assert np.array_equal(vp[bt[pos // bs], pos % bs], vals[t])
    assert kp[0].sum() == 0 and kp[bt[0], :3].sum() == 0  # nothing else written
    with pytest.raises(IndexError):
        oracle.append(0, keys, vals, kp, vp, bt, 8)  # runs past the table


def test_append_fp8_per_block_scales():
    rng = np.random.default_rng(3)
    nb, bs, hkv, d = 4, 4, 2, 8
    kp = np.zeros((nb, bs, hkv, d), np.uint8)
    vp = np.zeros_like(kp)
    ks = np.zeros(nb, np.float16)
    vs = np.zeros(nb, np.float16)
    bt = np.array([2, 0, 3], np.int32)
    k1 = (rng.standard_normal((6, hkv, d)) * 2).astype(np.float16)
    v1 = rng.standard_normal((6, hkv, d)).astype(np.float16)
    oracle.append(2, k1, v1, kp, vp, bt, 0, ks.view(np.uint16), vs.view(np.uint16))
    # block 2 holds tokens 0..3, block 0 tokens 4..5: scale = max|x| over them / 448
    for p, toks in ((2, slice(0, 4)), (0, slice(4, 6))):
        assert ks[p] == np.float16(np.float32(np.abs(k1[toks]).max()) / np.float32(448.0))
        assert vs[p] == np.float16(np.float32(np.abs(v1[toks]).max()) / np.float32(448.0))
    assert ks[3] == 0 and ks[1] == 0  # untouched blocks keep their scale
    old_bytes = kp[2].copy()
    # a small second append into block 0 keeps its scale (sticky) and block 2's bytes
    k2 = (rng.standard_normal((1, hkv, d)) * 0.01).astype(np.float16)
    before = ks[0]
    oracle.append(2, k2, k2, kp, vp, bt, 6, ks.view(np.uint16), vs.view(np.uint16))
    assert ks[0] == before and np.array_equal(kp[2], old_bytes)
    # bytes are the codec applied with the block's scale
    assert np.array_equal(kp[0, 2], oracle.quantize_fp8(k2[0], ks[0]))


# ---------------------------------------------------------------- attention

def sim_main_fixture():
    """The inputs of the sim's own example (Reference/paged_attention_sim.py:141-178):
    numpy's legacy generator seeded with 42, drawn in the same order (q, then the
    K pool, then the V pool), 16 physical blocks of 4 tokens, d = 8, table [3, 7]."""
    rs = np.random.RandomState(42)
    S, bs, d = 8, 4, 8
    q = rs.randn(S, d).astype(np.float32)
    kp = rs.randn(16, bs, d).astype(np.float32)
    vp = rs.randn(16, bs, d).astype(np.float32)
    return q, kp, vp, np.array([3, 7], np.int32), bs


def test_sim_matches_dense_attention_and_histories():
    """The sim's self-check on its own seeded example (:204-236): the paged result
    equals dense softmax(q k^T) v (threshold 1e-5 there; fp64 here), and the m/l
    histories equal the running max and sum after each logical block."""
    q, kp, vp, bt, bs = sim_main_fixture()
    S = q.shape[0]
    out, mh, lh = oracle.sim_forward(q, kp, vp, bt, bs)
    keys = np.concatenate([kp[3], kp[7]]).astype(np.float64)
    vals = np.concatenate([vp[3], vp[7]]).astype(np.float64)
    for i in range(S):
        assert np.allclose(out[i], dense_attention(q[i], keys, vals, 1.0), rtol=1e-12, atol=1e-12)
    scores = q.astype(np.float64) @ keys.T
    for lb in range(2):
        m = scores[:, : (lb + 1) * bs].max(axis=1)
        l = np.exp(scores[:, : (lb + 1) * bs] - m[:, None]).sum(axis=1)
        assert np.allclose(mh[lb], m) and np.allclose(lh[lb], l)


@pytest.mark.parametrize("dtype", [0, 1])
def test_decode_equals_sim_reduction(dtype):
    """Decode of (b, h) = last row of the sim run on L copies of q/sqrt(d)."""
    rng = np.random.default_rng(5 + dtype)
    B, H, hkv, d, bs = 3, 4, 2, 16, 4
    q, k, v, bt, lens = make_case(rng, B, H, hkv, d, bs, dtype, [5, 12, 1])
    out = oracle.decode(dtype, q, k, v, bt, lens, H)
    for b in range(B):
        L = int(lens[b])
        nlb = (L + bs - 1) // bs
        for h in range(H):
            kvh = h // (H // hkv)
            qs = np.tile(q[b, h].astype(np.float32) / np.float32(math.sqrt(d)), (L, 1))
            sim, _, _ = oracle.sim_forward(qs, k[:, :, kvh, :].astype(np.float32), v[:, :, kvh, :].astype(np.float32),
                                           bt[b, :nlb], bs)
            assert np.allclose(out[b, h], sim[L - 1], rtol=1e-6, atol=1e-7)


def test_decode_matches_dense_and_closed_forms():
    rng = np.random.default_rng(7)
    B, H, hkv, d, bs = 4, 8, 2, 32, 8
    q, k, v, bt, lens = make_case(rng, B, H, hkv, d, bs, 0, [1, 9, 30, 64])
    out = oracle.decode(0, q, k, v, bt, lens, H)
    for b in range(B):
        L = int(lens[b])
        tok = np.arange(L)
        for h in range(H):
            kvh = h // (H // hkv)
            keys = k[bt[b, tok // bs], tok % bs, kvh]
            vals = v[bt[b, tok // bs], tok % bs, kvh]
            assert np.allclose(out[b, h], dense_attention(q[b, h], keys, vals, 1 / math.sqrt(d)), rtol=1e-10)
    # L = 1 returns v_0 exactly
    assert np.array_equal(out[0, 0], v[bt[0, 0], 0, 0].astype(np.float64))
    # identical keys: output is the mean of the V rows
    k2 = k.copy()
    k2[:, :, :, :] = k[0, 0, 0]
    o2 = oracle.decode(0, q, k2, v, bt, lens, H)
    tok = np.arange(int(lens[3]))
    assert np.allclose(o2[3, 0], v[bt[3, tok // bs], tok % bs, 0].astype(np.float64).mean(0), rtol=1e-10)


def test_decode_placement_and_block_size_invariance():
    rng = np.random.default_rng(8)
    H, hkv, d = 4, 2, 16
    L = 45
    keys = rng.standard_normal((L, hkv, d)).astype(np.float32)
    vals = rng.standard_normal((L, hkv, d)).astype(np.float32)
    q = rng.standard_normal((1, H, d)).astype(np.float32)
    outs = []
    for bs in (4, 8, 16, 32):
        nlb = (L + bs - 1) // bs
        nb = nlb + 5
        perm = rng.permutation(nb)[:nlb].astype(np.int32)
        kp = rng.standard_normal((nb, bs, hkv, d)).astype(np.float32)  # junk elsewhere
        vp = rng.standard_normal((nb, bs, hkv, d)).astype(np.float32)
        for t in range(L):
            kp[perm[t // bs], t % bs] = keys[t]
            vp[perm[t // bs], t % bs] = vals[t]
        outs.append(oracle.decode(0, q, kp, vp, perm[None, :], np.array([L], np.uint32), H))
    for o in outs[1:]:
        assert np.allclose(o, outs[0], rtol=1e-12, atol=1e-14)


def test_window_equals_suffix_decode():
    rng = np.random.default_rng(9)
    H, hkv, d, bs = 4, 4, 16, 4
    q, k, v, bt, lens = make_case(rng, 1, H, hkv, d, bs, 0, [37])
    W = 10
    out = oracle.decode(0, q, k, v, bt, lens, H, window=W)
    L = 37
    tok = np.arange(L - W, L)
    for h in range(H):
        keys = k[bt[0, tok // bs], tok % bs, h]
        vals = v[bt[0, tok // bs], tok % bs, h]
        assert np.allclose(out[0, h], dense_attention(q[0, h], keys, vals, 1 / math.sqrt(d)), rtol=1e-10)


def test_prefill_rows_are_decodes():
    rng = np.random.default_rng(10)
    H, hkv, d, bs = 4, 2, 16, 4
    off, T = 6, 9
    q, k, v, bt, _ = make_case(rng, 1, H, hkv, d, bs, 0, [off + T])
    qr = rng.standard_normal((T, H, d)).astype(np.float32)
    causal = oracle.prefill(0, qr, k, v, bt[0], off, causal=True)
    full = oracle.prefill(0, qr, k, v, bt[0], off, causal=False)
    for t in range(T):
        one = oracle.decode(0, qr[t][None], k, v, bt, np.array([off + t + 1], np.uint32), H)
        assert np.allclose(causal[t], one[0], rtol=1e-12)
        allk = oracle.decode(0, qr[t][None], k, v, bt, np.array([off + T], np.uint32), H)
        assert np.allclose(full[t], allk[0], rtol=1e-12)


def test_split_context_merge_equals_single_pass():
    rng = np.random.default_rng(11)
    d, L = 16, 50
    q = rng.standard_normal(d)
    keys = rng.standard_normal((L, d))
    vals = rng.standard_normal((L, d))
    s = keys @ q
    for cuts in ([25], [1, 7, 30], [10, 20, 30, 40]):
        bounds = [0] + cuts + [L]
        m, l, o = [], [], []
        for a, b in zip(bounds[:-1], bounds[1:]):
            mp = s[a:b].max()
            e = np.exp(s[a:b] - mp)
            m.append(mp)
            l.append(e.sum())
            o.append(e @ vals[a:b])
        merged = oracle.merge(np.array(m), np.array(l), np.array(o))
        assert np.allclose(merged, dense_attention(q, keys, vals, 1.0), rtol=1e-12)


def test_fp8_decode_uses_dequantised_pool():
    rng = np.random.default_rng(12)
    B, H, hkv, d, bs = 2, 4, 2, 16, 4
    q, k, v, bt, lens = make_case(rng, B, H, hkv, d, bs, 2, [9, 13])
    nb = k.shape[0]
    kp = np.zeros((nb, bs, hkv, d), np.uint8)
    vp = np.zeros_like(kp)
    ks = np.zeros(nb, np.float16)
    vs = np.zeros(nb, np.float16)
    for b in range(B):
        L = int(lens[b])
        tok = np.arange(L)
        oracle.append(2, k[bt[b, tok // bs], tok % bs], v[bt[b, tok // bs], tok % bs], kp, vp, bt[b], 0,
                      ks.view(np.uint16), vs.view(np.uint16))
    out = oracle.decode(2, q, kp, vp, bt, lens, H, k_scale=ks.view(np.uint16), v_scale=vs.view(np.uint16))
    kd = oracle.dequant_pool(kp, ks).astype(np.float32)
    vd = oracle.dequant_pool(vp, vs).astype(np.float32)
    ref = oracle.decode(0, q.astype(np.float32), kd, vd, bt, lens, H)
    assert np.allclose(out, ref, rtol=1e-12, atol=1e-14)


def test_backward_matches_finite_differences():
    """The backward restatement equals central differences of the dense fp64
    forward loss sum(dO * O) in q, k and v (window and GQA included)."""
    rng = np.random.default_rng(17)
    T, H, hkv, d, bs, W = 6, 4, 2, 4, 2, 4
    nb = 5
    bt = np.array([3, 0, 4], np.int32)
    kp = rng.standard_normal((nb, bs, hkv, d))
    vp = rng.standard_normal((nb, bs, hkv, d))
    q = rng.standard_normal((T, H, d))
    go = rng.standard_normal((T, H, d))
    m, l, _ = oracle.forward_stats(q, kp, vp, bt, window=W)
    dq, dk, dv = oracle.backward(q, kp, vp, bt, go, m, l, window=W)

    def loss(q_, kp_, vp_):
        return float((oracle.forward_stats(q_, kp_, vp_, bt, window=W)[2] * go).sum())
    eps = 1e-6
    num_q = np.zeros_like(q)
    for idx in np.ndindex(q.shape):
        a, b = q.copy(), q.copy()
        a[idx] += eps
        b[idx] -= eps
        num_q[idx] = (loss(a, kp, vp) - loss(b, kp, vp)) / (2 * eps)
    assert np.allclose(dq, num_q, atol=1e-7, rtol=1e-6)
    for pool, grad, which in ((kp, dk, "k"), (vp, dv, "v")):
        for j in range(T):
            for g in range(hkv):
                for e in range(d):
                    a, b = pool.copy(), pool.copy()
                    blk, s = bt[j // bs], j % bs
                    a[blk, s, g, e] += eps
                    b[blk, s, g, e] -= eps
                    num = ((loss(q, a, vp) - loss(q, b, vp)) if which == "k" else
                           (loss(q, kp, a) - loss(q, kp, b))) / (2 * eps)
                    assert abs(grad[j, g, e] - num) <= 1e-7 + 1e-6 * abs(num), (which, j, g, e)
    # keys before the window start get no gradient
    assert not dk[:T - W].any() and not dv[:T - W].any()
