"""The framework-facing cache (adapter.py): the semantics of the reference's MLX
adapter PagedMetalKVCache (PagedMetalKVCache.swift:27-293) for torch tensors.

CPU: the mask policy (makeMask, :178-190).  GPU: a prompt in two chunks and then
single-token steps through ``paged_attention``, each output against dense fp64
softmax attention over the keys and values given so far; shape and mask refusals;
the fallback of ``paged_attention_with_cache_update``.
"""
import numpy as np
import pytest

from helpers import TOL, row_rel_err


def test_make_mask_policy():
    import torch
    from pagedattentionmetal_amd.adapter import make_mask
    assert make_mask(1, 7) == "none"
    assert make_mask(5, 0) == "causal"
    assert make_mask(5, 3, window_size=8) == "causal"
    m = make_mask(3, 2, return_array=True)
    assert m.dtype == torch.bool and tuple(m.shape) == (3, 5)
    # row i is query position offset + i: keys 0 .. offset + i
    assert m.tolist() == [[True, True, True, False, False],
                          [True, True, True, True, False],
                          [True, True, True, True, True]]
    w = make_mask(4, 1, window_size=2)  # n > window: an explicit window mask
    assert w.tolist() == [[True, True, False, False, False],
                          [False, True, True, False, False],
                          [False, False, True, True, False],
                          [False, False, False, True, True]]


def _dense(q, keys, vals, causal_from=None):
    """q [S,H,d], keys/vals [L,Hkv,d] -> [S,H,d] in fp64; row i sees keys
    0 .. causal_from + i when causal_from is given, else all."""
    S, H, d = q.shape
    L, hkv, _ = keys.shape
    G = H // hkv
    out = np.zeros((S, H, d))
    for i in range(S):
        n = L if causal_from is None else causal_from + i + 1
        for h in range(H):
            k = keys[:n, h // G].astype(np.float64)
            v = vals[:n, h // G].astype(np.float64)
            s = k @ q[i, h].astype(np.float64) / np.sqrt(d)
            p = np.exp(s - s.max())
            out[i, h] = (p[:, None] * v).sum(0) / p.sum()
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,H,hkv,d,bs", [(1, 32, 8, 128, 16), (0, 8, 2, 64, 16), (1, 16, 4, 64, 8)])
def test_paged_cache_prompt_chunks_then_decode(dtype, H, hkv, d, bs):
    import torch
    from pagedattentionmetal_amd import PagedLayerSpec
    from pagedattentionmetal_amd.adapter import PagedTorchKVCache
    tdt = torch.float32 if dtype == 0 else torch.float16
    lay = PagedLayerSpec(d, H, hkv, bs, dtype)
    cache = PagedTorchKVCache(3, lay, max_blocks=64)
    rng = np.random.default_rng(11 + dtype + d)
    ks, vs = [], []
    for step, (S, mask) in enumerate([(37, "causal"), (20, "causal"), (1, "none"), (1, "none"), (1, "none")]):
        q = rng.standard_normal((1, H, S, d)).astype(np.float32)
        k = rng.standard_normal((1, hkv, S, d)).astype(np.float32)
        v = rng.standard_normal((1, hkv, S, d)).astype(np.float32)
        before = cache.offset
        out = cache.paged_attention(torch.from_numpy(q).to("cuda", tdt), torch.from_numpy(k).to("cuda", tdt),
                                    torch.from_numpy(v).to("cuda", tdt), mask)
        assert tuple(out.shape) == (1, H, S, d) and cache.offset == before + S
        io = np.float32 if dtype == 0 else np.float16
        ks.append(k[0].transpose(1, 0, 2).astype(io))
        vs.append(v[0].transpose(1, 0, 2).astype(io))
        keys, vals = np.concatenate(ks), np.concatenate(vs)
        qs = q[0].transpose(1, 0, 2).astype(io)
        ref = _dense(qs, keys, vals, causal_from=before if mask == "causal" else None)
        got = out[0].transpose(0, 1).float().cpu().numpy()
        err = row_rel_err(got, ref)
        assert err <= TOL[dtype], f"step {step}: rel err {err:.3e}"
    assert cache.meta_state == ["paged-hip", "3", str(cache.offset), str(bs)]


@pytest.mark.gpu
def test_paged_cache_refusals_and_fallback():
    import torch
    from pagedattentionmetal_amd import PagedLayerSpec
    from pagedattentionmetal_amd.adapter import (PagedTorchKVCache, UnsupportedMask, UnsupportedShape,
                                                 paged_attention_with_cache_update)
    lay = PagedLayerSpec(64, 8, 2, 16, 1)
    cache = PagedTorchKVCache(1, lay, max_blocks=8)
    q = torch.randn((1, 8, 4, 64), device="cuda", dtype=torch.float16)
    k = torch.randn((1, 2, 4, 64), device="cuda", dtype=torch.float16)
    with pytest.raises(UnsupportedShape):
        cache.paged_attention(q.expand(2, -1, -1, -1), k.expand(2, -1, -1, -1), k.expand(2, -1, -1, -1))
    with pytest.raises(UnsupportedShape):
        cache.paged_attention(q, k[:, :1], k[:, :1])
    with pytest.raises(UnsupportedMask):
        cache.paged_attention(q, k, k, torch.ones((4, 4), dtype=torch.bool))
    assert cache.offset == 0  # refused calls append nothing

    calls = []
    def native(*args):
        calls.append(args[5] if not torch.is_tensor(args[5]) else "array")
        return "native"
    # a materialised mask and a foreign scale go to the caller's attention
    assert paged_attention_with_cache_update(q, k, k, cache, 64 ** -0.5, torch.ones((4, 4), dtype=torch.bool),
                                             fallback=native) == "native"
    assert paged_attention_with_cache_update(q, k, k, cache, 0.5, "causal", fallback=native) == "native"
    assert calls == ["array", "causal"] and cache.offset == 0
    out = paged_attention_with_cache_update(q, k, k, cache, 64 ** -0.5, "causal", fallback=native)
    assert torch.is_tensor(out) and cache.offset == 4 and len(calls) == 2


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,H,hkv,d,bs", [(1, 32, 8, 128, 16), (0, 8, 2, 64, 8)])
def test_decode_step_matches_append_then_decode(dtype, H, hkv, d, bs):
    """pam_decode_step (device-resident table and length, patched by the append
    kernel) against pam_append_tokens + pam_append_kv + pam_decode on a twin
    cache: two sequences sharing a hashed prefix whose partial tail block is
    copied on the first step (a full re-stage), then 40 steps each across
    several block boundaries.  Outputs, pools and bookkeeping are identical."""
    import ctypes as C
    import torch
    from pagedattentionmetal_amd import api
    L = api.lib()
    tdt = torch.float32 if dtype == 0 else torch.float16
    rng = np.random.default_rng(99 + dtype)
    P = 2 * bs + bs // 4  # prompt: two full blocks and a partial third
    hashes = (C.c_uint64 * 3)(11, 22, 33)
    prompt_k = torch.from_numpy(rng.standard_normal((P, hkv, d)).astype(np.float32)).to("cuda", tdt)
    prompt_v = torch.from_numpy(rng.standard_normal((P, hkv, d)).astype(np.float32)).to("cuda", tdt)
    steps = [(sid, torch.from_numpy(rng.standard_normal((3, max(H, hkv), d)).astype(np.float32)).to("cuda", tdt))
             for _ in range(40) for sid in (2, 1)]
    res = []
    for use_step in (True, False):
        eng = api.PagedAttentionEngine()
        eng.set_graceful_degradation(False)
        cm = api.KVCacheManager(eng, 64, bs, d, hkv, dtype)
        for sid in (1, 2):
            cm.allocate_sequence(sid)
            assert L.pam_append_tokens_hashed(eng.handle, cm.handle, sid, P, hashes, 3) == 0
        # sequence 2 shares all three blocks of sequence 1 (prefix hits)
        assert cm.get_block_table(1) == cm.get_block_table(2)
        eng._check(L.pam_append_kv(eng.handle, cm.handle, 1, prompt_k.data_ptr(), prompt_v.data_ptr(), 0, P, hkv))
        outs = []
        for sid, x in steps:
            k, v, q = x[0, :hkv].contiguous(), x[1, :hkv].contiguous(), x[2, :H].contiguous()
            out = torch.empty((H, d), dtype=tdt, device="cuda")
            if use_step:
                eng._check(L.pam_decode_step(eng.handle, cm.handle, sid, k.data_ptr(), v.data_ptr(), q.data_ptr(),
                                             out.data_ptr(), H))
            else:
                pos = cm.get_sequence_length(sid)
                cm.append_tokens(sid, 1)
                eng._check(L.pam_append_kv(eng.handle, cm.handle, sid, k.data_ptr(), v.data_ptr(), pos, 1, hkv))
                ids = (C.c_int64 * 1)(sid)
                eng._check(L.pam_decode(eng.handle, cm.handle, ids, 1, q.data_ptr(), out.data_ptr(), H))
            outs.append(out)
        torch.cuda.synchronize()
        res.append(([o.cpu() for o in outs], cm.k_pool().cpu(), cm.v_pool().cpu(), cm.get_block_table(1),
                    cm.get_block_table(2), cm.get_sequence_length(2)))
        L.pam_free_sequence(cm.handle, 1)  # releases the device table
        cm.close()
        eng.close()
    a, b = res
    assert a[3:] == b[3:] and a[5] == P + 40
    assert a[3] != a[4]  # the shared tail was copied on write
    for i, (x, y) in enumerate(zip(a[0], b[0])):
        assert torch.equal(x, y), f"step {i}"
    assert torch.equal(a[1], b[1]) and torch.equal(a[2], b[2])
    assert all(torch.isfinite(o.float()).all() for o in a[0])
