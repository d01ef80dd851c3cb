"""Code-object loading and launch (the reference's pipeline manager,
PagedAttentionEngine.swift:151-198, 248-333): an engine bound to
libpam_kernels.hsaco launches decode, decodeLayers, prefill and the mixed step
through hipModuleLaunchKernel and gives the library kernels' results bit for bit;
pam_module_launch drives an entry with packed arguments."""
import struct

import numpy as np
import pytest

import oracle
from helpers import TOL, make_case, row_rel_err, to_dev, to_host

pytestmark = pytest.mark.gpu


def _engine(module):
    from pagedattentionmetal_amd import PagedAttentionEngine
    e = PagedAttentionEngine()
    e.set_graceful_degradation(False)
    if module:
        e.load_module()
    return e


def _spec(H, hkv, d, bs, dtype, window=0):
    from pagedattentionmetal_amd import PagedLayerSpec
    return PagedLayerSpec(d, H, hkv, bs, dtype, window)


def test_module_decode_prefill_layers_mixed_bit_identical():
    import torch
    rng = np.random.default_rng(808)
    H, hkv, d, bs = 32, 8, 128, 16
    lens = [3000, 17, 900, 4096, 1]
    q, k, v, bt, lens_u = make_case(rng, len(lens), H, hkv, d, bs, 1, lens)
    args = (to_dev(q), to_dev(k), to_dev(v), to_dev(bt), to_dev(lens_u))
    B, nb = len(lens), bt.shape[1]
    T, off = 700, 1500
    qp = rng.standard_normal((T, H, d)).astype(np.float16)
    qs = [to_dev(rng.standard_normal((B, H, d)).astype(np.float16)) for _ in range(3)]
    ctx = np.array([40, 0, 1000], np.int32)
    ql = np.array([1, 300, 1], np.int32)
    mq = to_dev(rng.standard_normal((int(ql.sum()), H, d)).astype(np.float16))
    res = []
    for module in (False, True):
        e = _engine(module)
        out = {}
        o = torch.zeros((B, H, d), dtype=torch.float16, device="cuda")
        e.decode(*args, o, B, nb, _spec(H, hkv, d, bs, 1))
        out["decode"] = to_host(o)
        outs = [torch.zeros((B, H, d), dtype=torch.float16, device="cuda") for _ in range(3)]
        e.decode_layers(qs, *args[1:], outs, B, nb, [_spec(H, hkv, d, bs, 1)] * 3)
        out["layers"] = [to_host(t) for t in outs]
        o = torch.zeros((T, H, d), dtype=torch.float16, device="cuda")
        e.prefill(to_dev(qp), args[1], args[2], args[3][0].contiguous(), o, T, _spec(H, hkv, d, bs, 1), causal=True,
                  q_offset=off)
        out["prefill"] = to_host(o)
        o = torch.zeros_like(mq)
        e.mixed_step(mq, o, args[1], args[2], args[3][:3].contiguous(), ctx, ql, _spec(H, hkv, d, bs, 1))
        out["mixed"] = to_host(o)
        res.append(out)
        e.close()
    for key in ("decode", "prefill", "mixed"):
        assert np.array_equal(res[0][key].view(np.uint16), res[1][key].view(np.uint16)), key
    for i in range(3):
        assert np.array_equal(res[0]["layers"][i].view(np.uint16), res[1]["layers"][i].view(np.uint16)), i
    ref = oracle.decode(1, q, k, v, bt, lens_u, H, n_threads=8)
    assert row_rel_err(res[1]["decode"].astype(np.float64), ref) <= TOL[1]


def test_module_launch_named_entry_with_packed_arguments():
    import torch
    e = _engine(True)
    f = e.module_function("pam_fill_u32")
    n = 100_003
    dst = torch.zeros(n + 64, dtype=torch.int32, device="cuda")
    # pam_fill_u32(uint32_t *dst, uint32_t value, uint64_t n): 8 + 4 (+4 padding) + 8 bytes
    e.module_launch(f, ((n + 255) // 256,), (256,), struct.pack("<QI4xQ", dst.data_ptr(), 0xC0FFEE, n))
    h = to_host(dst)
    assert (h[:n] == 0xC0FFEE).all() and (h[n:] == 0).all()
    from pagedattentionmetal_amd.api import PagedAttentionError
    with pytest.raises(PagedAttentionError, match="no entry"):
        e.module_function("pam_no_such_kernel")
    # the failed lookup is not left behind for torch's next launch check
    torch.zeros(4, device="cuda").add_(1)
    torch.cuda.synchronize()
    e.close()


def _c3_step(torch, e, w, pools, mode, fp8):
    """One c3 mixed step (append of the new tokens included) on fresh copies of
    the pools; returns the output and the pools' bytes afterwards."""
    from pagedattentionmetal_amd import api
    kp0, vp0, q, nk, nv, ks0, vs0 = pools
    kp, vp = kp0.clone(), vp0.clone()
    ks = ks0.clone() if ks0 is not None else None
    vs = vs0.clone() if vs0 is not None else None
    bt = torch.from_numpy(w.block_tables).cuda()
    out = torch.zeros_like(q)
    e.set_mixed_launch(mode)
    lay = api.PagedLayerSpec(w.head_dim, w.num_heads, w.num_kv_heads, w.block_size, 2 if fp8 else 1)
    e.mixed_step(q, out, kp, vp, bt, w.context_lens, w.query_lens, lay, new_keys=nk, new_values=nv, k_scale=ks,
                 v_scale=vs)
    torch.cuda.synchronize()
    res = [to_host(out), to_host(kp), to_host(vp)]
    if fp8:
        res += [to_host(ks), to_host(vs)]
    return res


def test_module_strict_runs_c1_and_c3_from_the_code_object():
    """A strict module-bound engine (no library kernel may run) decodes c1 (f32,
    VALU rows), a 2100-row GQA decode (workgroup form + reduce kernel) and the c3
    mixed step with its append (f16 in both launch forms, and over e4m3 pools
    quantised by the FP8 append), bit for bit as the library's kernels do."""
    import torch
    from pagedattentionmetal_amd import api, workloads
    from pagedattentionmetal_amd.api import PagedAttentionError
    w1 = workloads.config(1)
    q1, kp1, vp1 = workloads.device_pools(w1)
    bt1 = torch.from_numpy(w1.block_tables).cuda()
    l1 = torch.from_numpy(w1.seq_lens.view("int32")).cuda()
    lay1 = api.PagedLayerSpec(w1.head_dim, w1.num_heads, w1.num_kv_heads, w1.block_size, w1.data_type, w1.window)
    # more rows than the stream-K form takes: the workgroup form and the reduce kernel
    rng = np.random.default_rng(2100)
    lens = rng.integers(1, 400, 2100).tolist()
    qw, kw, vw, btw, lw = make_case(rng, len(lens), 16, 4, 128, 16, 1, lens)
    dw = [to_dev(a) for a in (qw, kw, vw, btw, lw)]
    w3 = workloads.mixed_config()
    kp3, vp3, q3, nk3, nv3 = workloads.mixed_pools(w3)
    # e4m3 pools: the c3 context quantised through the FP8 append kernel (one
    # sequence at a time), by the engine under test
    res = []
    for module in (False, True):
        e = _engine(module)
        if module:
            e.set_module_strict(True)
        out = {}
        o = torch.zeros_like(q1)
        e.set_partition_tokens(0)
        e.decode(q1, kp1, vp1, bt1, l1, o, w1.batch, w1.max_num_blocks, lay1)
        out["c1"] = to_host(o)
        e.set_partition_tokens(64)  # split rows: partitions merged by the reduce kernel
        o = torch.zeros(qw.shape, dtype=torch.float16, device="cuda")
        e.decode(*dw[:5], o, len(lens), btw.shape[1], _spec(16, 4, 128, 16, 1))
        out["wg"] = to_host(o)
        e.set_partition_tokens(0)
        for mode in (0, 2):
            out[f"c3_{mode}"] = _c3_step(torch, e, w3, (kp3, vp3, q3, nk3, nv3, None, None), mode, False)
        k8 = torch.zeros(kp3.shape, dtype=torch.uint8, device="cuda")
        v8 = torch.zeros_like(k8)
        s8k = torch.zeros(kp3.shape[0], dtype=torch.float16, device="cuda")
        s8v = torch.zeros_like(s8k)
        bt3 = torch.from_numpy(w3.block_tables).cuda()
        lay8 = api.PagedLayerSpec(w3.head_dim, w3.num_kv_heads, w3.num_kv_heads, w3.block_size, 2)
        for b in range(len(w3.context_lens)):
            L = int(w3.context_lens[b])
            if L == 0:
                continue
            tok = torch.arange(L, device="cuda")
            phys = bt3[b][tok // w3.block_size].long()
            e.append_to_cache(kp3[phys, tok % w3.block_size].contiguous(), vp3[phys, tok % w3.block_size].contiguous(),
                              k8, v8, bt3[b].contiguous(), 0, L, lay8, k_scale=s8k, v_scale=s8v)
        out["c3_fp8"] = _c3_step(torch, e, w3, (k8, v8, q3, nk3, nv3, s8k, s8v), 0, True)
        if module:
            # the backward kernels are not in the code object: refused, not run
            with pytest.raises(PagedAttentionError, match="code object"):
                T = 16
                qb = torch.zeros((T, 32, 128), dtype=torch.float16, device="cuda")
                kb = torch.zeros((1, 16, 8, 128), dtype=torch.float16, device="cuda")
                m = torch.zeros((T, 32), dtype=torch.float32, device="cuda")
                e.backward(qb, kb, kb, torch.zeros(1, dtype=torch.int32, device="cuda"), qb, m, m + 1,
                           torch.empty_like(qb), torch.zeros_like(kb), torch.zeros_like(kb), T,
                           _spec(32, 8, 128, 16, 1))
        res.append(out)
        e.close()
    lib_, mod = res
    assert np.array_equal(lib_["c1"].view(np.uint32), mod["c1"].view(np.uint32))
    assert np.array_equal(lib_["wg"].view(np.uint16), mod["wg"].view(np.uint16))
    for key in ("c3_0", "c3_2", "c3_fp8"):
        for i, (a, b) in enumerate(zip(lib_[key], mod[key])):
            assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), (key, i)
    ref = oracle.decode(0, to_host(q1), to_host(kp1), to_host(vp1), w1.block_tables, w1.seq_lens, w1.num_heads,
                        n_threads=8)
    assert row_rel_err(mod["c1"].astype(np.float64), ref) <= TOL[0]
    ref = oracle.decode(1, qw, kw, vw, btw, lw, 16, n_threads=8)
    assert row_rel_err(mod["wg"].astype(np.float64), ref) <= TOL[1]


def test_module_strict_d64_prefill_bit_identical():
    """The code object's d = 64 prefill entries (f16, e4m3) give the library
    kernel's bits in a strict module-bound engine."""
    import torch
    rng = np.random.default_rng(6464)
    H, hkv, d, bs, T, off = 16, 4, 64, 16, 300, 700
    for dtype in (1, 2):
        q, k, v, bt, _ = make_case(rng, 1, H, hkv, d, bs, 1, [off + T])
        qp = to_dev(rng.standard_normal((T, H, d)).astype(np.float16))
        outs = []
        for module in (False, True):
            e = _engine(module)
            if module:
                e.set_module_strict(True)
            kd, vd, ks, vs = to_dev(k), to_dev(v), None, None
            if dtype == 2:
                # quantise the same f16 rows into e4m3 pools through the append
                nb = k.shape[0]
                kd = torch.zeros((nb, bs, hkv, d), dtype=torch.uint8, device="cuda")
                vd = torch.zeros_like(kd)
                ks = torch.zeros(nb, dtype=torch.float16, device="cuda")
                vs = torch.zeros_like(ks)
                tok = np.arange(off + T)
                kr = to_dev(k[bt[0, tok // bs], tok % bs])
                vr = to_dev(v[bt[0, tok // bs], tok % bs])
                e.append_to_cache(kr, vr, kd, vd, to_dev(bt[0]), 0, off + T, _spec(hkv, hkv, d, bs, 2), k_scale=ks,
                                  v_scale=vs)
            o = torch.zeros((T, H, d), dtype=torch.float16, device="cuda")
            e.prefill(qp, kd, vd, to_dev(bt[0]), o, T, _spec(H, hkv, d, bs, dtype), causal=True, q_offset=off,
                      k_scale=ks, v_scale=vs)
            outs.append(to_host(o))
            e.close()
        assert np.array_equal(outs[0].view(np.uint16), outs[1].view(np.uint16)), dtype
        if dtype == 1:
            ref = oracle.prefill(1, to_host(qp), k, v, bt[0], off, causal=True, n_threads=8)
            assert row_rel_err(outs[0].astype(np.float64), ref) <= TOL[1]
