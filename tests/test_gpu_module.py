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
