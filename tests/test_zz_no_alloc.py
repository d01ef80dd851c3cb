"""The allocation-free decode entry point (pam_engine_decode_noalloc) against
pam_engine_decode, through the C ABI: same request, same bits, on two calls in
a row (the second with a smaller input), so the fixed scratch's leftovers from
the first call do not leak into the second.  Requests too large for the fixed
scratch are refused with an error."""
import ctypes as C

import numpy as np
import pytest

import oracle
from helpers import TOL, make_case, row_rel_err, to_dev, to_host

pytestmark = pytest.mark.gpu


def _request(lib_mod, q, k, v, bt, lens, out, B, nb, H, hkv, d, bs, dtype, ks=None, vs=None):
    lay = lib_mod.LayerSpec(d, H, hkv, bs, dtype, 0)
    ptr = lambda t: None if t is None else t.data_ptr()
    nbytes = lambda t: 0 if t is None else t.numel() * t.element_size()
    return lib_mod.DecodeRequest(ptr(q), ptr(k), ptr(v), ptr(bt), ptr(lens), ptr(out), B, nb, lay, ptr(ks), ptr(vs),
                                 nbytes(q), nbytes(k), nbytes(v), nbytes(bt), nbytes(lens), nbytes(out))


@pytest.mark.parametrize("case", ["mfma_streamk", "valu_partitions"])
def test_noalloc_decode_matches_decode(case):
    import torch
    from pagedattentionmetal_amd import _lib
    lib = _lib.load()
    ctx = lib.pam_create_context()
    try:
        assert lib.pam_engine_set_graceful_degradation(ctx, False) == 0
        assert lib.pam_engine_setup_noalloc(ctx) == 0, lib.pam_last_error(ctx)
        rng = np.random.default_rng(4242)
        if case == "mfma_streamk":
            H, hkv, d, bs, dtype = 32, 8, 128, 16, 1
            calls = [[3000, 17, 900, 4096, 1, 2500, 700, 64], [1500, 33]]
        else:  # f32: VALU kernel, split-context partitions and the reduce kernel
            H, hkv, d, bs, dtype = 8, 8, 128, 16, 0
            calls = [[700, 12, 300], [90]]
        for i, lens in enumerate(calls):
            q, k, v, bt, lens_u = make_case(rng, len(lens), H, hkv, d, bs, dtype, lens)
            B, nb = len(lens), bt.shape[1]
            qd, kd, vd, btd, ld = to_dev(q), to_dev(k), to_dev(v), to_dev(bt), to_dev(lens_u)
            tdt = torch.float32 if dtype == 0 else torch.float16
            out_a = torch.full((B, H, d), 7.0, dtype=tdt, device="cuda")
            out_b = torch.full((B, H, d), -3.0, dtype=tdt, device="cuda")
            ra = _request(_lib, qd, kd, vd, btd, ld, out_a, B, nb, H, hkv, d, bs, dtype)
            rb = _request(_lib, qd, kd, vd, btd, ld, out_b, B, nb, H, hkv, d, bs, dtype)
            assert lib.pam_engine_decode(ctx, C.byref(ra)) == 0, lib.pam_last_error(ctx)
            assert lib.pam_engine_decode_noalloc(ctx, C.byref(rb)) == 0, lib.pam_last_error(ctx)
            torch.cuda.synchronize()
            a, b = to_host(out_a), to_host(out_b)
            bits = np.uint32 if dtype == 0 else np.uint16
            assert np.array_equal(a.view(bits), b.view(bits)), f"call {i}: noalloc differs from decode"
            ref = oracle.decode(dtype, q, k, v, bt, lens_u, H, n_threads=8)
            assert row_rel_err(b.astype(np.float64), ref) <= TOL[dtype], f"call {i}"
    finally:
        lib.pam_destroy_context(ctx)


def test_noalloc_refuses_what_does_not_fit():
    """A stream-K workspace above the fixed scratch is an error, not an allocation."""
    import torch
    from pagedattentionmetal_amd import _lib
    lib = _lib.load()
    ctx = lib.pam_create_context()
    try:
        assert lib.pam_engine_set_graceful_degradation(ctx, False) == 0
        # not set up yet: refused
        H, hkv, d, bs = 64, 4, 256, 16
        B = 2048
        q = torch.zeros((B, H, d), dtype=torch.float16, device="cuda")
        k = torch.zeros((4, bs, hkv, d), dtype=torch.float16, device="cuda")
        bt = torch.zeros((B, 1), dtype=torch.int32, device="cuda")
        lens = torch.ones(B, dtype=torch.int32, device="cuda")
        out = torch.empty_like(q)
        r = _request(_lib, q, k, k, bt, lens, out, B, 1, H, hkv, d, bs, 1)
        assert lib.pam_engine_decode_noalloc(ctx, C.byref(r)) == -1
        assert b"pam_engine_setup_noalloc" in lib.pam_last_error(ctx)
        assert lib.pam_engine_setup_noalloc(ctx) == 0
        # (2048 rows + units) x 64 heads x (256 + 2) floats: far above 32 MiB
        assert lib.pam_engine_decode_noalloc(ctx, C.byref(r)) == -1
        assert b"fixed" in lib.pam_last_error(ctx)
        # graceful degradation does not turn the size limit into zeros and success
        assert lib.pam_engine_set_graceful_degradation(ctx, True) == 0
        assert lib.pam_engine_decode_noalloc(ctx, C.byref(r)) == -1
        assert b"fixed" in lib.pam_last_error(ctx)
    finally:
        lib.pam_destroy_context(ctx)
