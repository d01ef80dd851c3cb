"""pam_synth_normal on the GPU against the host generator: the same values bit
for bit after rounding (f32 and f16 outputs, with and without outliers)."""
import numpy as np
import pytest

from oracle import synth as ref

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype,std,outliers", [("f32", 1.0, False), ("f16", 0.5, False), ("f16", 1.0, True)])
def test_device_normals_equal_host(dtype, std, outliers):
    import torch
    from pagedattentionmetal_amd import workloads as wl
    seed, n = wl.SEED_BASE + 4, 1 << 20
    tdt = torch.float32 if dtype == "f32" else torch.float16
    ostream, frac = (wl.S_K_OUTLIERS, 0.01) if outliers else (-1, 0.0)
    got = wl.device_normals((n,), tdt, seed, wl.S_K, std, ostream, frac).cpu().numpy()
    x = wl.normals(seed, wl.S_K, n) * std
    if outliers:
        hit = wl.uniforms(seed, wl.S_K_OUTLIERS, n) < frac
        x = np.where(hit, x * 8.0, x)
        assert 0.008 < hit.mean() < 0.012
    want = x.astype(np.float32)
    if dtype == "f16":
        want = want.astype(np.float16)
    diff = np.flatnonzero(got.view(np.uint32 if dtype == "f32" else np.uint16)
                          != want.view(np.uint32 if dtype == "f32" else np.uint16))
    assert diff.size == 0, f"{diff.size} of {n} differ, first at {diff[:5].tolist()}"
    # a slice against the element-wise restatement
    for i in range(0, n, n // 256):
        e = np.float32(ref.element(seed, wl.S_K, i, std, ostream, frac))
        assert (np.float16(e) if dtype == "f16" else e) == got[i]


def test_workload_pools_are_the_generator_streams():
    import torch
    from pagedattentionmetal_amd import workloads as wl
    w = wl.config(1)
    q, k, v = wl.device_pools(w)
    assert q.dtype == torch.float32 and k.shape == (w.pool_blocks, 16, 8, 128)
    flat = k.reshape(-1)[:4096].cpu().numpy()
    assert np.array_equal(flat, wl.normals(w.seed, wl.S_K, 4096).astype(np.float32))
    qf = q.reshape(-1)[:4096].cpu().numpy()
    assert np.array_equal(qf, wl.normals(w.seed, wl.S_Q, 4096).astype(np.float32))
