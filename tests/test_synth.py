"""The synthetic-data generator of the measured workloads (host side): the
SplitMix64 known answers, the numpy version against the element-wise
restatement in oracle/synth.py, and the distributions it produces."""
import numpy as np
import pytest

from oracle import synth as ref
from pagedattentionmetal_amd import workloads as wl

# published SplitMix64 outputs for seed 1234567 (Vigna's splitmix64.c)
KNOWN = [6457827717110365317, 3203168211198807973, 9817491932198370423, 4593380528125082431,
         16408922859458223821]


def test_splitmix_known_answers():
    assert [ref.splitmix(1234567, k) for k in range(5)] == KNOWN
    assert wl.splitmix(1234567, 0, np.arange(5)).tolist() == KNOWN


@pytest.mark.parametrize("stream,start", [(0, 0), (3, 12345), (8, (1 << 39) - 40)])
def test_numpy_draws_equal_restatement(stream, start):
    seed = wl.SEED_BASE + 2
    u = wl.uniforms(seed, stream, 64, start)
    assert u.tolist() == [ref.uniform(seed, stream, start + i) for i in range(64)]
    n = wl.normals(seed, stream, 20, start // 2)
    assert n.tolist() == [ref.normal(seed, stream, start // 2 + i) for i in range(20)]


def test_distributions():
    from scipy import stats
    x = wl.normals(wl.SEED_BASE + 4, wl.S_K, 200_000)
    assert abs(x.mean()) < 0.01 and abs(x.var() - 1.0) < 0.01
    assert stats.kstest(x, "norm").pvalue > 1e-3
    u = wl.uniforms(wl.SEED_BASE + 4, wl.S_PERM, 200_000)
    assert u.min() >= 0.0 and u.max() < 1.0
    assert stats.kstest(u, "uniform").pvalue > 1e-3
    p = wl.permutation(wl.SEED_BASE + 2, 32768)
    assert np.array_equal(np.sort(p), np.arange(32768))
    assert (p != np.arange(32768)).mean() > 0.99


def test_configs_follow_the_survey_shapes():
    c1 = wl.config(1)
    assert c1.batch == 4 and ((c1.seq_lens >= 17) & (c1.seq_lens <= 200)).all()
    c2 = wl.config(2)
    sh = c2.extra["sharers"]
    assert (c2.seq_lens[:sh] >= 513).all() and ((c2.seq_lens >= 128) & (c2.seq_lens <= 4096)).all()
    assert (c2.block_tables[:sh, :32] == c2.block_tables[0, :32]).all()
    used = np.concatenate([c2.block_tables[b, :(int(L) + 15) // 16] for b, L in enumerate(c2.seq_lens)])
    assert len(set(used.tolist())) == len(used) - 32 * (sh - 1)  # only the prefix is shared
    c4 = wl.config(4)
    assert ((c4.seq_lens >= 16) & (c4.seq_lens <= 8192)).all()
    assert 600 < np.median(c4.seq_lens) < 1700
    c5 = wl.config(5)
    assert ((c5.seq_lens >= 16384) & (c5.seq_lens <= 131072)).all()
    m = wl.mixed_config()
    assert (m.query_lens[:8] == 512).all() and (m.query_lens[8:] == 1).all()
    assert ((m.context_lens[:8] >= 0) & (m.context_lens[:8] <= 3584)).all()
    assert ((m.context_lens[8:] + 1 >= 256) & (m.context_lens[8:] + 1 <= 4096)).all()
