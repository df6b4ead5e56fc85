"""Synthetic generators: deterministic for a seed, independent of the thread
count, exact nnz with distinct coordinates, the configured shapes."""
import os
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def lin(t):
    return np.ravel_multi_index(tuple(t.idx.astype(np.int64)), t.dims)


def test_zipf_deterministic_and_distinct(ca):
    a = ca.synth_zipf((300, 200, 500), (1.1, 1.1, 1.1), 50000, 0, 5)
    b = ca.synth_zipf((300, 200, 500), (1.1, 1.1, 1.1), 50000, 0, 5)
    c = ca.synth_zipf((300, 200, 500), (1.1, 1.1, 1.1), 50000, 0, 6)
    assert np.array_equal(a.idx, b.idx) and np.array_equal(a.val, b.val)
    assert not np.array_equal(a.idx, c.idx)
    assert a.nnz == 50000 and len(np.unique(lin(a))) == 50000
    assert np.all(a.val > 0)                                     # log-normal
    assert np.all(a.idx.max(axis=1) < np.array(a.dims))


def test_zipf_is_heavy_tailed(ca):
    t = ca.synth_zipf((2000, 1500, 3000), (1.1, 1.1, 1.1), 200000, 0, 1)
    for m in range(3):
        c = np.sort(np.bincount(t.idx[m], minlength=t.dims[m]))[::-1]
        assert c[0] > 20 * np.median(c[c > 0])


def test_thread_count_independent(ca):
    code = ("import sys; sys.path.insert(0, %r); import cptc_amd as ca, hashlib;"
            "t = ca.synth_zipf((400, 300, 700), (1.1, 1.1, 1.1), 80000, 0, 9);"
            "print(hashlib.sha1(t.idx.tobytes() + t.val.tobytes()).hexdigest())") % ROOT
    outs = []
    for nt in ("1", "3", "8"):
        env = dict(os.environ, OMP_NUM_THREADS=nt)
        outs.append(subprocess.run([sys.executable, "-c", code], env=env, check=True,
                                   capture_output=True, text=True).stdout.strip())
    assert outs[0] == outs[1] == outs[2]


def test_value_kinds(ca):
    p = ca.synth_zipf((183, 24, 1140, 1717), (0, 0, 1.2, 1.2), 20000, 2, 3)
    assert p.nmodes == 4 and np.all(p.val >= 1) and np.all(p.val == np.round(p.val))
    assert abs(p.val.mean() - 3.0) < 0.1                          # 1 + Poisson(2)
    n = ca.synth_zipf((50, 60, 70), (0, 0, 0), 20000, 1, 3)
    assert abs(n.val.mean()) < 0.05 and abs(n.val.std() - 1) < 0.05


def test_blocks_and_lowrank_small(ca):
    b = ca.synth_blocks3(64, 10, 0.1, 0.6, 2e-4, 4)
    assert b.dims == (64, 64, 64) and len(np.unique(lin(b))) == b.nnz
    assert 10 * 4096 * 0.1 * 0.5 < b.nnz < 10 * 4096 * 0.6 + 2000
    l = ca.synth_lowrank3(32, 2, 0.9, 0.1, 4)
    assert abs(l.nnz / 32 ** 3 - 0.9) < 0.02 and len(np.unique(lin(l))) == l.nnz


def test_units5_small(ca):
    u = ca.synth_units5((32, 32, 32, 8, 4), 20, 0.05, 0.5, 100000, 4, 2)
    assert u.nmodes == 5 and u.nnz == 100000 and len(np.unique(lin(u))) == u.nnz


@pytest.mark.parametrize("cfg,nnz", [(2, None), (4, 3300000)])
def test_configs_shapes(ca, cfg, nnz):
    t = ca.synth_config(cfg)
    dims = {2: (512, 512, 512), 4: (183, 24, 1140, 1717)}[cfg]
    assert t.dims == dims
    if nnz:
        assert t.nnz == nnz
    else:
        assert 2.5e6 < t.nnz < 3.5e6
    assert len(np.unique(lin(t))) == t.nnz
