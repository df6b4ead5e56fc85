"""The HIP path's layouts against the committed fixtures (tests/golden/):
device CADR permutations, hybrid partition and row-sorted views of the
order-3 driver; device HITS ranks, relabelled coordinates, dense units and
views of the generic driver — byte for byte."""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    d = np.load(os.path.join(GOLDEN, name), allow_pickle=False)
    return {k: d[k] for k in d.files}


def test_order3_layout_matches_golden(ca, dev):
    g = _load("layout3.npz")
    t = ca.Tensor(tuple(int(x) for x in g["dims"]), g["idx"], g["val"])
    with ca.Als3(t, R=8, threshold=0.03) as h:
        for m in range(3):
            assert np.array_equal(h.perm(m), g["perm%d" % m]), m
        assert int(h.info.dense_cutoff) == int(g["cutoff"])
        tl = h.tiles()
        for k in ("tiles", "pool_off", "pool_lid", "pool_val"):
            assert np.array_equal(tl[k], g[k]), k
        for m in range(3):
            v = h.view(0, m)
            for k in ("coords", "vals", "blk_row", "blk_start", "blk_cnt"):
                assert np.array_equal(v[k], g["view%d_%s" % (m, k)]), (m, k)


def test_generic_layout_matches_golden(ca, dev):
    g = _load("layoutN.npz")
    dims = tuple(int(x) for x in g["dims"])
    t = ca.Tensor(dims, g["idx"], g["val"])
    gen = ca.Gen(t, R=8, reorder="hits", rounds=3, threshold=0.03)
    try:
        assert np.array_equal(gen.coords(), g["ridx"])
        for m in range(len(dims)):
            assert np.array_equal(gen.rank(m), g["rank%d" % m]), m
        u = gen.units()
        assert int(gen.info.cutoff) == int(g["unit_cutoff"])
        for k in ("unit6", "outer_coords", "lid", "val", "is_dense"):
            assert np.array_equal(u[k].ravel(), g["unit_" + k].ravel()), k
        for n in range(len(dims)):
            v = gen.view(n)
            assert np.array_equal(v["scoords"].ravel(), g["view%d_scoords" % n].ravel()), n
            for k in ("vals", "skip", "row", "start", "cnt", "single"):
                assert np.array_equal(v[k], g["view%d_%s" % (n, k)]), (n, k)
    finally:
        gen.close()
