"""The committed layout fixtures (tests/golden/, written by
tests/golden/make_golden.py) against the CPU oracle: the oracle must keep
producing the same bytes for CADR, the hybrid partition, the order-3 views,
HITS, the dense units and the N-order views.  Pure host code."""
import os

import numpy as np
import pytest

from golden.make_golden import layout3, layoutN

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    d = np.load(os.path.join(GOLDEN, name), allow_pickle=False)
    return {k: d[k] for k in d.files}


@pytest.mark.parametrize("name,fn", [("layout3.npz", layout3), ("layoutN.npz", layoutN)])
def test_oracle_reproduces_golden(orc, name, fn):
    g = _load(name)
    dims = tuple(int(x) for x in g["dims"])
    got = fn(orc, dims, g["idx"], g["val"])
    assert set(got) == set(g) - {"dims", "idx", "val"}
    for k, v in got.items():
        assert v.dtype == g[k].dtype and np.array_equal(v, g[k]), k


def test_golden_fixtures_are_not_trivial():
    g3 = _load("layout3.npz")
    assert len(g3["tiles"]) > 0 and len(g3["view0_vals"]) > 0       # both halves present
    assert int(g3["cutoff"]) == int(4096 * 0.03)
    gn = _load("layoutN.npz")
    assert len(gn["unit_unit6"]) > 0 and 0 < int(gn["unit_is_dense"].sum()) < gn["idx"].shape[1]
    assert any(not np.array_equal(gn["rank%d" % m], np.arange(len(gn["rank%d" % m])))
               for m in range(4))
