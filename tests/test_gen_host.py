"""Host side of the generic N-order path (no GPU): the reordering entry point
cptc_gen_reorder against the oracle's restatement of apply_reordering
(generic.cu:1176-1376), bit for bit, and the unit-key hash."""
import numpy as np
import pytest

import cptc_amd as ca


def _tensor(rng, dims, nnz, zipf=None):
    cols = []
    for m, d in enumerate(dims):
        if zipf and zipf[m]:
            p = 1.0 / np.arange(1, d + 1) ** zipf[m]
            cols.append(rng.choice(d, nnz, p=p / p.sum()))
        else:
            cols.append(rng.integers(0, d, nnz))
    idx = np.ascontiguousarray(np.stack(cols).astype(np.uint32))
    return ca.Tensor(tuple(dims), idx, rng.random(nnz) + 0.5)


@pytest.mark.parametrize("how,rounds,budget", [("hits", 3, 8000000), ("hits", 1, 8000000),
                                               ("hits", 3, 777), ("cadr", 3, 8000000),
                                               ("none", 3, 8000000), ("bogus", 3, 8000000)])
def test_reorder_matches_oracle(orc, how, rounds, budget):
    rng = np.random.default_rng(11)
    t = _tensor(rng, (60, 20, 300, 45), 20000, zipf=(1.1, 0, 1.2, 1.0))
    new, ranks, applied = ca.gen_reorder(t, how, rounds, budget)
    ohow = "cadr" if how == "bogus" else how
    ref_idx, ref_rank = orc.reorder_nd(t.idx, t.val, t.dims, ohow, rounds, budget)
    assert np.array_equal(new.idx, ref_idx)
    if ohow == "none":
        assert not applied
        assert all(np.array_equal(r, np.arange(d)) for r, d in zip(ranks, t.dims))
    else:
        assert applied
        for m in range(4):
            assert np.array_equal(ranks[m], ref_rank[m]), m


def test_reorder_auto_both_branches(orc):
    rng = np.random.default_rng(5)
    dense = _tensor(rng, (32, 32, 32, 2), 30000)
    sparse = _tensor(rng, (5000, 5000, 5000, 2), 3000)
    outcomes = set()
    for t in (dense, sparse):
        new, ranks, applied = ca.gen_reorder(t, "auto", 3, 8000000)
        ref_idx, ref_rank = orc.reorder_nd(t.idx, t.val, t.dims, "auto", 3, 8000000)
        assert np.array_equal(new.idx, ref_idx)
        assert applied == (len(ref_rank) > 0)
        if applied:
            assert all(np.array_equal(ranks[m], ref_rank[m]) for m in range(4))
        outcomes.add(applied)
    assert outcomes == {True, False}


def test_reorder_default_by_order(orc):
    rng = np.random.default_rng(6)
    t3 = _tensor(rng, (50, 40, 30), 5000, zipf=(1.0, 1.0, 0))
    t4 = _tensor(rng, (50, 40, 30, 9), 5000, zipf=(1.0, 1.0, 0, 0))
    n3, r3, _ = ca.gen_reorder(t3, None)
    n4, r4, _ = ca.gen_reorder(t4, None)
    assert np.array_equal(n3.idx, orc.reorder_nd(t3.idx, t3.val, t3.dims, "cadr", 3, 8000000)[0])
    assert np.array_equal(n4.idx, orc.reorder_nd(t4.idx, t4.val, t4.dims, "hits", 3, 8000000)[0])


def test_reorder_config4_scale(orc):
    """Bit-exact HITS on the config-4 generator (3.3 M elements)."""
    t = ca.synth_config(4)
    new, ranks, applied = ca.gen_reorder(t, "hits", 3, 8000000)
    ref_idx, ref_rank = orc.reorder_nd(t.idx, t.val, t.dims, "hits", 3, 8000000)
    assert applied
    for m in range(4):
        assert np.array_equal(ranks[m], ref_rank[m]), m
    assert np.array_equal(new.idx, ref_idx)


def test_reorder_rejects_bad_index():
    t = ca.Tensor((4, 4, 4, 4), np.array([[0], [1], [9], [2]], np.uint32), np.ones(1))
    with pytest.raises(ca.CptcError):
        ca.gen_reorder(t, "hits")


def test_hash_matches_oracle(orc):
    for x in [0, 1, 2 ** 63, 0xDEADBEEF, 2 ** 64 - 1, 123456789 << 20]:
        assert ca.gen_hash(x) == orc.splitbit_hash(x)
