"""Edge cases of the order-3 driver against the oracle: an empty tensor, a
single nonzero, rows that end exactly at and just past the 1024-element
segment length (and one spanning three segments), and ranks 1, 2, 3 (odd
widths, the 1-rank-per-lane kernels) and 200 (past the 128-rank block: rank
blocks on the grid, per-tile atomics instead of tile groups)."""
import numpy as np
import pytest

from conftest import rel_err

pytestmark = pytest.mark.gpu


def oracle_layout(orc, t, thr):
    idx = t.idx.astype(np.int32)
    perms = orc.cadr3(idx[0], idx[1], idx[2], t.dims)
    idx = np.stack([perms[m][idx[m]] for m in range(3)]).astype(np.int32)
    p = orc.partition3(idx[0], idx[1], idx[2], t.val, t.dims, thr)
    v = orc.views3(p["sp_i"], p["sp_j"], p["sp_k"], p["sp_val"], t.dims)
    return perms, p, v


def oracle_mttkrp(orc, p, v, F, R, dims, mode, mfma):
    ref = orc.mttkrp3_view(v, mode, *(f.ravel() for f in F), R, dims[mode])
    if mfma:
        ref = ref + orc.mttkrp3_tiles(p, mode, *(f.ravel() for f in F), R, dims)
    elif len(p["pool_val"]):
        dv = orc.dense_views3(p, dims)
        ref = ref + orc.mttkrp3_view(dv, mode, *(f.ravel() for f in F), R, dims[mode])
    return ref.reshape(dims[mode], R)


def check_against_oracle(ca, orc, t, R, thr, iters, fit_tol):
    perms, p, v = oracle_layout(orc, t, thr)
    with ca.Als3(t, R=R, threshold=thr) as h:
        mfma = int(h.info.use_mfma) == 1 and len(p["tiles"]) > 0
        for m in range(3):
            assert np.array_equal(h.perm(m), perms[m])
            got = h.view(0, m)
            for k in ("coords", "vals", "blk_row", "blk_start", "blk_cnt"):
                assert np.array_equal(got[k], np.asarray(v[m][k])), (m, k)
        F = [h.factor(m) for m in range(3)]
        for mode in range(3):
            ref = oracle_mttkrp(orc, p, v, F, R, t.dims, mode, mfma)
            assert rel_err(h.mttkrp(mode), ref) <= (1e-5 if mfma else 1e-12), mode
        dv = orc.dense_views3(p, t.dims) if (not mfma and len(p["pool_val"])) else None
        o = orc.Als3(v, dv, p if mfma else None, float(np.sum(t.val ** 2)), t.dims, R,
                     *(f.ravel() for f in F), None)
        fit, _, _ = h.run(iters)
        ofit, _, _ = o.iterate(iters)
        assert np.max(np.abs(fit - ofit)) <= fit_tol, (fit, ofit)
        return v


def test_empty_tensor(ca, dev):
    """No nonzeros: every MTTKRP is zero and the fit is 0 (||X|| = 0).  The
    first update zeroes the factor and lambda (norms < 1e-14), and the next
    one divides by that zero lambda as the reference does unconditionally
    (factor_divide_lambda_kernel, als.cu:345-360): the factors become NaN,
    as they do in the reference."""
    t = ca.Tensor((5, 6, 7), np.zeros((3, 0), np.uint32), np.zeros(0))
    with ca.Als3(t, R=4) as h:
        assert int(h.info.sparse_nnz) == 0 and int(h.info.num_dense_tiles) == 0
        for m in range(3):
            assert np.all(h.mttkrp(m) == 0.0)
        fit, _, _ = h.run(1)
        assert np.all(fit == 0.0)
        assert np.all(h.lam() == 0.0) or np.all(np.isnan(h.lam()))
        assert np.all(np.isnan(h.factor(1))) and np.all(np.isnan(h.factor(2)))


@pytest.mark.parametrize("big", [0, 1, 2])
def test_dim_beyond_packed_coordinates(ca, dev, big):
    """A mode of 32768 or more indices does not fit the views' 15-bit packed
    coordinate.  The reference then skips building the views and computes a
    zero sparse MTTKRP (partition.cu:1896-1906, sparse.cu:839-843); here
    creating the driver fails with an error that names the limit, whichever
    mode is too long (32767 still works)."""
    dims = [20, 30, 40]
    dims[big] = 32768
    rng = np.random.default_rng(big)
    idx = np.stack([rng.integers(0, d, 500) for d in dims]).astype(np.uint32)
    idx[big, 0] = 32767
    t = ca.Tensor(tuple(dims), idx, rng.random(500) + 0.5)
    with pytest.raises(ca.CptcError, match="32768"):
        ca.Als3(t, R=8)
    dims[big] = 32767
    idx[big, 0] = 32766
    t = ca.Tensor(tuple(dims), idx, rng.random(500) + 0.5)
    with ca.Als3(t, R=8) as h:
        assert int(h.info.sparse_nnz) + int(h.info.dense_nnz) == 500


def test_single_nonzero(ca, orc, dev):
    t = ca.Tensor((3, 4, 5), np.array([[1], [2], [3]], np.uint32), np.array([2.5]))
    check_against_oracle(ca, orc, t, R=4, thr=0.03, iters=10, fit_tol=1e-8)


@pytest.mark.parametrize("R", [16, 128])
def test_segment_boundaries(ca, orc, dev, R):
    """Rows of exactly 1024, 1025 and 2049 elements (one, two and three
    segments) in mode 0; no tiles (threshold 1.0)."""
    rng = np.random.default_rng(R)
    cells = np.array(np.meshgrid(np.arange(48), np.arange(48), indexing="ij")).reshape(2, -1)
    parts = []
    for i, n in enumerate((1024, 1025, 2049)):
        c = cells[:, rng.choice(cells.shape[1], n, replace=False)]
        parts.append(np.vstack([np.full((1, n), i), c]))
    idx = np.concatenate(parts, axis=1)
    idx = idx[:, rng.permutation(idx.shape[1])].astype(np.uint32)
    t = ca.Tensor((3, 48, 48), idx, rng.random(idx.shape[1]) + 0.5)
    v = check_against_oracle(ca, orc, t, R=R, thr=1.0, iters=5, fit_tol=1e-8)
    # mode 0's segments: 1 + 2 + 3 after CADR (rows reordered by degree)
    assert sorted(np.asarray(v[0]["blk_cnt"]).tolist()) == sorted([1024, 1024, 1, 1024, 1024, 1])


@pytest.mark.parametrize("R", [1, 2, 3, 200])
def test_rank_edges(ca, orc, dev, R):
    t = ca.synth_zipf((300, 200, 500), (1.3, 1.3, 1.3), 20000, 0, 5)
    check_against_oracle(ca, orc, t, R=R, thr=0.03, iters=5, fit_tol=1e-4)
