"""Pins the oracle's arithmetic: MTTKRP (row views and dense tiles), Gram,
pseudoinverse and the ALS iteration, against closed forms computed with
numpy on dense tensors.

mttkrp3_view   sparse.cu:614-711   Y_(n) = X_(n) (khatri-rao) = einsum, duplicates summed
mttkrp3_tiles  dense.cu:89-1077    einsum over the tile with last-write-wins cells
gram           als.cu:115-134      F^T F
pinv_sym       solver.cu:900-1002  Moore-Penrose conditions; inverse for SPD
als3_iterate   als.cu:362-821      an independent numpy ALS (einsum MTTKRP, numpy
                                   pinv, same normalisation); Gram fit == exact fit
"""
import numpy as np
import pytest

from conftest import rel_err

EIN = {0: "ijk,jr,kr->ir", 1: "ijk,ir,kr->jr", 2: "ijk,ir,jr->kr"}


def mttkrp_dense(X, F, mode):
    others = [F[m] for m in range(3) if m != mode]
    return np.einsum(EIN[mode], X, *others)


def dense_from(idx, val, dims):
    X = np.zeros(dims)
    np.add.at(X, tuple(idx), val)
    return X


def build(orc, idx, val, dims, thr):
    p = orc.partition3(idx[0], idx[1], idx[2], val, dims, thr)
    v = orc.views3(p["sp_i"], p["sp_j"], p["sp_k"], p["sp_val"], dims)
    return p, v


@pytest.mark.parametrize("R", [1, 5, 16])
def test_mttkrp_view_closed_form(orc, R):
    rng = np.random.default_rng(R)
    dims = (19, 23, 17)
    n = 2500
    idx = np.stack([rng.integers(0, d, n) for d in dims]).astype(np.int32)
    idx[:, -200:] = idx[:, :200]                      # duplicates are summed
    val = rng.standard_normal(n)
    p, v = build(orc, idx, val, dims, 1.0)            # cutoff 4096: no tiles
    assert len(p["tiles"]) == 0
    F = [rng.random((d, R)) for d in dims]
    X = dense_from(idx, val, dims)
    for mode in range(3):
        got = orc.mttkrp3_view(v, mode, F[0].ravel(), F[1].ravel(), F[2].ravel(), R,
                               dims[mode]).reshape(dims[mode], R)
        assert rel_err(got, mttkrp_dense(X, F, mode)) < 1e-13


@pytest.mark.parametrize("R", [3, 16, 20])
def test_mttkrp_tiles_closed_form(orc, R):
    rng = np.random.default_rng(100 + R)
    dims = (40, 37, 45)                                 # partial boundary tiles
    cells = np.array(np.meshgrid(np.arange(32, 40), np.arange(16, 37), np.arange(0, 45),
                                 indexing="ij")).reshape(3, -1)
    keep = rng.random(cells.shape[1]) < 0.6
    dense_part = cells[:, keep]
    bg = np.stack([rng.integers(0, d, 800) for d in dims])
    idx = np.concatenate([dense_part, bg], axis=1).astype(np.int32)
    # unique coordinates (tile cells hold one value)
    lin = np.ravel_multi_index(tuple(idx), dims)
    _, first = np.unique(lin, return_index=True)
    idx = idx[:, np.sort(first)]
    val = rng.standard_normal(idx.shape[1])
    p, v = build(orc, idx, val, dims, 0.03)
    assert len(p["tiles"]) > 0 and len(p["sp_val"]) > 0
    F = [rng.random((d, R)) for d in dims]
    X = dense_from(idx, val, dims)
    for mode in range(3):
        got = orc.mttkrp3_view(v, mode, F[0].ravel(), F[1].ravel(), F[2].ravel(), R,
                               dims[mode]).reshape(dims[mode], R)
        got += orc.mttkrp3_tiles(p, mode, F[0].ravel(), F[1].ravel(), F[2].ravel(), R,
                                 dims).reshape(dims[mode], R)
        assert rel_err(got, mttkrp_dense(X, F, mode)) < 1e-13


def test_mttkrp_tiles_last_write_wins(orc):
    rng = np.random.default_rng(7)
    dims, R = (16, 16, 16), 4
    cells = np.array(np.meshgrid(*[np.arange(16)] * 3, indexing="ij")).reshape(3, -1)
    idx = np.concatenate([cells, cells[:, :100]], axis=1).astype(np.int32)  # 100 duplicates
    val = rng.standard_normal(idx.shape[1])
    p = orc.partition3(idx[0], idx[1], idx[2], val, dims, 0.5)
    assert len(p["tiles"]) == 1
    X = np.zeros(dims)
    X[tuple(idx)] = val          # numpy fancy assignment: last write wins
    F = [rng.random((16, R)) for _ in range(3)]
    for mode in range(3):
        got = orc.mttkrp3_tiles(p, mode, F[0].ravel(), F[1].ravel(), F[2].ravel(), R,
                                dims).reshape(16, R)
        assert rel_err(got, mttkrp_dense(X, F, mode)) < 1e-13


def test_gram(orc):
    rng = np.random.default_rng(2)
    F = rng.standard_normal((301, 13))
    assert rel_err(orc.gram(F.ravel(), 13).reshape(13, 13), F.T @ F) < 1e-14


@pytest.mark.parametrize("R", [1, 4, 32, 128])
def test_pinv_spd_is_inverse(orc, R):
    rng = np.random.default_rng(R)
    F = rng.random((4 * R + 10, R))
    A = (F.T @ F) * ((F.T @ F) / R)                     # Hadamard of Grams: SPD
    got, _ = orc.pinv_sym(A.ravel(), R)
    assert rel_err(got.reshape(R, R), np.linalg.inv(A)) < 1e-9


def test_pinv_singular_moore_penrose(orc):
    rng = np.random.default_rng(4)
    R = 12
    F = rng.random((50, R))
    F[:, 5] = F[:, 2]                                   # rank-deficient Gram
    F[:, 9] = 0.0
    A = F.T @ F
    P, _ = orc.pinv_sym(A.ravel(), R)
    P = P.reshape(R, R)
    assert rel_err(A @ P @ A, A) < 1e-10
    assert rel_err(P @ A @ P, P) < 1e-8
    assert rel_err(P, P.T) < 1e-14
    assert rel_err(P, np.linalg.pinv(A, rcond=1e-10)) < 1e-6
    Z, _ = orc.pinv_sym(np.zeros(R * R), R)
    assert np.all(Z == 0.0)


def numpy_als(X, F, iters):
    """Independent restatement of als.cu:612-729 on a dense tensor."""
    F = [f.copy() for f in F]
    R = F[0].shape[1]
    lam = np.ones(R)
    X2 = np.sum(X * X)
    fits = []
    for _ in range(iters):
        for mode in range(3):
            p, q = [m for m in range(3) if m != mode]
            FtF = (F[p].T @ F[p]) * (F[q].T @ F[q])
            M = mttkrp_dense(X, F, mode)
            w, V = np.linalg.eigh(FtF)
            tol = R * np.spacing(np.max(np.abs(w)))
            winv = np.where(np.abs(w) > tol, 1.0 / np.where(w == 0, 1, w), 0.0)
            A = M @ (V * winv) @ V.T
            A = A / lam
            n = np.sqrt(np.sum(A * A, axis=0))
            A = np.where(n < 1e-14, 0.0, A / np.where(n < 1e-14, 1.0, n))
            lam = np.where(n < 1e-14, 0.0, lam * n)
            F[mode] = A
        iprod = np.sum(lam * np.sum(F[2] * M, axis=0))
        model2 = np.sum(np.outer(lam, lam) * (F[0].T @ F[0]) * (F[1].T @ F[1]) * (F[2].T @ F[2]))
        fits.append(1.0 - np.sqrt(max(X2 - 2 * iprod + model2, 0.0)) / np.sqrt(X2))
    return np.array(fits), F, lam


def test_als_matches_numpy_restatement(orc):
    rng = np.random.default_rng(11)
    dims, R = (21, 18, 25), 6
    n = 3000
    idx = np.stack([rng.integers(0, d, n) for d in dims]).astype(np.int32)
    lin = np.ravel_multi_index(tuple(idx), dims)
    _, first = np.unique(lin, return_index=True)
    idx = idx[:, np.sort(first)]
    val = rng.random(idx.shape[1]) + 0.5
    p, v = build(orc, idx, val, dims, 1.0)
    F = [rng.random((d, R)) for d in dims]
    x_sq = float(np.sum(val * val))
    o = orc.Als3(v, None, None, x_sq, dims, R, F[0].ravel(), F[1].ravel(), F[2].ravel(), None)
    fits, _, _ = o.iterate(6)
    rfits, rF, rlam = numpy_als(dense_from(idx, val, dims), F, 6)
    assert np.max(np.abs(fits - rfits)) < 1e-9
    for m in range(3):
        assert rel_err(o.factor(m).reshape(dims[m], R), rF[m]) < 1e-7
    assert rel_err(o.lam(), rlam) < 1e-8


def test_gram_fit_equals_exact_fit(orc):
    rng = np.random.default_rng(12)
    dims, R = (30, 20, 26), 5
    n = 4000
    idx = np.stack([rng.integers(0, d, n) for d in dims]).astype(np.int32)
    lin = np.ravel_multi_index(tuple(idx), dims)
    _, first = np.unique(lin, return_index=True)
    idx = idx[:, np.sort(first)]
    val = rng.random(idx.shape[1])
    p, v = build(orc, idx, val, dims, 1.0)
    A, B, C = orc.init_factors3(dims, R, 42)
    o = orc.Als3(v, None, None, float(np.sum(val * val)), dims, R, A, B, C, None)
    for _ in range(4):
        fit, _, _ = o.iterate(1)
        res, x2 = o.residual(True)
        # the Gram fit models every cell of the tensor; the exact residual only
        # the stored ones, so compare on the dense completion of the model
        Xh = np.einsum("r,ir,jr,kr->ijk", o.lam(), *(o.factor(m).reshape(dims[m], R)
                                                    for m in range(3)))
        X = dense_from(idx, val, dims)
        exact = 1.0 - np.linalg.norm(X - Xh) / np.linalg.norm(X)
        assert abs(fit[0] - exact) < 1e-10
        stored = Xh[tuple(idx)]
        assert abs(res - np.sum((val - stored) ** 2)) < 1e-9 * max(1.0, res)
        assert abs(x2 - np.sum(val * val)) < 1e-12 * x2
