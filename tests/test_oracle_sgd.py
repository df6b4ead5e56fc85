"""Pins the oracle's CP-SGD functions (sgd.cu:51-288) on the CPU.

sgd3_sample     the SplitMix64-finalised counter hash, restated with Python
                integers (64-bit wrap by masking)
sgd3_step       one element's gradient step = closed form; batch elements in
                order, each reading the rows as the previous ones left them
sgd3_normalize  column norms, 0 below 1e-14, lambda = norms
sgd3_loss       sum (v - sum_r lambda a b c)^2
"""
import numpy as np
import pytest

M64 = (1 << 64) - 1


def py_sample(seed, batch, nnz):
    out = []
    for b in range(batch):
        x = (seed + b * 0x9E3779B97F4A7C15) & M64
        x ^= x >> 30
        x = (x * 0xBF58476D1CE4E5B9) & M64
        x ^= x >> 27
        x = (x * 0x94D049BB133111EB) & M64
        x ^= x >> 31
        out.append(x % nnz)
    return np.array(out, np.uint32)


@pytest.mark.parametrize("seed,batch,nnz", [(42, 1000, 37806916), (43, 777, 1), (0, 513, 12345),
                                            ((1 << 64) - 3, 300, 2 ** 31 - 1)])
def test_sample_hash(orc, seed, batch, nnz):
    got = orc.sgd3_sample(seed, batch, nnz)
    assert np.array_equal(got, py_sample(seed, batch, nnz))
    assert got.max() < nnz


def packed(i, j, k):
    return (np.asarray(i, np.uint64) << np.uint64(30)) | (np.asarray(j, np.uint64) << np.uint64(15)) \
        | np.asarray(k, np.uint64)


def test_step_closed_form_distinct_rows(orc):
    rng = np.random.default_rng(1)
    R, n = 16, 50
    dims = (60, 70, 80)
    i, j, k = (rng.permutation(d)[:n] for d in dims)     # every row used once
    coords, vals = packed(i, j, k), rng.standard_normal(n)
    A, B, C = (rng.standard_normal((d, R)) for d in dims)
    lam = rng.random(R) + 0.5
    idx = rng.permutation(n).astype(np.uint32)
    g = 1e-2
    a, b, c = orc.sgd3_step(coords, vals, idx, A.ravel(), B.ravel(), C.ravel(), lam, R, g)
    e = vals - np.einsum("r,er,er,er->e", lam, A[i], B[j], C[k])
    A2, B2, C2 = A.copy(), B.copy(), C.copy()
    A2[i] += g * e[:, None] * B[j] * C[k]
    B2[j] += g * e[:, None] * A[i] * C[k]
    C2[k] += g * e[:, None] * A[i] * B[j]
    for got, ref in ((a, A2), (b, B2), (c, C2)):
        assert np.allclose(got.reshape(ref.shape), ref, rtol=1e-14, atol=1e-14)


def test_step_sequential_shared_rows(orc):
    """Two elements on the same rows: the second reads the first one's step."""
    R = 4
    rng = np.random.default_rng(2)
    A, B, C = (rng.standard_normal((2, R)) for _ in range(3))
    lam = np.ones(R)
    coords = packed([1, 1], [0, 0], [1, 1])
    vals = np.array([0.7, -0.3])
    idx = np.array([0, 1], np.uint32)
    g = 0.1
    a, b, c = orc.sgd3_step(coords, vals, idx, A.ravel(), B.ravel(), C.ravel(), lam, R, g)
    A2, B2, C2 = A.copy(), B.copy(), C.copy()
    for v in vals:
        x, y, z = A2[1].copy(), B2[0].copy(), C2[1].copy()
        e = v - np.sum(lam * x * y * z)
        A2[1] += g * e * y * z
        B2[0] += g * e * x * z
        C2[1] += g * e * x * y
    assert np.allclose(a.reshape(2, R), A2, rtol=1e-15, atol=1e-15)
    assert np.allclose(b.reshape(2, R), B2, rtol=1e-15, atol=1e-15)
    assert np.allclose(c.reshape(2, R), C2, rtol=1e-15, atol=1e-15)


def test_normalize_and_loss(orc):
    rng = np.random.default_rng(3)
    rows, R = 40, 6
    F = rng.standard_normal((rows, R))
    F[:, 2] = 0.0
    f, lam = orc.sgd3_normalize(F.ravel(), rows, R)
    n = np.linalg.norm(F, axis=0)
    assert np.allclose(lam, np.where(n < 1e-14, 0.0, n), rtol=1e-15)
    exp = np.where(n < 1e-14, 0.0, F / np.where(n < 1e-14, 1.0, n))
    assert np.allclose(f.reshape(rows, R), exp, rtol=1e-15, atol=1e-15)
    dims = (10, 11, 12)
    A, B, C = (rng.standard_normal((d, R)) for d in dims)
    i, j, k = (rng.integers(0, d, 30) for d in dims)
    vals = rng.standard_normal(30)
    idx = rng.integers(0, 30, 50).astype(np.uint32)
    loss = orc.sgd3_loss(packed(i, j, k), vals, idx, A.ravel(), B.ravel(), C.ravel(), lam, R)
    xh = np.einsum("r,er,er,er->e", lam, A[i], B[j], C[k])
    assert abs(loss - np.sum((vals[idx] - xh[idx]) ** 2)) <= 1e-12 * loss
