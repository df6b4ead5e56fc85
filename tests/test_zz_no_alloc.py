"""cptc_solve_pinv_noalloc: the allocation-free variant of cptc_solve_pinv
(workspace in a static device array) gives the same result, bit for bit, on
consecutive calls with different sizes and on both solve paths."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _spd(rng, R):
    Fa, Fb = rng.random((3 * R + 20, R)), rng.random((2 * R + 30, R))
    return (Fa.T @ Fa) * (Fb.T @ Fb)


def _kahan(R):
    L = np.eye(R) + np.tril(np.full((R, R), -1.0), -1)
    return L @ L.T


def _solve(ca, fn, A, Y, lam):
    R = A.shape[0]
    dA, dY, dl = (ca.DevBuf.from_numpy(np.ascontiguousarray(x)) for x in (A, Y, lam))
    out = ca.DevBuf.zeros(Y.shape)
    rc = fn(dA.data_ptr(), dY.data_ptr(), out.data_ptr(), Y.shape[0], R, dl.data_ptr(), None)
    assert rc == 0, ca.lib.cptc_last_error()
    ca.sync()
    return out.numpy()


@pytest.mark.parametrize("first,second", [((128, 5000, "spd"), (32, 700, "spd")),
                                          ((64, 3000, "kahan"), (16, 100, "spd")),
                                          ((128, 2000, "kahan"), (100, 1500, "kahan"))])
def test_noalloc_matches_solve_pinv(ca, dev, first, second):
    rng = np.random.default_rng(first[0] + second[0])
    for R, dim, kind in (first, second):
        A = _spd(rng, R) if kind == "spd" else _kahan(R)
        Y = rng.standard_normal((dim, R))
        lam = rng.random(R) + 0.5
        ref = _solve(ca, ca.lib.cptc_solve_pinv, A, Y, lam)
        got = _solve(ca, ca.lib.cptc_solve_pinv_noalloc, A, Y, lam)
        assert np.array_equal(got, ref), (R, dim, kind)
        assert np.all(np.isfinite(got))


def test_noalloc_rejects_large_rank(ca, dev):
    R, dim = 129, 10
    A = np.eye(R)
    Y = np.zeros((dim, R))
    dA, dY = ca.DevBuf.from_numpy(A), ca.DevBuf.from_numpy(Y)
    out = ca.DevBuf.zeros((dim, R))
    rc = ca.lib.cptc_solve_pinv_noalloc(dA.data_ptr(), dY.data_ptr(), out.data_ptr(), dim, R,
                                        None, None)
    assert rc != 0 and b"exceeds the allocation-free maximum" in ca.lib.cptc_last_error()
