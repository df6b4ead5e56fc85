"""Pins the oracle's generic N-order path (oracle/cptc_oracle_nd.cpp,
generic.cu) against independent numpy restatements and closed forms.

reorder_nd  generic.cu:1180-1376  HITS scores with np.add.at (element-order sums),
                                  rank by lexsort(score desc, index asc); CADR by
                                  lexsort(degree desc, index asc); auto's probe
dense_nd    generic.cu:578-725    the splitbit hash of (tile, outer tuple) in python
                                  integers, counts, first-occurrence unit order
views_nd    generic.cu:1848-1958  stable argsort by the target coordinate
mttkrp_*    generic.cu:271-561    einsum on dense 4- and 5-order tensors
chol_solve  generic.cu:746-819    numpy Cholesky of FtF + eps I
als_nd      generic.cu:2032-2214  an independent numpy ALS (Gram fit formula)
"""
import numpy as np
import pytest

from conftest import rel_err

M64 = (1 << 64) - 1


def py_hash(x):
    x = (x + 0x9E3779B97F4A7C15) & M64
    x = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & M64
    x = ((x ^ (x >> 27)) * 0x94D049BB133111EB) & M64
    return x ^ (x >> 31)


def rand_nd(rng, dims, nnz, dup=False, zipf=None):
    cols = []
    for m, d in enumerate(dims):
        if zipf and zipf[m]:
            p = 1.0 / np.arange(1, d + 1) ** zipf[m]
            cols.append(rng.choice(d, nnz, p=p / p.sum()))
        else:
            cols.append(rng.integers(0, d, nnz))
    idx = np.stack(cols).astype(np.uint32)
    if not dup:
        lin = np.ravel_multi_index(tuple(idx.astype(np.int64)), dims)
        _, first = np.unique(lin, return_index=True)
        idx = idx[:, np.sort(first)]
    return np.ascontiguousarray(idx), rng.random(idx.shape[1]) + 0.5


def np_hits(idx, dims, rounds, stride=1):
    N = len(dims)
    s = [np.ones(d) for d in dims]
    sel = np.arange(0, idx.shape[1], stride)
    for _ in range(rounds):
        ns = []
        for m in range(N):
            p = np.ones(len(sel))
            for q in range(N):
                if q != m:
                    p = p * s[q][idx[q, sel]]
            acc = np.zeros(dims[m])
            np.add.at(acc, idx[m, sel], p)        # sequential, element order
            ns.append(acc)
        for m in range(N):
            mx = max(0.0, ns[m].max())
            s[m] = ns[m] / mx if mx > 0 else ns[m]
    ranks = []
    for m in range(N):
        order = np.lexsort((np.arange(dims[m]), -s[m]))
        r = np.empty(dims[m], np.uint32)
        r[order] = np.arange(dims[m])
        ranks.append(r)
    return ranks


@pytest.mark.parametrize("rounds,budget", [(1, 8000000), (3, 8000000), (3, 1000)])
def test_hits_matches_numpy(orc, rounds, budget):
    rng = np.random.default_rng(rounds)
    dims = (30, 12, 45, 20)
    idx, val = rand_nd(rng, dims, 5000, zipf=(0, 0, 1.2, 1.2))
    new, rank = orc.reorder_nd(idx, val, dims, "hits", rounds, budget)
    stride = idx.shape[1] // budget if idx.shape[1] > budget else 1
    ref = np_hits(idx, dims, rounds, stride)
    for m in range(4):
        assert np.array_equal(rank[m], ref[m]), m
        assert np.array_equal(new[m], ref[m][idx[m]])


def test_cadr_nd_and_none(orc):
    rng = np.random.default_rng(2)
    dims = (25, 40, 33)
    idx, val = rand_nd(rng, dims, 3000, zipf=(1.1, 0, 1.1))
    new, rank = orc.reorder_nd(idx, val, dims, "cadr", 3, 8000000)
    for m in range(3):
        deg = np.bincount(idx[m], minlength=dims[m])
        order = np.lexsort((np.arange(dims[m]), -deg))
        r = np.empty(dims[m], np.uint32)
        r[order] = np.arange(dims[m])
        assert np.array_equal(rank[m], r)
    same, rank0 = orc.reorder_nd(idx, val, dims, "none", 3, 8000000)
    assert len(rank0) == 0 and np.array_equal(same, idx)


def np_probe(idx, dims, ranks=None):
    N = len(dims)
    st = idx.shape[1] // 2000000 if idx.shape[1] > 2000000 else 1
    nbj, nbk = (dims[1] + 15) // 16, (dims[2] + 15) // 16
    cnt = {}
    for e in range(0, idx.shape[1], st):
        co = [int(ranks[m][idx[m, e]]) if ranks else int(idx[m, e]) for m in range(N)]
        tile = ((co[0] // 16) * nbj + co[1] // 16) * nbk + co[2] // 16
        o = 0
        for m in range(3, N):
            o = (o * 1000003 + co[m]) & M64
        k = py_hash(tile ^ ((o * 0x9E3779B97F4A7C15) & M64))
        cnt[k] = cnt.get(k, 0) + 1
    tiles = sum(1 for v in cnt.values() if v * st >= 122)
    inn = sum(v * st for v in cnt.values() if v * st >= 122)
    return inn / (tiles * 4096.0) if tiles else 0.0


def test_auto_reorder_follows_probe(orc):
    rng = np.random.default_rng(4)
    # a dense-ish tensor (probe fill high) and a hopeless one (probe fill ~0)
    dims = (32, 32, 32, 2)
    dense, dv = rand_nd(rng, dims, 30000)
    sparse, sv = rand_nd(rng, (4000, 4000, 4000, 2), 3000)
    for idx, val, d in ((dense, dv, dims), (sparse, sv, (4000, 4000, 4000, 2))):
        new, rank = orc.reorder_nd(idx, val, d, "auto", 3, 8000000)
        f_raw = np_probe(idx, d)
        if f_raw < 0.02:
            assert len(rank) == 0 and np.array_equal(new, idx)
            continue
        hits = np_hits(idx, d, 3)
        relab = np.stack([hits[m][idx[m]] for m in range(4)])
        f_hits = np_probe(relab, d, hits)      # the reference maps twice
        if f_hits >= 0.11:
            assert all(np.array_equal(rank[m], hits[m]) for m in range(4))
            assert np.array_equal(new, relab)
        else:
            assert len(rank) == 0 and np.array_equal(new, idx)


def np_dense_nd(idx, val, dims, thr, inner=(0, 1, 2)):
    N = len(dims)
    cutoff = int(4096.0 * thr)
    outer = [m for m in range(N) if m not in inner]
    keys = []
    for e in range(idx.shape[1]):
        a, b, c = (int(idx[m, e]) for m in inner)
        o = 0
        for m in outer:
            o = (o * 1000003 + int(idx[m, e])) & M64
        tile = ((a // 16) << 40) | ((b // 16) << 20) | (c // 16)
        keys.append(py_hash(tile ^ ((o * 0x9E3779B97F4A7C15) & M64)))
    cnt = {}
    for k in keys:
        cnt[k] = cnt.get(k, 0) + 1
    units, order = {}, []
    for e, k in enumerate(keys):
        if cnt[k] >= cutoff and k not in units:
            units[k] = len(order)
            order.append(e)
    members = [[] for _ in order]
    for e, k in enumerate(keys):
        if k in units:
            members[units[k]].append(e)
    return order, members


def clustered(rng, dims, inner, frac, nbg):
    """A half-filled 16^3 block on the inner modes at outer coordinate 0,
    plus uniform background."""
    N = len(dims)
    lo = [0, 0, 16]
    cells = np.array(np.meshgrid(*[np.arange(l, l + 16) for l in lo], indexing="ij"))
    cells = cells.reshape(3, -1)[:, rng.random(4096) < frac]
    clus = np.zeros((N, cells.shape[1]), np.uint32)
    for s, m in enumerate(inner):
        clus[m] = cells[s]
    bg, _ = rand_nd(rng, dims, nbg)
    return np.ascontiguousarray(np.concatenate([clus, bg], axis=1))


@pytest.mark.parametrize("N,thr,inner", [(4, 0.03, (0, 1, 2)), (5, 0.01, (0, 1, 2)),
                                         (4, 0.0001, (0, 1, 2)), (4, 0.03, (1, 2, 3)),
                                         (5, 0.03, (0, 2, 4))])
def test_dense_nd_matches_python(orc, N, thr, inner):
    rng = np.random.default_rng(N)
    dims = (40, 35, 48, 33, 34)[:N]
    idx = clustered(rng, dims, inner, 0.3, 2000)
    val = rng.random(idx.shape[1])
    u = orc.dense_nd(idx, val, dims, thr, inner)
    order, members = np_dense_nd(idx, val, dims, thr, inner)
    outer = [m for m in range(N) if m not in inner]
    assert len(u["unit6"]) == len(order) and len(order) > 0
    off = 0
    for k, (e0, mem) in enumerate(zip(order, members)):
        row = u["unit6"][k]
        assert list(row[:3]) == [idx[m, e0] // 16 for m in inner]
        assert row[3] == len(mem) and row[4] == off and row[5] == k * (N - 3)
        a, b, c = inner
        lid = [(idx[a, e] % 16) * 256 + (idx[b, e] % 16) * 16 + idx[c, e] % 16 for e in mem]
        assert u["lid"][off:off + len(mem)].tolist() == lid
        assert u["val"][off:off + len(mem)].tolist() == val[mem].tolist()
        assert u["outer_coords"][k * (N - 3):(k + 1) * (N - 3)].tolist() == \
            [int(idx[m, e0]) for m in outer]
        off += len(mem)
    flags = np.zeros(idx.shape[1], np.uint8)
    for mem in members:
        flags[mem] = 1
    assert np.array_equal(u["is_dense"], flags)


def test_views_nd_matches_numpy(orc):
    rng = np.random.default_rng(7)
    dims = (3, 50, 2000, 7)
    idx, val = rand_nd(rng, dims, 9000, dup=True)
    isd = (rng.random(idx.shape[1]) < 0.2).astype(np.uint8)
    v = orc.views_nd(idx, val, dims, isd, True)
    for n in range(4):
        order = np.argsort(idx[n], kind="stable")
        others = [m for m in range(4) if m != n]
        assert np.array_equal(v[n]["scoords"].reshape(3, -1), idx[others][:, order])
        assert np.array_equal(v[n]["vals"], val[order])
        assert np.array_equal(v[n]["skip"], isd[order])
        rows, starts, counts = np.unique(idx[n][order], return_index=True, return_counts=True)
        br, bs, bc, sg = [], [], [], []
        for r, s, c in zip(rows, starts, counts):
            for c0 in range(0, c, 1024):
                br.append(r); bs.append(s + c0); bc.append(min(1024, c - c0))
                sg.append(0 if n < 3 else int(c <= 1024))
        assert v[n]["row"].tolist() == br and v[n]["start"].tolist() == bs
        assert v[n]["cnt"].tolist() == bc and v[n]["single"].tolist() == sg


def dense_of(idx, val, dims):
    X = np.zeros(dims)
    np.add.at(X, tuple(idx.astype(np.int64)), val)
    return X


def einsum_mttkrp(X, F, n):
    N = X.ndim
    letters = "abcdefg"[:N]
    spec = letters + "," + ",".join(letters[m] + "r" for m in range(N) if m != n) + \
        "->" + letters[n] + "r"
    return np.einsum(spec, X, *[F[m] for m in range(N) if m != n], optimize=True)


@pytest.mark.parametrize("N,R,inner", [(4, 8, (0, 1, 2)), (4, 16, (0, 1, 2)),
                                       (5, 32, (0, 1, 2)), (3, 5, (0, 1, 2)),
                                       (4, 8, (1, 2, 3)), (4, 8, (0, 2, 3)),
                                       (5, 16, (1, 3, 4))])
def test_mttkrp_nd_closed_form(orc, N, R, inner):
    rng = np.random.default_rng(N * 10 + R)
    dims = (40, 30, 36, 33, 34)[:N]
    idx = clustered(rng, dims, inner, 0.5, 3000)
    # duplicates: repeat a few elements
    idx = np.ascontiguousarray(np.concatenate([idx, idx[:, :50]], axis=1))
    val = rng.standard_normal(idx.shape[1])
    F = [rng.random((d, R)) for d in dims]
    X = dense_of(idx, val, dims)
    enabled = N >= 4
    u = orc.dense_nd(idx, val, dims, 0.03, inner) if enabled else None
    if enabled:
        assert len(u["unit6"]) > 0
    isd = u["is_dense"] if enabled else None
    v = orc.views_nd(idx, val, dims, isd, enabled, inner)
    for n in range(N):
        is_inner = enabled and n in inner
        if enabled:
            assert all(v[n]["single"] == 0) or not is_inner
        out = np.zeros(dims[n] * R)
        if is_inner:
            out = orc.mttkrp_units_nd(idx, val, dims, u, n, [f.ravel() for f in F], R)
        out = orc.mttkrp_seg_nd(idx, val, dims, v, n, is_inner, [f.ravel() for f in F], R, out)
        assert rel_err(out.reshape(dims[n], R), einsum_mttkrp(X, F, n)) < 1e-12, n


def test_chol_solve_nd(orc):
    rng = np.random.default_rng(3)
    R = 16
    A = rng.random((40, R))
    FtF = A.T @ A
    Y = rng.standard_normal((100, R))
    got = orc.chol_solve_nd(FtF.ravel(), Y.ravel(), R).reshape(100, R)
    eps = 1e-12 * np.trace(FtF) / R + 1e-300
    L = np.linalg.cholesky(FtF + eps * np.eye(R))
    ref = np.linalg.solve(L.T, np.linalg.solve(L, Y.T)).T
    assert rel_err(got, ref) < 1e-11


def np_als_nd(X, F, iters):
    N = X.ndim
    R = F[0].shape[1]
    F = [f.copy() for f in F]
    lam = np.ones(R)
    X2 = np.sum(X * X)
    fits = []
    for _ in range(iters):
        for n in range(N):
            FtF = np.ones((R, R))
            for m in range(N):
                if m != n:
                    FtF = FtF * (F[m].T @ F[m])
            M = einsum_mttkrp(X, F, n)
            eps = 1e-12 * (np.trace(FtF) / R if np.trace(FtF) > 0 else 1.0) + 1e-300
            Fn = np.linalg.solve(FtF + eps * np.eye(R), M.T).T
            nr = np.sqrt(np.sum(Fn * Fn, axis=0))
            nr = np.where(~np.isfinite(nr) | (nr < 1e-14), 1.0, nr)
            F[n] = Fn / nr
            lam = nr
        model2 = np.sum(np.outer(lam, lam) * np.prod([F[m].T @ F[m] for m in range(N)], axis=0))
        iprod = np.sum(lam * np.sum(F[N - 1] * M, axis=0))
        fits.append(1 - np.sqrt(max(X2 - 2 * iprod + model2, 0)) / np.sqrt(X2))
    return np.array(fits), F, lam


@pytest.mark.parametrize("dense", [False, True])
def test_als_nd_matches_numpy(orc, dense):
    rng = np.random.default_rng(9)
    dims = (36, 20, 34, 3)
    R = 6
    cells = np.array(np.meshgrid(np.arange(16), np.arange(16), np.arange(16), indexing="ij"))
    cells = cells.reshape(3, -1)[:, rng.random(4096) < 0.4]
    clus = np.concatenate([cells, np.full((1, cells.shape[1]), 2)])
    bg, _ = rand_nd(rng, dims, 2500)
    idx = np.concatenate([clus.astype(np.uint32), bg], axis=1)
    lin = np.ravel_multi_index(tuple(idx.astype(np.int64)), dims)
    _, first = np.unique(lin, return_index=True)
    idx = np.ascontiguousarray(idx[:, np.sort(first)])
    val = rng.random(idx.shape[1]) + 0.1
    fits, ip, m2, F, lam = orc.als_nd(idx, val, dims, [], R, 42, False, dense, 0.03, 5)
    # initial factors: mt19937(42) in mode order (no reordering applied)
    bg2 = np.random.MT19937()
    bg2._legacy_seeding(42)
    raw = bg2.random_raw(2 * sum(dims) * R).astype(np.float64)
    u01 = (raw[0::2] + raw[1::2] * 2.0 ** 32) / 2.0 ** 64
    F0, o = [], 0
    for d in dims:
        F0.append(u01[o:o + d * R].reshape(d, R))
        o += d * R
    rfits, rF, rlam = np_als_nd(dense_of(idx, val, dims), F0, 5)
    assert np.max(np.abs(fits - rfits)) < 1e-9
    for m in range(4):
        assert rel_err(F[m].reshape(dims[m], R), rF[m]) < 1e-7
    res = orc.residual_nd(idx, val, dims, F, lam, R)
    Xh = np.einsum("r,ar,br,cr,dr->abcd", lam, *[f.reshape(d, R) for f, d in zip(F, dims)])
    assert abs(res - np.sum((val - Xh[tuple(idx.astype(np.int64))]) ** 2)) < 1e-9 * max(res, 1)


def test_selftest_tensor_shape(orc):
    idx, val, dims, F = orc.selftest_tensor()
    assert dims == (40, 24, 36, 3) and idx.shape[0] == 4 and idx.shape[1] == len(val)
    assert 4000 < len(val) < 3 * 2 * 4096 + 3 * 8 * 8 * 4 + 4000
    assert all(len(F[m]) == dims[m] * 8 for m in range(4))
    assert np.all(idx.max(axis=1) < np.array(dims))


def np_selftest_tensor():
    """generic.cu:1389-1441 restated with numpy's MT19937 (legacy seeding =
    std::mt19937(1234)) and libstdc++'s generate_canonical<double, 53> (two
    32-bit draws per double). The residual scatter's push(...) arguments draw
    right to left: that is g++'s order for this call (the reference's nvcc host
    pass compiles it with g++), so the value is drawn first and i last."""
    bg = np.random.MT19937()
    bg._legacy_seeding(1234)
    buf = []

    def uv():
        if not buf:
            raw = bg.random_raw(2 * 4096).astype(np.float64)
            buf.extend(((raw[0::2] + raw[1::2] * 2.0 ** 32) / 2.0 ** 64).tolist()[::-1])
        return buf.pop()

    dims = (40, 24, 36, 3)
    co, vals = [[], [], [], []], []

    def push(c, v):
        for m in range(4):
            co[m].append(c[m])
        vals.append(v)

    for l in range(dims[3]):
        for t in ((0, 0, 0), (1, 0, 1)):
            for a in range(16):
                for b in range(16):
                    for c in range(16):
                        if uv() < 0.5:
                            push((t[0] * 16 + a, t[1] * 16 + b, t[2] * 16 + c, l), 1.0 + uv())
    for l in range(dims[3]):
        for a in range(32, dims[0]):
            for b in range(16, dims[1]):
                for c in range(32, dims[2]):
                    if uv() < 0.6:
                        push((a, b, c, l), 1.0 + uv())
    for _ in range(4000):
        d = [uv() for _ in range(5)][::-1]        # right-to-left argument evaluation
        push(tuple(int(d[m] * dims[m]) % dims[m] for m in range(4)), 1.0 + d[4])
    F = [np.array([uv() for _ in range(dims[m] * 8)]) for m in range(4)]
    return np.array(co, np.uint32), np.array(vals), dims, F


def test_selftest_tensor_mt19937(orc):
    idx, val, dims, F = orc.selftest_tensor()
    ridx, rval, rdims, rF = np_selftest_tensor()
    assert tuple(dims) == rdims
    assert np.array_equal(idx, ridx)
    assert np.array_equal(val, rval)
    for m in range(4):
        assert np.array_equal(np.asarray(F[m]), rF[m])
