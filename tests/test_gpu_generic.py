"""Generic N-order path on the GPU, through the C ABI, against the CPU oracle
(oracle/cptc_oracle_nd.cpp) and numpy closed forms.

Bars: layout (reorder, dense units, views) bit-exact; FP64 segment MTTKRP
<= 1e-10 relative; dense-unit MTTKRP (FP32 MFMA, FP64 epilogue) <= 1e-5
relative to FP64; ridge Cholesky <= 1e-11; fit within 1e-4 of the oracle
after 20 iterations (1e-8 when no dense units are involved).
"""
import ctypes as C
import os
import subprocess

import numpy as np
import pytest

from conftest import rel_err

pytestmark = pytest.mark.gpu


def dbuf(ca, a):
    return ca.DevBuf.from_numpy(np.ascontiguousarray(a))


def fptrs(bufs):
    return (C.c_void_p * len(bufs))(*[b.data_ptr() for b in bufs])


def clustered(rng, dims, inner, frac, nbg, outer_at=0):
    """Half-filled 16^3 blocks on the inner modes (one per outer value 0..1)
    plus uniform background, duplicates removed, element order shuffled."""
    N = len(dims)
    parts = []
    for o in range(2):
        cells = np.array(np.meshgrid(np.arange(16), np.arange(16), np.arange(16, 32),
                                     indexing="ij")).reshape(3, -1)
        cells = cells[:, rng.random(4096) < frac]
        blk = np.zeros((N, cells.shape[1]), np.int64)
        for s, m in enumerate(inner):
            blk[m] = cells[s] % dims[m]
        for m in range(N):
            if m not in inner:
                blk[m] = (outer_at + o) % dims[m]
        parts.append(blk)
    parts.append(np.stack([rng.integers(0, d, nbg) for d in dims]))
    idx = np.concatenate(parts, axis=1)
    lin = np.ravel_multi_index(tuple(idx), dims)
    _, first = np.unique(lin, return_index=True)
    idx = idx[:, np.sort(first)]
    idx = idx[:, rng.permutation(idx.shape[1])]
    return np.ascontiguousarray(idx.astype(np.uint32))


def tensor(ca, idx, dims, rng):
    return ca.Tensor(tuple(dims), idx, rng.random(idx.shape[1]) + 0.25)


# ------------------------------------------------------------ layout parity --

@pytest.mark.parametrize("N,inner,how", [(4, (0, 1, 2), "hits"), (5, (0, 1, 2), "hits"),
                                         (4, (1, 2, 3), "cadr"), (5, (0, 2, 4), "none")])
def test_layout_bit_exact(ca, orc, dev, N, inner, how):
    rng = np.random.default_rng(N)
    dims = (40, 35, 48, 33, 20)[:N]
    t = tensor(ca, clustered(rng, dims, inner, 0.4, 6000), dims, rng)
    g = ca.Gen(t, R=8, reorder=how, inner=inner)
    ref_idx, ref_rank = orc.reorder_nd(t.idx, t.val, dims, how, 3, 8000000)
    assert np.array_equal(g.coords(), ref_idx)
    for m in range(N):
        exp = ref_rank[m] if len(ref_rank) else np.arange(dims[m])
        assert np.array_equal(g.rank(m), exp)
    u = orc.dense_nd(ref_idx, t.val, dims, 0.03, inner)
    got = g.units()
    assert g.info.dense_enabled == 1 and int(g.info.n_units) == len(u["unit6"]) > 0
    assert int(g.info.cutoff) == u["cutoff"]
    for k in ("unit6", "outer_coords", "lid", "val", "is_dense"):
        assert np.array_equal(got[k], np.asarray(u[k]).reshape(got[k].shape)), k
    views = orc.views_nd(ref_idx, t.val, dims, u["is_dense"], True, inner)
    for n in range(N):
        v = g.view(n)
        ref = views[n]
        assert np.array_equal(v["scoords"].ravel(), ref["scoords"]), n
        assert np.array_equal(v["vals"], ref["vals"])
        assert np.array_equal(v["skip"], ref["skip"])
        for k in ("row", "start", "cnt", "single"):
            assert np.array_equal(v[k], ref[k]), (n, k)


def test_layout_no_dense_for_order3_and_threshold0(ca, orc, dev):
    rng = np.random.default_rng(3)
    dims = (40, 35, 48)
    t = tensor(ca, clustered(rng, dims, (0, 1, 2), 0.4, 3000), dims, rng)
    g = ca.Gen(t, R=4)
    assert g.info.dense_enabled == 0 and g.info.reorder.decode() == "cadr"
    views = orc.views_nd(g.coords(), t.val, dims, None, False)
    for n in range(3):
        assert np.array_equal(g.view(n)["single"], views[n]["single"])
    dims4 = (40, 35, 48, 2)
    t4 = tensor(ca, clustered(rng, dims4, (0, 1, 2), 0.4, 3000), dims4, rng)
    g4 = ca.Gen(t4, R=4, threshold=0.0)
    assert g4.info.dense_enabled == 0


def zipf_tensor(ca, rng, dims, nnz, zipf):
    cols = []
    for m, d in enumerate(dims):
        if zipf[m]:
            p = 1.0 / np.arange(1, d + 1) ** zipf[m]
            cols.append(rng.choice(d, nnz, p=p / p.sum()))
        else:
            cols.append(rng.integers(0, d, nnz))
    return ca.Tensor(tuple(dims), np.ascontiguousarray(np.stack(cols).astype(np.uint32)),
                     rng.random(nnz) + 0.5)


@pytest.mark.parametrize("how,rounds,budget", [("hits", 3, 8000000), ("hits", 1, 8000000),
                                               ("hits", 3, 777), ("cadr", 3, 8000000),
                                               ("none", 3, 8000000), ("bogus", 3, 8000000),
                                               (None, 3, 8000000)])
def test_device_reorder_matches_oracle(ca, orc, dev, how, rounds, budget):
    """The driver's device reordering (sampled HITS, CADR, none, unknown ->
    cadr, default by order) against the oracle, bit for bit."""
    rng = np.random.default_rng(11)
    t = zipf_tensor(ca, rng, (60, 20, 300, 45), 20000, (1.1, 0, 1.2, 1.0))
    g = ca.Gen(t, R=4, reorder=how, rounds=rounds, sample=budget, dense=False)
    ohow = {"bogus": "cadr", None: "hits"}.get(how, how)
    ref_idx, ref_rank = orc.reorder_nd(t.idx, t.val, t.dims, ohow, rounds, budget)
    assert g.info.reorder.decode() == ohow
    assert np.array_equal(g.coords(), ref_idx)
    for m in range(4):
        exp = ref_rank[m] if len(ref_rank) else np.arange(t.dims[m])
        assert np.array_equal(g.rank(m), exp), m


def test_device_reorder_auto_both_branches(ca, orc, dev):
    rng = np.random.default_rng(5)
    dense = zipf_tensor(ca, rng, (32, 32, 32, 2), 30000, (0, 0, 0, 0))
    sparse = zipf_tensor(ca, rng, (5000, 5000, 5000, 2), 3000, (0, 0, 0, 0))
    outcomes = set()
    for t in (dense, sparse):
        g = ca.Gen(t, R=4, reorder="auto", dense=False)
        ref_idx, ref_rank = orc.reorder_nd(t.idx, t.val, t.dims, "auto", 3, 8000000)
        assert np.array_equal(g.coords(), ref_idx)
        applied = g.info.reorder.decode() == "hits"
        assert applied == (len(ref_rank) > 0)
        if applied:
            assert all(np.array_equal(g.rank(m), ref_rank[m]) for m in range(4))
        outcomes.add(applied)
    assert outcomes == {True, False}


def test_device_reorder_config5_sampled(ca, orc, dev):
    """Config 5 (20 M elements): HITS over every second element (stride 2),
    rows of up to ~1.3 M terms summed in element order."""
    t = ca.synth_config(5)
    g = ca.Gen(t, R=2, dense=False)
    ref_idx, ref_rank = orc.reorder_nd(t.idx, t.val, t.dims, "hits", 3, 8000000)
    for m in range(5):
        assert np.array_equal(g.rank(m), ref_rank[m]), m
    assert np.array_equal(g.coords(), ref_idx)


# ------------------------------------------------------------ kernel parity --

@pytest.mark.parametrize("N,R", [(2, 5), (3, 16), (4, 1), (4, 3), (4, 8), (4, 16), (5, 31),
                                 (5, 32), (6, 16), (8, 8)])
def test_seg_kernel_vs_oracle(ca, orc, dev, N, R):
    rng = np.random.default_rng(N * 100 + R)
    dims = (70, 9, 300, 40, 25, 6, 11, 13)[:N]
    nnz = 40000
    idx = np.ascontiguousarray(np.stack([rng.integers(0, d, nnz) for d in dims]).astype(np.uint32))
    idx[:, -2000:] = idx[:, :2000]               # duplicates
    val = rng.standard_normal(nnz)
    isd = (rng.random(nnz) < 0.3).astype(np.uint8)
    views = orc.views_nd(idx, val, dims, isd, True)
    F = [rng.standard_normal((d, R)) for d in dims]
    dF = [dbuf(ca, f) for f in F]
    for n in range(N):
        v = views[n]
        bufs = {k: dbuf(ca, v[k]) for k in ("scoords", "vals", "skip", "row", "start", "cnt",
                                            "single")}
        for use_skip in (False, True):
            init = rng.standard_normal(dims[n] * R)
            out = dbuf(ca, init.copy())
            rc = ca.lib.cptc_mttkrp_seg_nd(
                N, n, bufs["scoords"].data_ptr(), None, bufs["vals"].data_ptr(),
                bufs["skip"].data_ptr() if use_skip else None, nnz, bufs["row"].data_ptr(),
                bufs["start"].data_ptr(), bufs["cnt"].data_ptr(), bufs["single"].data_ptr(),
                len(v["row"]), fptrs(dF), out.data_ptr(), R, None)
            assert rc == 0, ca.lib.cptc_last_error()
            ca.sync()
            ref = orc.mttkrp_seg_nd(idx, val, dims, views, n, use_skip,
                                    [f.ravel() for f in F], R, init.copy())
            assert rel_err(out.numpy(), ref) <= 1e-10, (n, use_skip)


def test_seg_kernel_single_store(ca, orc, dev):
    """single segments store (overwrite), the others accumulate."""
    rng = np.random.default_rng(1)
    dims = (30, 20, 10, 5)
    nnz = 3000
    idx = np.ascontiguousarray(np.stack([rng.integers(0, d, nnz) for d in dims]).astype(np.uint32))
    val = rng.random(nnz)
    views = orc.views_nd(idx, val, dims, None, False)
    F = [rng.random((d, 8)) for d in dims]
    dF = [dbuf(ca, f) for f in F]
    n = 3
    v = views[n]
    assert v["single"].all()          # every row fits one segment
    bufs = {k: dbuf(ca, v[k]) for k in ("scoords", "vals", "row", "start", "cnt", "single")}
    init = np.full(dims[n] * 8, 7.0)
    out = dbuf(ca, init.copy())
    assert ca.lib.cptc_mttkrp_seg_nd(4, n, bufs["scoords"].data_ptr(), None,
                                     bufs["vals"].data_ptr(), None, nnz, bufs["row"].data_ptr(), bufs["start"].data_ptr(),
                                     bufs["cnt"].data_ptr(), bufs["single"].data_ptr(),
                                     len(v["row"]), fptrs(dF), out.data_ptr(), 8, None) == 0
    ca.sync()
    ref = orc.mttkrp_seg_nd(idx, val, dims, views, n, False, [f.ravel() for f in F], 8,
                            init.copy())
    assert rel_err(out.numpy(), ref) <= 1e-12


def seg_table(rows, limit=1024):
    """Row segments of a row-sorted view (<= limit elements; single when the
    row has one segment), as the view builders make them."""
    urow, start, cnt = np.unique(rows, return_index=True, return_counts=True)
    seg = [(r, s + o, min(limit, c - o), c <= limit)
           for r, s, c in zip(urow, start, cnt) for o in range(0, c, limit)]
    return [np.array([x[k] for x in seg], dt) for k, dt in
            ((0, np.uint32), (1, np.uint32), (2, np.uint32), (3, np.uint8))]


@pytest.mark.parametrize("N,R,dims,order", [
    (2, 8, (300, 5000), "runs"), (3, 32, (70, 9, 300), "runs"), (3, 16, (70, 9, 300), "shuffled"),
    (4, 2, (40, 3, 300, 2), "runs"), (4, 16, (183, 24, 1140, 1717), "runs"),
    (5, 32, (64, 64, 64, 32, 16), "runs"), (5, 32, (64, 64, 64, 32, 16), "shuffled"),
    (5, 30, (5000, 70000, 9, 300, 40), "runs"), (6, 8, (70, 9, 300, 40, 25, 6), "runs"),
    (8, 16, (70, 9, 30, 40, 25, 6, 11, 13), "runs")])
def test_seg_keys_kernel_vs_closed_form(ca, dev, N, R, dims, order):
    """The packed-key segment kernel against sum_e v_e prod F (numpy), on
    views sorted by row then levels (runs) and with rows in random element
    order; 4- and 8-byte keys; levels by dimension, not mode order."""
    rng = np.random.default_rng(N * 1000 + R)
    nnz = 60000
    # skewed coordinates so that rows exceed one segment and runs repeat
    idx = np.stack([np.minimum((rng.pareto(1.2, nnz) * d / 8).astype(np.int64), d - 1)
                    for d in dims]).astype(np.uint32)
    idx[:, -3000:] = idx[:, :3000]               # duplicates
    val = rng.standard_normal(nnz)
    F = [rng.standard_normal((d, R)) for d in dims]
    dF = [dbuf(ca, f) for f in F]
    kinds = set()
    for n in range(N):
        lev = sorted([m for m in range(N) if m != n], key=lambda m: dims[m])
        bits = [max(1, int(dims[m] - 1).bit_length()) for m in lev]
        kb = ca.lib.cptc_level_key_bytes(len(lev), (C.c_int * len(lev))(*bits))
        assert kb == (4 if sum(bits) <= 32 else 8)
        if order == "runs":
            perm = np.lexsort(tuple(idx[m] for m in reversed(lev)) + (idx[n],))
        else:
            perm = np.argsort(idx[n], kind="stable")
        rows = idx[n][perm]
        sc = np.ascontiguousarray(np.stack([idx[m][perm] for m in lev]))
        srow, sst, scnt, ssingle = seg_table(rows)
        b = {k: dbuf(ca, a) for k, a in (("sc", sc), ("val", val[perm]), ("row", srow),
                                         ("st", sst), ("cnt", scnt), ("single", ssingle))}
        keys = ca.DevBuf.zeros(nnz * kb // 8 + 1)
        lb = (C.c_int * len(lev))(*bits)
        assert ca.lib.cptc_pack_level_keys(len(lev), b["sc"].data_ptr(), nnz, lb,
                                           keys.data_ptr(), kb, None) == 0
        init = rng.standard_normal((dims[n], R))
        out = dbuf(ca, init.copy())
        rc = ca.lib.cptc_mttkrp_seg_nd_keys(
            N, n, keys.data_ptr(), kb, (C.c_int * len(lev))(*lev), lb, b["val"].data_ptr(), nnz,
            b["row"].data_ptr(), b["st"].data_ptr(), b["cnt"].data_ptr(), b["single"].data_ptr(),
            len(srow), fptrs(dF), out.data_ptr(), R, None)
        assert rc == 0, ca.lib.cptc_last_error()
        ca.sync()
        contrib = val[:, None] * np.prod([F[m][idx[m]] for m in range(N) if m != n], axis=0)
        M = np.zeros((dims[n], R))
        np.add.at(M, idx[n], contrib)
        exp = init.copy()
        for r, single in zip(srow, ssingle):
            exp[r] = M[r] if single else init[r]
        multi = np.unique(srow[ssingle == 0])
        exp[multi] += M[multi]
        kinds |= set(ssingle.tolist())
        assert rel_err(out.numpy().reshape(dims[n], R), exp) <= 1e-10, (n, order)
    assert kinds == {0, 1}, "both store and atomic rows exercised"


@pytest.mark.parametrize("N,R,dims,rev", [(2, 32, (9000, 90), False),
                                          (3, 8, (20000, 100, 200), False),
                                          (4, 32, (8000, 40, 30, 20), False),
                                          (4, 32, (8000, 40, 30, 20), True),
                                          (5, 16, (8000, 64, 64, 32, 16), False),
                                          (5, 16, (8000, 64, 64, 32, 16), True),
                                          (2, 32, (9000, 250), False),
                                          (4, 16, (3000, 24, 1140, 1717), False)])
def test_seg_keys_leaf_lds(ca, dev, N, R, dims, rev):
    """The dims variant (last level's factor staged in LDS, persistent grid)
    against the closed form and against the global-gather variant, on mode 0
    with thousands of segments: the first four shapes' leaf factors fit 24 KB
    (LDS path; the second has 4-byte keys), the last two do not.  rev: levels
    in descending dimension order, so the leaf is the smallest factor and
    the non-leaf levels are larger than it."""
    rng = np.random.default_rng(N * 31 + R)
    nnz = 400000
    idx = np.stack([np.minimum((rng.pareto(1.1, nnz) * d / 6).astype(np.int64), d - 1)
                    for d in dims]).astype(np.uint32)
    val = rng.standard_normal(nnz)
    F = [rng.standard_normal((d, R)) for d in dims]
    dF = [dbuf(ca, f) for f in F]
    n = 0
    lev = sorted(range(1, N), key=lambda m: dims[m], reverse=rev)
    bits = [max(1, int(dims[m] - 1).bit_length()) for m in lev]
    lb = (C.c_int * len(lev))(*bits)
    kb = ca.lib.cptc_level_key_bytes(len(lev), lb)
    perm = np.lexsort(tuple(idx[m] for m in reversed(lev)) + (idx[n],))
    sc = np.ascontiguousarray(np.stack([idx[m][perm] for m in lev]))
    srow, sst, scnt, ssingle = seg_table(idx[n][perm])
    assert len(srow) >= 2048 and set(ssingle.tolist()) == {0, 1}
    b = {k: dbuf(ca, a) for k, a in (("sc", sc), ("val", val[perm]), ("row", srow),
                                     ("st", sst), ("cnt", scnt), ("single", ssingle))}
    keys = ca.DevBuf.zeros(nnz * kb // 8 + 1)
    assert ca.lib.cptc_pack_level_keys(len(lev), b["sc"].data_ptr(), nnz, lb, keys.data_ptr(),
                                       kb, None) == 0
    init = rng.standard_normal((dims[n], R))
    outs = []
    for with_dims in (False, True):
        out = dbuf(ca, init.copy())
        args = [N, n, keys.data_ptr(), kb, (C.c_int * len(lev))(*lev), lb, b["val"].data_ptr(),
                nnz, b["row"].data_ptr(), b["st"].data_ptr(), b["cnt"].data_ptr(),
                b["single"].data_ptr(), len(srow), fptrs(dF)]
        if with_dims:
            rc = ca.lib.cptc_mttkrp_seg_nd_keys_dims(*args, (C.c_uint64 * N)(*dims),
                                                     out.data_ptr(), R, None)
        else:
            rc = ca.lib.cptc_mttkrp_seg_nd_keys(*args, out.data_ptr(), R, None)
        assert rc == 0, ca.lib.cptc_last_error()
        ca.sync()
        outs.append(out.numpy().reshape(dims[n], R))
    contrib = val[:, None] * np.prod([F[m][idx[m]] for m in range(1, N)], axis=0)
    M = np.zeros((dims[n], R))
    np.add.at(M, idx[n], contrib)
    exp = init.copy()
    exp[srow[ssingle == 1]] = M[srow[ssingle == 1]]
    multi = np.unique(srow[ssingle == 0])
    exp[multi] += M[multi]
    assert rel_err(outs[1], exp) <= 1e-10
    assert rel_err(outs[1], outs[0]) <= 1e-13


@pytest.mark.parametrize("kern", ["fp32", "bf16x3", "bf16x3c"])
@pytest.mark.parametrize("N,R,inner,G", [(4, 8, (0, 1, 2), 0), (4, 16, (0, 1, 2), 4),
                                         (5, 32, (0, 1, 2), 16), (4, 20, (1, 2, 3), 0),
                                         (4, 8, (0, 2, 3), 2), (5, 16, (1, 3, 4), 16),
                                         (4, 3, (0, 1, 3), 0)])
def test_units_kernel_vs_oracle(ca, orc, dev, N, R, inner, G, kern):
    rng = np.random.default_rng(N * 7 + R)
    dims = (40, 30, 36, 33, 34)[:N]
    idx = clustered(rng, dims, inner, 0.5, 3000)
    idx = np.ascontiguousarray(np.concatenate([idx, idx[:, :60]], axis=1))   # duplicates
    val = rng.standard_normal(idx.shape[1])
    u = orc.dense_nd(idx, val, dims, 0.02, inner)
    nu = len(u["unit6"])
    assert nu > 0
    F = [rng.random((d, R)) for d in dims]
    dF = [dbuf(ca, f) for f in F]
    d6 = dbuf(ca, np.ascontiguousarray(u["unit6"], np.uint32))
    dlid, dval = dbuf(ca, u["lid"]), dbuf(ca, u["val"])
    doc = dbuf(ca, u["outer_coords"] if len(u["outer_coords"]) else np.zeros(1, np.uint32))
    tiles = ca.DevBuf.zeros((nu, 4096), np.float32)
    W = ca.DevBuf.zeros((nu, R), np.float64)
    assert ca.lib.cptc_units_pack_nd(d6.data_ptr(), nu, dlid.data_ptr(), dval.data_ptr(),
                                     tiles.data_ptr(), None) == 0
    outer = [m for m in range(N) if m not in inner]
    om = (C.c_int * max(len(outer), 1))(*outer)
    assert ca.lib.cptc_units_weights_nd(d6.data_ptr(), nu, doc.data_ptr(), len(outer), om,
                                        fptrs(dF), R, W.data_ptr(), None) == 0
    ca.sync()
    # weights: exact FP64 products
    w_ref = np.ones((nu, R))
    for k in range(nu):
        for q, m in enumerate(outer):
            w_ref[k] *= F[m][u["outer_coords"][k * len(outer) + q]]
    assert np.array_equal(W.numpy(), w_ref)
    # tiles: FP64 sums of the pool rounded once
    T = np.zeros((nu, 4096))
    for k in range(nu):
        n_, st = u["unit6"][k][3], u["unit6"][k][4]
        np.add.at(T[k], u["lid"][st:st + n_], u["val"][st:st + n_])
    assert np.array_equal(tiles.numpy(), T.astype(np.float32))
    for slot, n in enumerate(inner):
        out = ca.DevBuf.zeros((dims[n], R), np.float64)
        grp = (None, None, 0)
        if G:
            order = np.zeros(nu, np.uint32)
            off = np.zeros(nu + 1, np.uint32)
            ng = C.c_size_t()
            hdr = np.ascontiguousarray(u["unit6"], np.uint32).view(np.int32)
            assert ca.lib.cptc_dense_groups(hdr.ctypes.data, 6, nu, slot, G, order.ctypes.data,
                                            off.ctypes.data, C.byref(ng)) == 0
            gbufs = (dbuf(ca, order), dbuf(ca, off[:ng.value + 1].copy()))
            grp = (gbufs[0].data_ptr(), gbufs[1].data_ptr(), ng.value)
        args = [slot, d6.data_ptr(), nu, tiles.data_ptr(), W.data_ptr(), *grp,
                dF[inner[0]].data_ptr(), dF[inner[1]].data_ptr(), dF[inner[2]].data_ptr(),
                dims[inner[0]], dims[inner[1]], dims[inner[2]], out.data_ptr(), R]
        if kern == "fp32":
            rc = ca.lib.cptc_mttkrp_units_nd(*args, None)
        else:
            nb = ca.lib.cptc_tile_operands_bytes(max(dims[m] for m in inner), R)
            ws = ca.DevBuf.zeros((nb,), np.uint8)
            if kern == "bf16x3":
                rc = ca.lib.cptc_mttkrp_units_nd_ws(*args, ws.data_ptr(), nb, None)
            else:
                # the slot's compacted split unit image (the order-3 tiles' format)
                cm = ca.DevBuf.zeros((nu * 64,), np.uint32)
                so = ca.DevBuf.zeros((nu + 1,), np.uint32)
                tot = C.c_uint64()
                assert ca.lib.cptc_dense_tiles_compact3_mask(tiles.data_ptr(), nu, slot,
                                                             cm.data_ptr(), so.data_ptr(),
                                                             C.byref(tot), None) == 0
                sg = ca.DevBuf.zeros((max(tot.value, 1) * 4,), np.uint32)
                assert ca.lib.cptc_dense_tiles_compact3_fill(tiles.data_ptr(), nu, slot,
                                                             cm.data_ptr(), so.data_ptr(),
                                                             sg.data_ptr(), None) == 0
                rc = ca.lib.cptc_mttkrp_units_nd_cws(
                    slot, d6.data_ptr(), nu, cm.data_ptr(), so.data_ptr(), sg.data_ptr(),
                    tot.value, W.data_ptr(), *grp, dF[inner[0]].data_ptr(),
                    dF[inner[1]].data_ptr(), dF[inner[2]].data_ptr(), dims[inner[0]],
                    dims[inner[1]], dims[inner[2]], out.data_ptr(), R, ws.data_ptr(), nb, None)
        assert rc == 0, ca.lib.cptc_last_error()
        ca.sync()
        ref = orc.mttkrp_units_nd(idx, val, dims, u, n, [f.ravel() for f in F], R)
        assert rel_err(out.numpy(), ref.reshape(dims[n], R)) <= 1e-5, (slot, n)


@pytest.mark.parametrize("R", [1, 5, 16, 32])
def test_chol_ridge_solve(ca, orc, dev, R):
    rng = np.random.default_rng(R)
    A = rng.random((50, R))
    FtF = A.T @ A
    Y = rng.standard_normal((777, R))
    dA, dY = dbuf(ca, FtF), dbuf(ca, Y)
    out = ca.DevBuf.zeros((777, R))
    assert ca.lib.cptc_chol_ridge_solve(dA.data_ptr(), dY.data_ptr(), out.data_ptr(), 777, R,
                                        None) == 0
    ca.sync()
    ref = orc.chol_solve_nd(FtF.ravel(), Y.ravel(), R).reshape(777, R)
    assert rel_err(out.numpy(), ref) <= 1e-11


@pytest.mark.parametrize("R", [1, 7, 16, 17, 32])
@pytest.mark.parametrize("rows,rank_def", [(150, False), (1, False), (64, False), (65, False),
                                           (1717, False), (150, True)])
def test_chol_ridge_factor_apply(ca, dev, R, rows, rank_def):
    """The two halves of the ridge solve: L is the Cholesky factor of
    FtF + eps I (eps = 1e-12 tr / R + 1e-300), and factor + apply gives the
    same bits as cptc_chol_ridge_solve (one launch: every 64-row workgroup
    factors in one wave), for one and several workgroups and for a
    rank-deficient FtF whose later pivots fall to the eps ridge."""
    rng = np.random.default_rng(100 + R + rows)
    A = rng.random(((R + 1) // 2 if rank_def else 3 * R + 5, R))
    FtF = A.T @ A
    Y = rng.standard_normal((rows, R))
    dA, dY = dbuf(ca, FtF), dbuf(ca, Y)
    L = ca.DevBuf.zeros((R, R))
    out = ca.DevBuf.zeros((rows, R))
    ref = ca.DevBuf.zeros((rows, R))
    assert ca.lib.cptc_chol_ridge_factor(dA.data_ptr(), L.data_ptr(), R, None) == 0
    assert ca.lib.cptc_chol_ridge_apply(L.data_ptr(), dY.data_ptr(), out.data_ptr(), rows, R,
                                        None) == 0
    assert ca.lib.cptc_chol_ridge_solve(dA.data_ptr(), dY.data_ptr(), ref.data_ptr(), rows, R,
                                        None) == 0
    ca.sync()
    Lg = L.numpy()
    assert np.all(np.triu(Lg, 1) == 0.0)
    if not rank_def:
        eps = 1e-12 * np.trace(FtF) / R + 1e-300
        Lref = np.linalg.cholesky(FtF + eps * np.eye(R))
        assert rel_err(Lg, Lref) <= 1e-12
        assert rel_err(out.numpy(), np.linalg.solve(FtF + eps * np.eye(R), Y.T).T) <= 1e-10
    assert np.all(np.isfinite(ref.numpy()))
    assert np.array_equal(out.numpy(), ref.numpy())


def test_chol_ridge_singular_pivot(ca, orc, dev):
    """A rank-deficient FtF hits the s <= 0 -> sqrt(eps) branch."""
    R = 6
    v = np.arange(1.0, R + 1)
    FtF = np.outer(v, v)
    Y = np.ones((10, R))
    dA, dY = dbuf(ca, FtF), dbuf(ca, Y)
    out = ca.DevBuf.zeros((10, R))
    assert ca.lib.cptc_chol_ridge_solve(dA.data_ptr(), dY.data_ptr(), out.data_ptr(), 10, R,
                                        None) == 0
    ca.sync()
    ref = orc.chol_solve_nd(FtF.ravel(), Y.ravel(), R).reshape(10, R)
    assert np.all(np.isfinite(out.numpy()))
    assert rel_err(out.numpy(), ref) <= 1e-6


@pytest.mark.parametrize("rows,R,next_", [(1, 1, 2), (37, 5, 2), (64, 32, 0), (200, 16, -1),
                                           (2048, 32, 3), (65, 12, 2)])
def test_gen_normalize_gram(ca, dev, rows, R, next_):
    """The fused small-factor update (cptc_gen_normalize_gram): lambda and the
    normalised factor as numpy's column norms (a zero column keeps norm 1),
    the Gram of the normalised factor, the next mode's Hadamard product of
    the other Grams in mode order, FtV zeroed over exactly nzero entries."""
    rng = np.random.default_rng(rows * 100 + R)
    F = rng.standard_normal((rows, R))
    if R > 3:
        F[:, 3] = 0.0
    ngram, mode = 4, 1
    G = rng.standard_normal((ngram, R, R))
    dF, lam, dG = dbuf(ca, F), ca.DevBuf.zeros(R), dbuf(ca, G)
    ftf = ca.DevBuf.zeros((R, R))
    nz = 3 * R + 1
    ftv0 = rng.standard_normal(nz + 17)
    ftv = dbuf(ca, ftv0)
    assert ca.lib.cptc_gen_normalize_gram(dF.data_ptr(), rows, R, lam.data_ptr(), dG.data_ptr(),
                                          ngram, mode, next_, ftf.data_ptr(), ftv.data_ptr(), nz,
                                          None) == 0, ca.lib.cptc_last_error()
    ca.sync()
    n = np.linalg.norm(F, axis=0)
    n[~np.isfinite(n) | (n < 1e-14)] = 1.0
    Fn = F / n
    assert rel_err(lam.numpy(), n) <= 1e-14
    assert rel_err(dF.numpy(), Fn) <= 1e-14
    Gm = Fn.T @ Fn
    got = dG.numpy().reshape(ngram, R, R)
    assert rel_err(got[mode], Gm) <= 1e-13
    for g in range(ngram):
        if g != mode:
            assert np.array_equal(got[g], G[g])
    if next_ >= 0:
        ref = np.ones((R, R))
        for g in range(ngram):
            if g != next_:
                ref = ref * got[g]
        assert np.array_equal(ftf.numpy(), ref)   # the kernel's own Gram, in mode order
        assert np.all(ftv.numpy()[:nz] == 0.0) and np.array_equal(ftv.numpy()[nz:], ftv0[nz:])
    else:
        assert np.all(ftf.numpy() == 0.0) and np.array_equal(ftv.numpy(), ftv0)
    # sizes past the one-workgroup limit are an error, not a launch
    assert ca.lib.cptc_gen_normalize_gram(dF.data_ptr(), 70000, R, lam.data_ptr(), dG.data_ptr(),
                                          ngram, mode, next_, ftf.data_ptr(), ftv.data_ptr(), nz,
                                          None) != 0


def test_normalize_hadamard_residual(ca, orc, dev):
    rng = np.random.default_rng(2)
    R = 12
    F = rng.standard_normal((333, R))
    F[:, 3] = 0.0                               # a zero column keeps norm 1
    dF, lam = dbuf(ca, F), ca.DevBuf.zeros(R)
    assert ca.lib.cptc_gen_normalize(dF.data_ptr(), 333, R, lam.data_ptr(), None) == 0
    ca.sync()
    n = np.linalg.norm(F, axis=0)
    n[3] = 1.0
    assert rel_err(lam.numpy(), n) <= 1e-14
    assert rel_err(dF.numpy(), F / n) <= 1e-14
    G = rng.standard_normal((4, R, R))
    dG, out = dbuf(ca, G), ca.DevBuf.zeros((R, R))
    for skip in (0, 2, -1):
        assert ca.lib.cptc_gram_hadamard(dG.data_ptr(), 4, skip, R, out.data_ptr(), None) == 0
        ca.sync()
        ref = np.ones((R, R))
        for g in range(4):
            if g != skip:
                ref = ref * G[g]
        assert np.array_equal(out.numpy(), ref)
    dims = (20, 7, 30, 4)
    nnz = 2000
    idx = np.ascontiguousarray(np.stack([rng.integers(0, d, nnz) for d in dims]).astype(np.uint32))
    val = rng.standard_normal(nnz)
    Fs = [rng.random((d, R)) for d in dims]
    lamv = rng.random(R)
    o2 = ca.DevBuf.zeros(2)
    bufs = [dbuf(ca, idx), dbuf(ca, val), dbuf(ca, lamv)]   # alive until the kernel is done
    dFs = [dbuf(ca, f) for f in Fs]
    assert ca.lib.cptc_residual_nd(4, bufs[0].data_ptr(), bufs[1].data_ptr(), nnz, fptrs(dFs),
                                   bufs[2].data_ptr(), R, o2.data_ptr(), None) == 0
    ca.sync()
    ref = orc.residual_nd(idx, val, dims, [f.ravel() for f in Fs], lamv, R)
    assert abs(o2.numpy()[0] - ref) <= 1e-10 * ref
    assert abs(o2.numpy()[1] - np.sum(val * val)) <= 1e-12 * np.sum(val * val)


# ----------------------------------------------------------- driver parity --

@pytest.mark.parametrize("N,inner", [(4, (0, 1, 2)), (5, (0, 1, 2)), (4, (1, 2, 3))])
def test_driver_mttkrp_every_mode(ca, orc, dev, N, inner):
    rng = np.random.default_rng(10 + N)
    dims = (40, 35, 48, 33, 20)[:N]
    t = tensor(ca, clustered(rng, dims, inner, 0.5, 8000), dims, rng)
    R = 16
    g = ca.Gen(t, R=R, inner=inner)
    assert g.info.dense_enabled
    idx = g.coords()
    F = [rng.random((d, R)) for d in dims]
    for m in range(N):
        g.set_factor(m, F[m])
    u = orc.dense_nd(idx, t.val, dims, 0.03, inner)
    views = orc.views_nd(idx, t.val, dims, u["is_dense"], True, inner)
    for n in range(N):
        got = g.mttkrp(n)
        ref = np.zeros(dims[n] * R)
        if n in inner:
            ref = orc.mttkrp_units_nd(idx, t.val, dims, u, n, [f.ravel() for f in F], R)
        ref = orc.mttkrp_seg_nd(idx, t.val, dims, views, n, n in inner,
                                [f.ravel() for f in F], R, ref)
        tol = 1e-5 if n in inner else 1e-10
        assert rel_err(got, ref.reshape(dims[n], R)) <= tol, n


@pytest.mark.parametrize("dense,svd,how", [(True, False, "hits"), (False, False, "hits"),
                                           (False, True, "cadr"), (True, False, "auto")])
def test_als_fit_vs_oracle(ca, orc, dev, dense, svd, how):
    rng = np.random.default_rng(21)
    dims = (40, 35, 48, 6)
    idx = clustered(rng, dims, (0, 1, 2), 0.5, 12000)
    t = tensor(ca, idx, dims, rng)
    R = 8
    g = ca.Gen(t, R=R, seed=42, reorder=how, dense=dense, svd=svd)
    fit, ip, m2, ms = g.run(20)
    ridx, rrank = orc.reorder_nd(t.idx, t.val, dims, how, 3, 8000000)
    rfit, rip, rm2, rF, rlam = orc.als_nd(ridx, t.val, dims, rrank, R, 42, svd, dense, 0.03, 20)
    tol = 1e-4 if (dense and g.info.dense_enabled) else 1e-8
    assert np.max(np.abs(fit - rfit)) <= tol, (fit[-3:], rfit[-3:])
    if not (dense and g.info.dense_enabled):
        for m in range(4):
            assert rel_err(g.factor(m), rF[m].reshape(dims[m], R)) <= 1e-6
        assert rel_err(g.lam(), rlam) <= 1e-6
    res, x2 = g.residual()
    ref_res = orc.residual_nd(ridx, t.val, dims, [g.factor(m).ravel() for m in range(4)],
                              g.lam(), R)
    assert abs(res - ref_res) <= 1e-9 * max(ref_res, 1.0)
    assert abs(x2 - np.sum(t.val ** 2)) <= 1e-12 * x2
    # The Gram fit is the full-tensor fit: X^2 - 2 iprod + model^2 equals
    # ||X - Xhat||_F^2 over every cell.  The "exact" residual of the
    # reference sums over the nonzeros only, so it can only be smaller.
    X = np.zeros(dims)
    np.add.at(X, tuple(ridx.astype(np.int64)), t.val)
    Fm = [g.factor(m) for m in range(4)]
    Xh = np.einsum("r,ar,br,cr,dr->abcd", g.lam(), *Fm, optimize=True)
    full = np.sum((X - Xh) ** 2)
    gram_res = x2 - 2 * ip[-1] + m2[-1]
    assert abs(gram_res - full) <= 1e-8 * x2
    assert res <= full * (1 + 1e-12)


def test_profile_and_dump(ca, dev, tmp_path):
    rng = np.random.default_rng(4)
    dims = (40, 35, 48, 3)
    t = tensor(ca, clustered(rng, dims, (0, 1, 2), 0.5, 4000), dims, rng)
    g = ca.Gen(t, R=4, profile=True)
    g.run(3)
    ph, it = g.profile()
    assert it == 3 and np.all(ph >= 0) and ph.sum() > 0
    base = str(tmp_path / "dump")
    g.dump(base)
    lines = open(base + ".factors.txt").read().splitlines()
    assert lines[0].startswith("# cpTC factor dump")
    assert lines[1] == "order 4" and lines[2] == "rank 4" and lines[3] == "dims 40 35 48 3"
    assert lines[4] == "mode 0 40 4"
    assert np.allclose(np.array([float(x) for x in lines[5].split()]), g.factor(0)[0], rtol=0,
                       atol=1e-15)
    assert lines[-2] == "lambda 4"
    assert np.allclose([float(x) for x in lines[-1].split()], g.lam(), rtol=1e-15)


def test_dump_bytes(ca, dev, tmp_path):
    """GEN_DUMP (generic.cu:2253-2287) byte for byte: the comment line, 'order',
    'rank', 'dims', per mode 'mode m dim R' and one line per row, values
    space-separated as an ostream at precision 17 writes them (= '%.17g'),
    then 'lambda R' and the lambda line."""
    rng = np.random.default_rng(9)
    dims = (40, 35, 48, 3)
    t = tensor(ca, clustered(rng, dims, (0, 1, 2), 0.5, 4000), dims, rng)
    R = 5
    g = ca.Gen(t, R=R)
    g.run(2)
    F = [g.factor(m) for m in range(4)]
    lam = g.lam()
    base = str(tmp_path / "d")
    g.dump(base)
    g.close()
    fmt = lambda row: " ".join("%.17g" % x for x in row)
    exp = ["# cpTC factor dump (factors are column-normalised; lambda holds the norms)",
           "order 4", f"rank {R}", "dims " + " ".join(str(d) for d in dims)]
    for m in range(4):
        exp.append(f"mode {m} {dims[m]} {R}")
        exp.extend(fmt(F[m].reshape(dims[m], R)[i]) for i in range(dims[m]))
    exp += [f"lambda {R}", fmt(lam)]
    assert open(base + ".factors.txt", "rb").read() == ("\n".join(exp) + "\n").encode()


def test_rejects_unsupported(ca, dev):
    t = ca.Tensor((4, 4, 4, 4), np.zeros((4, 3), np.uint32), np.ones(3))
    with pytest.raises(ca.CptcError):
        ca.Gen(t, R=33)
    with pytest.raises(ca.CptcError):
        ca.Gen(ca.Tensor((4, 4, 4, 4), np.zeros((4, 0), np.uint32), np.zeros(0)), R=4)


def test_selftest(ca, dev):
    assert ca.gen_selftest(verbose=True) == 0


def fit_tol(fit, cap=1e-4):
    """Fit bound after 20 iterations: the task's 1e-4, but never more than
    1e-3 of the fit itself (config 5's fit is about 0.0023, where 1e-4 would
    be 4 % of it)."""
    return min(cap, 1e-3 * abs(fit))


def check_every_mode(g, orc, idx, vals, dims, R, u, inner, tag):
    """Every mode's MTTKRP of the driver (its own kernel choice: dense units
    on the matrix cores plus the FP64 segment kernel for the inner modes, the
    segment kernel or the per-unit sums for the outer ones) on its initial
    factors against the oracle: inner modes <= 1e-5 (matrix cores), outer
    modes <= 1e-10 (FP64), the reference's relative-L2 metric
    (generic.cu:1619-1629).  Returns the per-mode errors."""
    N = len(dims)
    F = [g.factor(m).ravel() for m in range(N)]
    views = orc.views_nd(idx, vals, dims, u["is_dense"], True, inner)
    errs = []
    for n in range(N):
        got = g.mttkrp(n)
        ref = np.zeros(dims[n] * R)
        if n in inner:
            ref = orc.mttkrp_units_nd(idx, vals, dims, u, n, F, R)
        ref = orc.mttkrp_seg_nd(idx, vals, dims, views, n, n in inner, F, R, ref)
        err = rel_err(got, ref.reshape(dims[n], R))
        errs.append(err)
        print(f"[{tag}] mode {n} ({'inner' if n in inner else 'outer'}) MTTKRP rel err "
              f"{err:.3e}", flush=True)
        assert err <= (1e-5 if n in inner else 1e-10), (tag, n, err)
    del views
    return errs


@pytest.mark.timeout(300)
def test_config4_full_size(ca, orc, dev):
    """Config 4 (3.3 M elements, order 4, R = 16): layout bit-exact, every
    mode's MTTKRP on the initial factors against the oracle, 20 iterations'
    fit against the oracle."""
    t = ca.synth_config(4)
    R = 16
    g = ca.Gen(t, R=R)
    ridx, rrank = orc.reorder_nd(t.idx, t.val, t.dims, "hits", 3, 8000000)
    assert np.array_equal(g.coords(), ridx)
    for m in range(4):
        assert np.array_equal(g.rank(m), rrank[m]), m
    u = orc.dense_nd(ridx, t.val, t.dims, 0.03)
    assert int(g.info.n_units) == len(u["unit6"])
    got = g.units()
    assert np.array_equal(got["is_dense"], u["is_dense"])
    assert np.array_equal(got["lid"], u["lid"])
    check_every_mode(g, orc, ridx, t.val, t.dims, R, u, (0, 1, 2), "cfg4")
    fit, _, _, _ = g.run(20)
    rfit = orc.als_nd(ridx, t.val, t.dims, rrank, R, 42, False, True, 0.03, 20)[0]
    print(f"[cfg4] fit {fit[-1]:.10f} oracle {rfit[-1]:.10f}", flush=True)
    assert np.max(np.abs(fit - rfit)) <= fit_tol(rfit[-1]), (fit, rfit)


@pytest.mark.timeout(600)
@pytest.mark.parametrize("N,inner,R", [(4, (0, 1, 2), 16), (5, (0, 1, 2), 16), (5, (1, 2, 3), 16),
                                     (5, (0, 1, 2), 32), (4, (1, 2, 3), 7), (5, (1, 2, 3), 20)])
def test_unit_sums_outer_modes(ca, orc, dev, N, inner, R, monkeypatch):
    """Every element in a dense unit (config 5's case): the outer modes'
    MTTKRP from per-unit inner sums (from the FP64 unit images on the matrix
    cores, cptc_gen_unit_sums_img, and with GEN_UNIT_SUMS_IMG=0 from the pools,
    cptc_gen_unit_sums; then cptc_gen_unit_scatter) against the oracle's FP64
    segment sum over all elements (<= 1e-10), and the same with
    GEN_UNIT_SUMS=0 (the segment kernel); inner modes unchanged (units on the
    matrix cores, <= 1e-5).  R = 7 and 20 pad the rank tiles."""
    rng = np.random.default_rng(30 + N + inner[0])
    dims = (40, 35, 48, 33, 20)[:N]
    t0 = tensor(ca, clustered(rng, dims, inner, 0.5, 8000), dims, rng)
    g0 = ca.Gen(t0, R=16, inner=inner)
    keep = g0.units()["is_dense"].astype(bool)
    u6 = g0.units()["unit6"].reshape(-1, 6)
    g0.close()
    assert keep.sum() > 1000
    assert u6[:, 3].max() > 100   # units of more than 64 elements (several batches)
    t = ca.Tensor(dims, np.ascontiguousarray(t0.idx[:, keep]), np.ascontiguousarray(t0.val[keep]))
    F = [rng.random((d, R)) for d in dims]
    for flag, img in (("1", "1"), ("1", "0"), ("0", "1")):
        monkeypatch.setenv("GEN_UNIT_SUMS", flag)
        monkeypatch.setenv("GEN_UNIT_SUMS_IMG", img)
        g = ca.Gen(t, R=R, inner=inner)
        assert g.info.dense_enabled and g.units()["is_dense"].all()
        assert int(g.info.unit_sums) == int(flag)
        assert int(g.info.unit_sums_img) == int(flag == "1" and img == "1")
        idx = g.coords()
        for m in range(N):
            g.set_factor(m, F[m])
        u = orc.dense_nd(idx, t.val, dims, 0.03, inner)
        views = orc.views_nd(idx, t.val, dims, u["is_dense"], True, inner)
        for n in range(N):
            got = g.mttkrp(n)
            ref = np.zeros(dims[n] * R)
            if n in inner:
                ref = orc.mttkrp_units_nd(idx, t.val, dims, u, n, [f.ravel() for f in F], R)
            ref = orc.mttkrp_seg_nd(idx, t.val, dims, views, n, n in inner,
                                    [f.ravel() for f in F], R, ref)
            tol = 1e-5 if n in inner else 1e-10
            assert rel_err(got, ref.reshape(dims[n], R)) <= tol, (flag, n)
        g.close()


@pytest.mark.parametrize("inner", [(1, 2, 3), (0, 1, 2)])
def test_unit_sums_driver_loop(ca, dev, inner, monkeypatch):
    """The per-unit sums as the driver keeps them: formed once per iteration
    at the first outer mode, reused by the later outer modes, dropped when an
    inner mode updates (inner (1,2,3): outer modes 0 and 4 sit on both sides
    of the inner ones, so the sums are formed twice per iteration).  Runs
    with GEN_UNIT_SUMS=1 and =0 (the segment kernel) from identical factors
    must agree: the two differ only in the order of FP64 additions (and of
    the FP64 atomics), which moves fits by ~1e-16 per iteration before ALS
    amplifies it (10x to 4000x per iteration), hence 1e-8 on fits and 1e-6
    relative on factors after 3 iterations."""
    N, R = 5, 16
    rng = np.random.default_rng(77 + inner[0])
    dims = (40, 35, 48, 33, 20)
    t0 = tensor(ca, clustered(rng, dims, inner, 0.5, 8000), dims, rng)
    g0 = ca.Gen(t0, R=R, inner=inner)
    keep = g0.units()["is_dense"].astype(bool)
    g0.close()
    t = ca.Tensor(dims, np.ascontiguousarray(t0.idx[:, keep]), np.ascontiguousarray(t0.val[keep]))
    F = [rng.random((d, R)) for d in dims]
    res = {}
    for flag in ("1", "0"):
        monkeypatch.setenv("GEN_UNIT_SUMS", flag)
        g = ca.Gen(t, R=R, inner=inner)
        assert g.units()["is_dense"].all()
        assert int(g.info.unit_sums) == int(flag)
        for m in range(N):
            g.set_factor(m, F[m])
        fit, _, _, _ = g.run(3)
        res[flag] = (fit, [g.factor(m) for m in range(N)], g.lam())
        g.close()
    (f1, F1, l1), (f0, F0, l0) = res["1"], res["0"]
    dfit = float(np.max(np.abs(f1 - f0)))
    derr = max(rel_err(F1[m], F0[m]) for m in range(N))
    print(f"[usum loop {inner}] fits {f1} vs {f0}: |dfit| {dfit:.3e}, factors {derr:.3e}",
          flush=True)
    assert dfit <= 1e-8
    assert derr <= 1e-6
    assert rel_err(l1, l0) <= 1e-6


@pytest.mark.timeout(600)
def test_config5_full_size(ca, orc, dev):
    """Config 5 (20 M elements, order 5, R = 32, 32 768 dense units): device
    reorder and units bit-exact; every mode's MTTKRP on the initial factors
    against the oracle (every element lies in a unit, so the inner modes are
    the dense units alone on the matrix cores, <= 1e-5, and the outer modes
    the per-unit FP64 sums, <= 1e-10); 20 iterations' fit against the
    oracle."""
    t = ca.synth_config(5)
    R = 32
    g = ca.Gen(t, R=R)
    print(f"[cfg5] nnz {t.nnz} units {int(g.info.n_units)}", flush=True)
    ridx, rrank = orc.reorder_nd(t.idx, t.val, t.dims, "hits", 3, 8000000)
    assert np.array_equal(g.coords(), ridx)
    for m in range(5):
        assert np.array_equal(g.rank(m), rrank[m]), m
    u = orc.dense_nd(ridx, t.val, t.dims, 0.03)
    assert int(g.info.n_units) == len(u["unit6"])
    got = g.units()
    assert np.array_equal(got["unit6"].ravel(), np.asarray(u["unit6"]).ravel())
    assert np.array_equal(got["is_dense"], u["is_dense"])
    assert got["is_dense"].all(), "config 5: every element in a unit (units-alone check)"
    del got
    check_every_mode(g, orc, ridx, t.val, t.dims, R, u, (0, 1, 2), "cfg5")
    fit, _, _, _ = g.run(20)
    g.close()
    rfit = orc.als_nd(ridx, t.val, t.dims, rrank, R, 42, False, True, 0.03, 20)[0]
    print(f"[cfg5] fit {fit[-1]:.10f} oracle {rfit[-1]:.10f}", flush=True)
    assert np.max(np.abs(fit - rfit)) <= fit_tol(rfit[-1]), (fit, rfit)


def _parse_dump(path):
    """GEN_DUMP text: order, rank, dims, N blocks of rows, lambda."""
    lines = [ln for ln in open(path).read().split("\n") if ln and not ln.startswith("#")]
    N = int(lines[0].split()[1])
    R = int(lines[1].split()[1])
    dims = [int(x) for x in lines[2].split()[1:]]
    pos, F = 3, []
    for m in range(N):
        hdr = lines[pos].split()
        assert hdr == ["mode", str(m), str(dims[m]), str(R)]
        F.append(np.array([[float(x) for x in ln.split()] for ln in lines[pos + 1:pos + 1 + dims[m]]]))
        pos += 1 + dims[m]
    assert lines[pos].split() == ["lambda", str(R)]
    lam = np.array([float(x) for x in lines[pos + 1].split()])
    return F, lam


def test_dump_input_order(ca, dev, tmp_path):
    """GEN_DUMP in the input's index order (an opt-in fix: the reference's
    dump is in the HITS-relabelled space): rows are the relabelled rows
    permuted by the rank maps, and the model evaluated at the input tensor's
    own coordinates gives the driver's exact residual."""
    rng = np.random.default_rng(21)
    dims = (60, 20, 90, 40)
    t = tensor(ca, clustered(rng, dims, (0, 1, 2), 0.5, 4000), dims, rng)
    g = ca.Gen(t, R=8, reorder="hits", rounds=3)
    g.run(5)
    res, x2 = g.residual()
    g.dump(str(tmp_path / "a"))
    g.dump(str(tmp_path / "b"), input_order=True)
    ranks = [g.rank(m) for m in range(4)]
    g.close()
    Fa, la = _parse_dump(str(tmp_path / "a.factors.txt"))
    Fb, lb = _parse_dump(str(tmp_path / "b.factors.txt"))
    assert np.array_equal(la, lb)
    assert any(not np.array_equal(r, np.arange(len(r))) for r in ranks)
    for m in range(4):
        assert np.array_equal(Fb[m], Fa[m][ranks[m].astype(np.int64)]), m
    xhat = np.zeros(t.nnz)
    for r in range(8):
        p = np.full(t.nnz, lb[r])
        for m in range(4):
            p = p * Fb[m][t.idx[m].astype(np.int64), r]
        xhat += p
    assert abs(np.sum((t.val - xhat) ** 2) - res) <= 1e-9 * x2


def cli_fit(out):
    """Fit of the last '[GEN] iter' line."""
    it = [l for l in out.splitlines() if l.startswith("[GEN] iter ")]
    return float(it[-1].split("fit=")[1].split()[0])


def test_cli_generic_switches(ca, dev, tmp_path):
    """The generic driver's switches through the CLI (generic.cu:1647-1663,
    1796-1840, 2114-2116; main.cu:102-130): GEN_REORDER (none / an unknown
    name falls back to cadr), GEN_REORDER_T, GEN_DENSE=0, a GEN_DENSE_INNER
    that is not three distinct modes (the dense path is disabled),
    GEN_SOLVER=svd (pseudoinverse instead of the ridge Cholesky: the same fit
    on a well-conditioned problem), GEN_SEED (another start), and
    ALS_GENERIC_FORCE=1, which sends an order-3 file down the generic path."""
    rng = np.random.default_rng(9)
    dims = (40, 35, 48, 3)
    t = tensor(ca, clustered(rng, dims, (0, 1, 2), 0.5, 3000), dims, rng)
    path = str(tmp_path / "t4.tns")
    ca.write_tns(path, t)

    def run(p=path, **env):
        r = subprocess.run([ca.CLI_PATH, p, "3", "8"], capture_output=True, text=True,
                           env=dict(os.environ, **env), timeout=120)
        assert r.returncode == 0, (env, r.stderr)
        return r.stdout

    base = run()
    assert "[GEN] reorder=hits(T=3)" in base and "[GEN] dense: units=" in base
    out = run(GEN_REORDER="none", GEN_DENSE="0")
    assert "[GEN] reorder=none" in out and "[GEN] dense: units=" not in out
    out = run(GEN_REORDER="bogus")
    assert "[GEN] unknown GEN_REORDER=bogus -> falling back to cadr" in out
    assert "[GEN] reorder=cadr" in out
    assert "[GEN] reorder=hits(T=1)" in run(GEN_REORDER_T="1")
    out = run(GEN_DENSE_INNER="0,0,1")
    assert "[GEN] dense path disabled: GEN_DENSE_INNER=0,0,1" in out
    assert "[GEN] dense: units=" not in out
    assert abs(cli_fit(run(GEN_SOLVER="svd")) - cli_fit(base)) <= 1e-6
    assert cli_fit(run(GEN_SEED="7")) != cli_fit(base)
    t3 = tensor(ca, clustered(rng, (40, 35, 48), (0, 1, 2), 0.5, 2000), (40, 35, 48), rng)
    p3 = str(tmp_path / "t3.tns")
    ca.write_tns(p3, t3)
    out = run(p3, ALS_GENERIC_FORCE="1")
    assert "[Main] order-3 tensor -> generic" in out and "[GEN] reorder=cadr" in out
    assert "[GEN] iter 3/3" in out


def test_cli_generic_and_selftest(ca, dev, tmp_path):
    rng = np.random.default_rng(8)
    dims = (40, 35, 48, 3)
    t = tensor(ca, clustered(rng, dims, (0, 1, 2), 0.5, 3000), dims, rng)
    path = str(tmp_path / "t4.tns")
    ca.write_tns(path, t)
    env = dict(os.environ, GEN_DUMP=str(tmp_path / "d"), GEN_PROFILE="1")
    r = subprocess.run([ca.CLI_PATH, path, "3", "8"], capture_output=True, text=True, env=env,
                       timeout=120)
    assert r.returncode == 0, r.stderr
    out = r.stdout
    for s in ("[Main] order-4 tensor -> generic", "[GEN] reorder=hits(T=3)", "[GEN] dense: units=",
              "[GEN] mode 3 view:", "[GEN] iter 3/3", "[GEN][profile] avg/iter", "[GEN] exact:",
              "[GEN] lambda =", "factors dumped"):
        assert s in out, s
    assert os.path.exists(str(tmp_path / "d.factors.txt"))
    r = subprocess.run([ca.CLI_PATH], capture_output=True, text=True,
                       env=dict(os.environ, GEN_SELFTEST="1"), timeout=120)
    assert r.returncode == 0 and "[SELFTEST] PASSED (0 failures)" in r.stdout, r.stdout
