"""Pins the oracle's layout functions (CADR, factor init, hybrid partition,
row-sorted views) against independent numpy restatements and invariants.

cadr3        cadr.cu:23-66     bijection + non-increasing degree; tie-free
                               inputs have a unique answer = stable argsort
init3        common.cu:66-123  numpy's MT19937 (legacy seeding = std::mt19937)
                               + libstdc++ generate_canonical (2 draws / double)
partition3   partition.cu:581-1493  stable argsort by block id, runs, cutoff
views3       partition.cu:1865-2329 stable lexsort on (target, o1, o0), segments
"""
import numpy as np
import pytest


def rand_coo(rng, dims, nnz, dup=False):
    idx = np.stack([rng.integers(0, d, nnz) for d in dims]).astype(np.int32)
    if dup:  # repeat some coordinates with different values
        k = nnz // 10
        idx[:, -k:] = idx[:, :k]
    val = rng.standard_normal(nnz)
    return idx, val


# ----------------------------------------------------------------- CADR ---

def test_cadr_invariants(orc):
    rng = np.random.default_rng(0)
    dims = (37, 50, 61)
    idx, _ = rand_coo(rng, dims, 3000)
    perms = orc.cadr3(idx[0], idx[1], idx[2], dims)
    for m in range(3):
        p = perms[m]
        assert sorted(p.tolist()) == list(range(dims[m]))          # bijection
        deg = np.bincount(idx[m], minlength=dims[m])
        new_deg = np.empty_like(deg)
        new_deg[p] = deg
        assert np.all(np.diff(new_deg) <= 0)                        # degree-descending


def test_cadr_tie_free_closed_form(orc):
    # distinct degrees: index x appears (perm-shuffled) 1..dim times
    rng = np.random.default_rng(1)
    dims = (12, 9, 15)
    cols = []
    for d in dims:
        order = rng.permutation(d)
        cols.append(np.repeat(order, np.arange(1, d + 1)))
    n = max(len(c) for c in cols)
    idx = np.stack([np.concatenate([c, np.full(n - len(c), c[-1])]) for c in cols]).astype(np.int32)
    perms = orc.cadr3(idx[0], idx[1], idx[2], dims)
    for m in range(3):
        deg = np.bincount(idx[m], minlength=dims[m])
        assert len(set(deg.tolist())) == dims[m]
        expect = np.empty(dims[m], np.int64)
        expect[np.argsort(-deg, kind="stable")] = np.arange(dims[m])
        assert perms[m].tolist() == expect.tolist()


# ------------------------------------------------------------ factor init ---

def mt_canonical(seed, n):
    bg = np.random.MT19937()
    bg._legacy_seeding(seed)            # init_genrand(seed) == std::mt19937(seed)
    raw = bg.random_raw(2 * n).astype(np.uint64)
    lo, hi = raw[0::2].astype(np.float64), raw[1::2].astype(np.float64)
    return (lo + hi * 2.0 ** 32) / 2.0 ** 64


def test_init_factors_mt19937(orc):
    dims, R = (7, 5, 9), 4
    A, B, C = orc.init_factors3(dims, R, 42)
    ref = mt_canonical(42, sum(dims) * R)
    got = np.concatenate([A, B, C])
    assert np.array_equal(got, ref)


# --------------------------------------------------------------- partition --

def np_partition(idx, val, dims, thr, num_cus=256):
    nb = [(d + 15) // 16 for d in dims]
    key = ((idx[0] // 16).astype(np.uint64) * nb[1] + idx[1] // 16) * nb[2] + idx[2] // 16
    order = np.argsort(key, kind="stable")
    sk = key[order]
    _, starts, counts = np.unique(sk, return_index=True, return_counts=True)
    if thr > 0:
        cutoff = min(max(int(4096.0 * thr), 1), 4096)
    else:
        s = num_cus / 24.0
        frac = (0.688 / s) / ((1.20 / s) + (0.688 / s))
        target = int(len(val) * frac)
        cs = np.sort(counts)[::-1]
        acc = np.cumsum(cs)
        hit = np.nonzero(acc >= target)[0]
        cutoff = int(cs[hit[0]]) if len(hit) else 1
    tiles, lid, pv, si, sj, sk2, sv = [], [], [], [], [], [], []
    for st, c in zip(starts, counts):
        e = order[st:st + c]
        if c >= cutoff:
            b = int(sk[st])
            tiles.append([b // nb[2] // nb[1], (b // nb[2]) % nb[1], b % nb[2], c])
            lid.extend((((idx[0][e] % 16) * 16 + idx[1][e] % 16) * 16 + idx[2][e] % 16).tolist())
            pv.extend(val[e].tolist())
        else:
            si.extend(idx[0][e].tolist())
            sj.extend(idx[1][e].tolist())
            sk2.extend(idx[2][e].tolist())
            sv.extend(val[e].tolist())
    return cutoff, np.array(tiles, np.int64).reshape(-1, 4), lid, pv, si, sj, sk2, sv


@pytest.mark.parametrize("thr,dup", [(0.03, False), (0.001, True), (0.0, False), (1.0, True)])
def test_partition_matches_numpy(orc, thr, dup):
    rng = np.random.default_rng(5)
    dims = (70, 45, 90)
    # clustered: half the elements inside a few 16^3 blocks
    idx, val = rand_coo(rng, dims, 6000, dup)
    idx[:, :3000] = np.stack([rng.integers(0, 16, 3000), rng.integers(16, 32, 3000),
                              rng.integers(32, 48, 3000)])
    p = orc.partition3(idx[0], idx[1], idx[2], val, dims, thr)
    cutoff, tiles, lid, pv, si, sj, sk, sv = np_partition(idx, val, dims, thr)
    assert p["cutoff"] == cutoff
    assert p["tiles"].tolist() == tiles.tolist()
    assert p["pool_lid"].tolist() == lid and p["pool_val"].tolist() == pv
    assert p["sp_i"].tolist() == si and p["sp_j"].tolist() == sj and p["sp_k"].tolist() == sk
    assert p["sp_val"].tolist() == sv
    off = p["pool_off"]
    assert off[0] == 0 and off[-1] == len(lid)
    assert np.array_equal(np.diff(off), tiles[:, 3]) if len(tiles) else len(off) == 1


def test_partition_every_element_once(orc):
    rng = np.random.default_rng(9)
    dims = (33, 40, 18)
    idx, val = rand_coo(rng, dims, 5000, True)
    p = orc.partition3(idx[0], idx[1], idx[2], val, dims, 0.002)
    assert len(p["pool_val"]) + len(p["sp_val"]) == len(val)
    assert np.isclose(np.sum(p["pool_val"]) + np.sum(p["sp_val"]), np.sum(val))


# ------------------------------------------------------------------- views --

def np_views(i, j, k, v, dims):
    i, j, k = (np.asarray(x, np.uint64) for x in (i, j, k))
    packed = (i << np.uint64(30)) | (j << np.uint64(15)) | k
    out = []
    for mode in range(3):
        t, o1, o0 = [(i, k, j), (j, k, i), (k, j, i)][mode]
        order = np.lexsort((o0, o1, t))        # last key primary; lexsort is stable
        tgt = t[order]
        rows, starts, counts = np.unique(tgt, return_index=True, return_counts=True)
        br, bs, bc = [], [], []
        for r, s, c in zip(rows, starts, counts):
            for c0 in range(0, c, 1024):
                br.append(int(r))
                bs.append(int(s + c0))
                bc.append(int(min(1024, c - c0)))
        out.append(dict(coords=packed[order], vals=np.asarray(v)[order], blk_row=br,
                        blk_start=bs, blk_cnt=bc))
    return out


def test_views_match_numpy(orc):
    rng = np.random.default_rng(3)
    dims = (40, 3000, 25)   # one long row mode to get multi-segment rows
    n = 20000
    i = rng.integers(0, 3, n).astype(np.uint32)        # 3 heavy rows in mode 0
    j = rng.integers(0, dims[1], n).astype(np.uint32)
    k = rng.integers(0, dims[2], n).astype(np.uint32)
    j[-500:] = j[:500]
    k[-500:] = k[:500]
    i[-500:] = i[:500]                                  # duplicates
    v = rng.standard_normal(n)
    got = orc.views3(i, j, k, v, dims)
    ref = np_views(i, j, k, v, dims)
    for mode in range(3):
        for key in ("coords", "vals", "blk_row", "blk_start", "blk_cnt"):
            assert np.array_equal(np.asarray(got[mode][key]), np.asarray(ref[mode][key])), (mode, key)
        assert max(got[mode]["blk_cnt"]) <= 1024
        assert int(np.sum(got[mode]["blk_cnt"])) == n


def test_views_reject_wide_dims(orc):
    with pytest.raises(RuntimeError):
        orc.views3(np.array([0], np.uint32), np.array([0], np.uint32), np.array([0], np.uint32),
                   np.array([1.0]), (40000, 2, 2))


# -------------------------------------------------------------- dense views --

def np_decode_pool(p):
    """partition.cu:2335-2379: each tile's pool entries, in tile then pool order,
    back to global coordinates (local id = (li*16 + lj)*16 + lk)."""
    i, j, k, v = [], [], [], []
    off = p["pool_off"]
    for t, (b0, b1, b2, cnt) in enumerate(p["tiles"].tolist()):
        lid = np.asarray(p["pool_lid"][off[t]:off[t] + cnt], np.int64)
        assert len(lid) == cnt
        i.append(b0 * 16 + (lid >> 8))
        j.append(b1 * 16 + ((lid >> 4) & 15))
        k.append(b2 * 16 + (lid & 15))
        v.append(np.asarray(p["pool_val"][off[t]:off[t] + cnt]))
    cat = (lambda xs, dt: np.concatenate(xs).astype(dt) if xs else np.zeros(0, dt))
    return (cat(i, np.uint32), cat(j, np.uint32), cat(k, np.uint32), cat(v, np.float64))


@pytest.mark.parametrize("dup", [False, True])
def test_dense_views_match_numpy(orc, dup):
    """dense_views3 (partition.cu:2387-2517) = the pool decoded in tile order, then
    the same stable (target, o1, o0) sort and 1024-element segments as views3."""
    rng = np.random.default_rng(21)
    dims = (70, 45, 90)
    idx, val = rand_coo(rng, dims, 6000, dup)
    # clustered blocks (two full tiles' worth of candidates) so several tiles qualify
    idx[:, :2500] = np.stack([rng.integers(0, 16, 2500), rng.integers(16, 32, 2500),
                              rng.integers(32, 48, 2500)])
    idx[:, 2500:4000] = np.stack([rng.integers(48, 64, 1500), rng.integers(0, 16, 1500),
                                  rng.integers(64, 80, 1500)])
    p = orc.partition3(idx[0], idx[1], idx[2], val, dims, 0.03)
    assert len(p["tiles"]) >= 2
    got = orc.dense_views3(p, dims)
    di, dj, dk, dv = np_decode_pool(p)
    # multiset: the decoded pool is exactly the elements the partition put into tiles
    sp = np.stack([p["sp_i"], p["sp_j"], p["sp_k"]]).astype(np.int64)
    both = np.concatenate([np.stack([di, dj, dk]).astype(np.int64), sp], axis=1)
    allv = np.concatenate([dv, p["sp_val"]])
    o_in = np.lexsort((val, idx[2], idx[1], idx[0]))
    o_out = np.lexsort((allv, both[2], both[1], both[0]))
    assert np.array_equal(idx[:, o_in].astype(np.int64), both[:, o_out])
    assert np.array_equal(val[o_in], allv[o_out])
    ref = np_views(di, dj, dk, dv, dims)
    for mode in range(3):
        for key in ("coords", "vals", "blk_row", "blk_start", "blk_cnt"):
            assert np.array_equal(np.asarray(got[mode][key]), np.asarray(ref[mode][key])), (mode, key)


def test_dense_views_mttkrp_closed_form(orc):
    """Residual view + dense view MTTKRP (the FP64 fallback path) equals the
    closed form Y = X_(n) (KR of the other factors) over the whole tensor, with
    duplicates summed (the FP64 kernels add every element)."""
    rng = np.random.default_rng(22)
    dims, R = (40, 37, 45), 5
    cells = np.array(np.meshgrid(np.arange(32, 40), np.arange(16, 37), np.arange(0, 45),
                                 indexing="ij")).reshape(3, -1)
    dense_part = cells[:, rng.random(cells.shape[1]) < 0.6]
    bg = np.stack([rng.integers(0, d, 900) for d in dims])
    idx = np.concatenate([dense_part, bg, dense_part[:, :50]], axis=1).astype(np.int32)
    val = rng.standard_normal(idx.shape[1])
    p = orc.partition3(idx[0], idx[1], idx[2], val, dims, 0.03)
    assert len(p["tiles"]) > 0 and len(p["sp_val"]) > 0
    rv = orc.views3(p["sp_i"], p["sp_j"], p["sp_k"], p["sp_val"], dims)
    dvw = orc.dense_views3(p, dims)
    X = np.zeros(dims)
    np.add.at(X, tuple(idx), val)
    F = [rng.random((d, R)) for d in dims]
    subs = ["ijk,jr,kr->ir", "ijk,ir,kr->jr", "ijk,ir,jr->kr"]
    for mode in range(3):
        got = sum(orc.mttkrp3_view(vw, mode, F[0].ravel(), F[1].ravel(), F[2].ravel(), R,
                                   dims[mode]).reshape(dims[mode], R) for vw in (rv, dvw))
        others = [F[m] for m in range(3) if m != mode]
        ref = np.einsum(subs[mode], X, *others)
        assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 1e-13
