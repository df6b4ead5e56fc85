"""Driver-level parity (cptc_als3_*): the device layout is bit-exact with the
oracle (CADR permutations, partition tiles and pools, row-sorted views), the
MTTKRP of every mode matches, and 20 ALS iterations reach the oracle's fit
within 1e-4 (FP64 path and MFMA dense-tile path)."""
import os
import subprocess

import numpy as np
import pytest

from conftest import rel_err

pytestmark = pytest.mark.gpu


def oracle_layout(orc, t, thr, cadr=True):
    idx = t.idx.astype(np.int32)
    if cadr:
        perms = orc.cadr3(idx[0], idx[1], idx[2], t.dims)
        idx = np.stack([perms[m][idx[m]] for m in range(3)]).astype(np.int32)
    else:
        perms = [np.arange(d, dtype=np.int32) for d in t.dims]
    p = orc.partition3(idx[0], idx[1], idx[2], t.val, t.dims, thr)
    v = orc.views3(p["sp_i"], p["sp_j"], p["sp_k"], p["sp_val"], t.dims)
    return perms, p, v


def clustered(ca, seed=0, n=64, blocks=12):
    return ca.synth_blocks3(n, blocks, 0.1, 0.6, 2e-3, seed)


CASES = [
    ("zipf", 0.03), ("zipf", 0.0), ("blocks", 0.03), ("blocks", 0.001), ("blocks", 0.3),
]


def make(ca, kind, seed=1):
    if kind == "zipf":
        return ca.synth_zipf((700, 400, 1500), (1.1, 1.1, 1.1), 120000, 0, seed)
    return clustered(ca, seed)


@pytest.mark.parametrize("kind,thr", CASES)
def test_layout_bit_exact(ca, orc, dev, kind, thr):
    t = make(ca, kind)
    perms, p, v = oracle_layout(orc, t, thr)
    with ca.Als3(t, R=8, threshold=thr, path=2) as h:     # FP64 path: dense views too
        for m in range(3):
            assert np.array_equal(h.perm(m), perms[m]), f"perm {m}"
        assert int(h.info.dense_cutoff) == p["cutoff"]
        tl = h.tiles()
        assert np.array_equal(tl["tiles"], p["tiles"])
        assert np.array_equal(tl["pool_off"], p["pool_off"])
        assert np.array_equal(tl["pool_lid"], p["pool_lid"])
        assert np.array_equal(tl["pool_val"], p["pool_val"])
        assert int(h.info.sparse_nnz) == len(p["sp_val"])
        for m in range(3):
            got = h.view(0, m)
            for k in ("coords", "vals", "blk_row", "blk_start", "blk_cnt"):
                assert np.array_equal(got[k], np.asarray(v[m][k])), (m, k)
        if len(p["pool_val"]):
            dv = orc.dense_views3(p, t.dims)
            for m in range(3):
                got = h.view(1, m)
                for k in ("coords", "vals", "blk_row", "blk_start", "blk_cnt"):
                    assert np.array_equal(got[k], np.asarray(dv[m][k])), ("dense", m, k)


@pytest.mark.parametrize("kind,thr,R", [("blocks", 0.03, 16), ("blocks", 0.001, 16),
                                        ("zipf", 0.03, 16), ("blocks", 0.03, 100)])
def test_fp64_merged_view(ca, orc, dev, kind, thr, R, monkeypatch):
    """FP64-only path with dense tiles and a residual: the kernels read one
    row-sorted view of every nonzero (bit-exact with the oracle's views3 of
    the whole relabelled tensor), its MTTKRP of every mode is within 1e-10 of
    the reference's two views (residual + dense pool, partition.cu:2387-2517),
    and 20 iterations' fits are within 1e-6 of ALS_FP64_MERGE=0, which keeps
    the two launches.  Without tiles or without a residual there is nothing
    to merge.  At R = 100 the FP64 kernel reads the blocked layout built over
    the merged view."""
    t = make(ca, kind)
    perms, p, v = oracle_layout(orc, t, thr)
    both = len(p["tiles"]) > 0 and len(p["sp_val"]) > 0
    monkeypatch.delenv("ALS_FP64_MERGE", raising=False)
    with ca.Als3(t, R=R, threshold=thr, path=2) as h:
        assert int(h.info.fp64_merged) == int(both)
        assert int(h.info.sparse_blocked) == int(R > 64)
        if both:
            idx = np.stack([perms[m][t.idx[m]] for m in range(3)]).astype(np.int32)
            av = orc.views3(idx[0], idx[1], idx[2], t.val, t.dims)
            for m in range(3):
                got = h.view(2, m)
                for k in ("coords", "vals", "blk_row", "blk_start", "blk_cnt"):
                    assert np.array_equal(got[k], np.asarray(av[m][k])), (m, k)
            F = [h.factor(m).ravel() for m in range(3)]
            dv = orc.dense_views3(p, t.dims)
            for mode in range(3):
                ref = (orc.mttkrp3_view(v, mode, *F, R, t.dims[mode]) +
                       orc.mttkrp3_view(dv, mode, *F, R, t.dims[mode]))
                assert rel_err(h.mttkrp(mode), ref.reshape(t.dims[mode], R)) <= 1e-10, mode
        fit, _, _ = h.run(20)
    monkeypatch.setenv("ALS_FP64_MERGE", "0")
    with ca.Als3(t, R=R, threshold=thr, path=2) as h2:
        assert int(h2.info.fp64_merged) == 0
        fit2, _, _ = h2.run(20)
    assert np.max(np.abs(fit - fit2)) <= 1e-6, (fit[-3:], fit2[-3:])


def test_cadr_entry_point_matches_oracle(ca, orc, dev):
    t = ca.synth_zipf((300, 256, 999), (1.1, 0.0, 1.3), 50000, 0, 2)
    perms, idx = ca.cadr3(t)
    ref = orc.cadr3(*(t.idx[m].astype(np.int32) for m in range(3)), t.dims)
    for m in range(3):
        assert np.array_equal(perms[m], ref[m])
        assert np.array_equal(idx[m], ref[m][t.idx[m]])


def test_views_reject_wide_dims(ca, dev):
    t = ca.Tensor((40000, 3, 3), np.array([[39999, 0], [0, 1], [0, 2]], np.uint32),
                  np.array([1.0, 2.0]))
    with pytest.raises(ca.CptcError):
        ca.Als3(t, R=4, cadr=False)


@pytest.mark.parametrize("kind,path,R", [("zipf", 2, 16), ("zipf", 2, 128), ("blocks", 1, 32),
                                         ("blocks", 2, 32), ("zipf", 1, 20)])
def test_mttkrp_every_mode(ca, orc, dev, kind, path, R):
    t = make(ca, kind, 3)
    perms, p, v = oracle_layout(orc, t, 0.03)
    with ca.Als3(t, R=R, threshold=0.03, path=path) as h:
        F = [h.factor(m) for m in range(3)]
        ref_init = orc.init_factors3(t.dims, R, 42)
        for m in range(3):
            assert np.array_equal(F[m].ravel(), ref_init[m])
        mfma = int(h.info.use_mfma) == 1 and len(p["tiles"]) > 0
        dv = orc.dense_views3(p, t.dims) if (not mfma and len(p["pool_val"])) else None
        for mode in range(3):
            ref = orc.mttkrp3_view(v, mode, *(f.ravel() for f in F), R, t.dims[mode])
            if mfma:
                ref = ref + orc.mttkrp3_tiles(p, mode, *(f.ravel() for f in F), R, t.dims)
            elif dv is not None:
                ref = ref + orc.mttkrp3_view(dv, mode, *(f.ravel() for f in F), R, t.dims[mode])
            got = h.mttkrp(mode)
            tol = 1e-5 if mfma else 1e-10
            assert rel_err(got, ref.reshape(t.dims[mode], R)) <= tol, mode


@pytest.mark.parametrize("kind,path,R,tk", [("zipf", 2, 16, None), ("blocks", 1, 16, None),
                                            ("blocks", 2, 16, None), ("zipf", 0, 64, None),
                                            ("blocks", 1, 32, "bf16x3"),
                                            ("blocks", 1, 48, "bf16x3")])
def test_als_fit_matches_oracle_20_iters(ca, orc, dev, kind, path, R, tk, monkeypatch):
    """20 iterations within 1e-4 of the oracle's fits (the FP64 oracle runs
    the same tile sums exactly); tk forces the tile kernel
    (ALS_TILE_KERNEL)."""
    if tk:
        monkeypatch.setenv("ALS_TILE_KERNEL", tk)
    t = make(ca, kind, 4)
    perms, p, v = oracle_layout(orc, t, 0.03)
    with ca.Als3(t, R=R, threshold=0.03, path=path) as h:
        F = [h.factor(m).ravel() for m in range(3)]
        mfma = int(h.info.use_mfma) == 1 and len(p["tiles"]) > 0
        if tk:
            assert mfma and int(h.info.tile_bf16x3) == int(tk == "bf16x3")
        tiles = p if mfma else None
        dv = orc.dense_views3(p, t.dims) if (not mfma and len(p["pool_val"])) else None
        o = orc.Als3(v, dv, tiles, float(np.sum(t.val ** 2)), t.dims, R, *F, None)
        fit, ms, mt = h.run(20)
        ofit, _, _ = o.iterate(20)
        assert np.max(np.abs(fit - ofit)) <= 1e-4, (fit[-3:], ofit[-3:])
        # iterations replayed from the captured graph have no per-mode events
        # (MTTKRP time NaN); the first and the last always run eagerly
        fin = np.isfinite(mt)
        assert fin[0] and fin[-1] and np.all(ms > 0)
        assert np.all(mt[fin] > 0) and np.all(mt[fin] <= ms[fin])
        assert int(h.info.graph_mode) == 1 or np.all(fin)
        res, x2 = h.residual()
        ores, ox2 = o.residual(True)
        assert abs(x2 - ox2) <= 1e-12 * ox2
        assert abs(res - ores) <= 1e-3 * ores
        lam = h.lam()
        assert rel_err(lam, o.lam()) <= 1e-3
        # unpermuted export: row x of the exported factor = row perm[x] in the relabelled space
        for m in range(3):
            assert np.array_equal(h.factor(m, unpermuted=True), h.factor(m)[perms[m]])


@pytest.mark.parametrize("kind,path,R", [("blocks", 1, 16), ("blocks", 2, 16), ("zipf", 2, 33)])
def test_residual3_identical_factors(ca, orc, dev, kind, path, R):
    """Exact residual (common.cu:251-650) on identical factors and lambda: the
    device sum over the residual view, the FP64 dense view or the tile pools
    equals the closed form sum_e (v_e - sum_r l_r a b c)^2 over the relabelled
    COO (duplicates included, every element once) and the oracle's sum."""
    t = make(ca, kind, 6)
    perms, p, v = oracle_layout(orc, t, 0.03)
    with ca.Als3(t, R=R, threshold=0.03, path=path) as h:
        h.run(2)                                    # lambda != 1 and factors of an ALS state
        F = [h.factor(m) for m in range(3)]
        lam = h.lam()
        assert np.any(np.abs(lam - 1.0) > 1e-3)
        res, x2 = h.residual()
        mfma = int(h.info.use_mfma) == 1 and len(p["tiles"]) > 0
    idx = [perms[m][t.idx[m]].astype(np.int64) for m in range(3)]
    xhat = np.einsum("r,er,er,er->e", lam, F[0][idx[0]], F[1][idx[1]], F[2][idx[2]])
    ref = float(np.sum((t.val - xhat) ** 2))
    assert abs(x2 - float(np.sum(t.val ** 2))) <= 1e-13 * x2
    assert abs(res - ref) <= 1e-12 * ref, (res, ref)
    dv = orc.dense_views3(p, t.dims) if (not mfma and len(p["pool_val"])) else None
    o = orc.Als3(v, dv, p if mfma else None, x2, t.dims, R, *(f.ravel() for f in F), lam)
    ores, ox2 = o.residual(True)
    assert abs(res - ores) <= 1e-12 * ores and abs(x2 - ox2) <= 1e-13 * ox2


@pytest.mark.parametrize("R", [16, 32, 128])
def test_fused_path_matches_oracle(ca, orc, dev, R, monkeypatch):
    """ALS_FUSED (als.cu:28, 529-555): one merged launch per mode.  MTTKRP of
    every mode within the MFMA bound of the oracle, 20 iterations within 1e-4
    of the oracle's fits and within 1e-6 of the two-stream driver's with the
    same (FP32) tile arithmetic (ALS_TILE_KERNEL=fp32)."""
    t = clustered(ca, 9)
    perms, p, v = oracle_layout(orc, t, 0.03)
    assert len(p["tiles"]) > 0 and len(p["sp_val"]) > 0
    with ca.Als3(t, R=R, threshold=0.03, path=1, fused=1) as h:
        assert int(h.info.fused) == 1 and int(h.info.tile_bf16x3) == 0
        F = [h.factor(m).ravel() for m in range(3)]
        for mode in range(3):
            ref = orc.mttkrp3_view(v, mode, *F, R, t.dims[mode])
            ref = ref + orc.mttkrp3_tiles(p, mode, *F, R, t.dims)
            assert rel_err(h.mttkrp(mode), ref.reshape(t.dims[mode], R)) <= 1e-5, mode
        fit, ms, mt = h.run(20)
        sp, _, kit = h.kernel_times()
        assert kit == 4 and np.all(sp > 0)   # a queued run times iterations 0, 8, 16 and 19
    o = orc.Als3(v, None, p, float(np.sum(t.val ** 2)), t.dims, R, *F, None)
    ofit, _, _ = o.iterate(20)
    assert np.max(np.abs(fit - ofit)) <= 1e-4, (fit[-3:], ofit[-3:])
    monkeypatch.setenv("ALS_TILE_KERNEL", "fp32")
    with ca.Als3(t, R=R, threshold=0.03, path=1, fused=0) as h2:
        assert int(h2.info.fused) == 0 and int(h2.info.tile_bf16x3) == 0
        fit2, _, _ = h2.run(20)
    monkeypatch.delenv("ALS_TILE_KERNEL")
    assert np.max(np.abs(fit - fit2)) <= 1e-6
    # the FP64 path and odd R never take the merged grid
    with ca.Als3(t, R=R, threshold=0.03, path=2, fused=1) as h3:
        assert int(h3.info.fused) == 0
    with ca.Als3(t, R=R + 1, threshold=0.03, path=1, fused=1) as h4:
        assert int(h4.info.fused) == 0


def test_gather_probe(ca, dev, monkeypatch):
    """cptc_als3_gather_probe: the blocked kernel's element-level row gathers
    alone run on the handle's blocked view (positive, finite times of the
    order of the full kernel's: at config 3 they take as long as the kernel,
    whose other work hides behind them), leave the factors and the next
    iterations untouched, and are refused without a blocked view."""
    t = ca.synth_zipf((3000, 2000, 5000), (1.1, 1.1, 1.1), 400000, 0, 17)
    monkeypatch.setenv("ALS_SPARSE_BLOCKED", "1")
    with ca.Als3(t, R=128, threshold=0.03, path=2) as h:
        assert int(h.info.sparse_blocked) == 1
        F = [h.factor(m).copy() for m in range(3)]
        ms = h.gather_probe(2)
        assert np.all(np.isfinite(ms)) and np.all(ms > 0), ms
        for m in range(3):
            assert np.array_equal(h.factor(m), F[m])
        fit, _, _ = h.run(2)
        sp, _, k = h.kernel_times(reset=True)
        assert k >= 1 and np.all(np.isfinite(fit))
        probe = h.gather_probe(2)
        assert np.all(probe < 4 * sp / k + 0.05), (probe, sp / k)
    monkeypatch.setenv("ALS_SPARSE_BLOCKED", "0")
    with ca.Als3(t, R=128, threshold=0.03, path=2) as h:
        assert int(h.info.sparse_blocked) == 0
        with pytest.raises(RuntimeError):
            h.gather_probe(1)


@pytest.mark.parametrize("R,path", [(128, 2), (100, 2), (66, 2), (128, 1)])
def test_blocked_sparse_view_matches_oracle(ca, orc, dev, R, path, monkeypatch):
    """R in (64, 128]: the FP64 residual MTTKRP over the blocked layout
    (target-row x run-level blocks, staged run-level rows in LDS,
    ALS_SPARSE_BLOCKED=1); every mode within 1e-10 of the oracle on the
    reference view (FP64 path) and of the row-segment kernel
    (ALS_SPARSE_BLOCKED=0), hot Zipf rows (staged block pairs) and cold ones
    (unstaged spans) alike.  Unforced, the driver picks the blocked layout only
    when no MFMA tile kernel runs beside the residual one (the FP32 tile
    kernel runs beside it; the split-bf16 one before it)."""
    t = ca.synth_zipf((3000, 2000, 5000), (1.1, 1.1, 1.1), 400000, 0, 17)
    perms, p, v = oracle_layout(orc, t, 0.03)
    outs = []
    for blocked in ("1", "0"):
        monkeypatch.setenv("ALS_SPARSE_BLOCKED", blocked)
        with ca.Als3(t, R=R, threshold=0.03, path=path) as h:
            assert int(h.info.sparse_blocked) == int(blocked)
            F = [h.factor(m).ravel() for m in range(3)]
            outs.append([h.mttkrp(m) for m in range(3)])
            mfma = int(h.info.use_mfma) == 1 and len(p["tiles"]) > 0
            dv = orc.dense_views3(p, t.dims) if (not mfma and len(p["pool_val"])) else None
    for mode in range(3):
        ref = orc.mttkrp3_view(v, mode, *F, R, t.dims[mode])
        if mfma:
            ref = ref + orc.mttkrp3_tiles(p, mode, *F, R, t.dims)
        elif dv is not None:
            ref = ref + orc.mttkrp3_view(dv, mode, *F, R, t.dims[mode])
        ref = ref.reshape(t.dims[mode], R)
        tol = 1e-5 if mfma else 1e-10
        assert rel_err(outs[0][mode], ref) <= tol, mode
        assert rel_err(outs[0][mode], outs[1][mode]) <= (1e-5 if mfma else 1e-12), mode
    monkeypatch.delenv("ALS_SPARSE_BLOCKED")
    for kern in ("fp32", "bf16x3"):
        monkeypatch.setenv("ALS_TILE_KERNEL", kern)
        with ca.Als3(t, R=R, threshold=0.03, path=path) as h:
            mf = int(h.info.use_mfma) == 1 and int(h.info.num_dense_tiles) > 0
            assert int(h.info.tile_bf16x3) == int(mf and kern == "bf16x3")
            assert int(h.info.tiles_beside) == int(mf and kern == "fp32")
            assert int(h.info.sparse_blocked) == int(not h.info.tiles_beside)
            if mf and kern == "bf16x3":
                assert int(h.info.tile_compact) == 1
                # the driver's MTTKRP with the split-bf16 tiles, against the oracle
                F = [h.factor(m).ravel() for m in range(3)]
                for mode in range(3):
                    ref = orc.mttkrp3_view(v, mode, *F, R, t.dims[mode])
                    ref = ref + orc.mttkrp3_tiles(p, mode, *F, R, t.dims)
                    assert rel_err(h.mttkrp(mode), ref.reshape(t.dims[mode], R)) <= 1e-5, mode
    monkeypatch.delenv("ALS_TILE_KERNEL")


@pytest.mark.parametrize("kind,R,path,fused", [("clustered", 32, 1, 0), ("clustered", 16, 1, 0),
                                                ("zipf", 100, 1, 0), ("clustered", 32, 2, 0),
                                                ("clustered", 32, 1, 1)])
def test_graph_replay_matches_eager(ca, dev, kind, R, path, fused, monkeypatch):
    """Quiet runs that replay the captured iteration (ALS_GRAPH=1) against
    the eager driver from the same state.  The MTTKRP's FP64 atomic adds
    land in a different order in any two runs (1e-16 after one iteration)
    and ALS amplifies that 10x to 4000x per iteration (zipf, R=100), so each
    comparison covers 3 iterations from identical factors (the 2nd replayed,
    the 1st and 3rd eager): fits within 1e-8 and factors within 1e-6
    relative, where a stale or missing launch in the replay shows at 1e-4
    and more.  Three rounds, with eager work and host waits between
    them (a single-mode MTTKRP, factors read back) and the factors set from
    the host before each (which leaves the captured state; the 1st iteration
    restores it and the cached graph is replayed again)."""
    t = make(ca, kind, 4)
    rng = np.random.default_rng(R)
    hs = {}
    for g in ("1", "0"):
        monkeypatch.setenv("ALS_GRAPH", g)
        hs[g] = ca.Als3(t, R=R, threshold=0.03, path=path, fused=fused)
        assert int(hs[g].info.graph_mode) == int(g)
    try:
        F = [hs["0"].factor(m) for m in range(3)]
        for rnd in range(3):
            if rnd:
                F = [hs["0"].factor(m) * (0.5 + rng.random(R)) for m in range(3)]
            out = {}
            for g, h in hs.items():
                for m in range(3):
                    h.set_factor(m, F[m])
                fit, ms, mt = h.run(3)
                out[g] = (fit, [h.factor(m) for m in range(3)], mt)
                h.mttkrp(1)
            assert np.max(np.abs(out["1"][0] - out["0"][0])) <= 1e-8, rnd
            for a_, b_ in zip(out["1"][1], out["0"][1]):
                assert rel_err(a_, b_) <= 1e-6, rnd
            assert np.isnan(out["1"][2][1]) and np.isfinite(out["1"][2][[0, 2]]).all()
            assert np.all(np.isfinite(out["0"][2]))
    finally:
        for h in hs.values():
            h.close()


@pytest.mark.parametrize("kind,R,bits", [("clustered", 32, 15), ("clustered", 5, 15),
                                         ("zipf", 16, 15), ("zipf_wide", 16, 3),
                                         ("zipf", 33, 0)])
def test_small_update_matches_separate_launches(ca, dev, kind, R, bits, monkeypatch):
    """The one-launch update (cptc_update_small3: every mode of at most 4096
    rows at R <= 32, bit 3 = mode C's launch also forms the fit) against
    ALS_SMALL_UPDATE=0, which runs the separate apply, Gram, scaling and fit
    launches, from the same factors: 3 iterations, eager and replayed from
    the captured graph, within test_graph_replay_matches_eager's bounds
    (fits 1e-8, factors 1e-6: the MTTKRP's atomic order and the new sums'
    order differ at 1e-16 and ALS amplifies that; a missing clear of FtV or
    a stale FtF shows at 1e-3 and more).  zipf_wide's mode C has 5000 rows,
    so modes A and B take the one launch and mode C the separate ones."""
    if kind == "zipf_wide":
        t = ca.synth_zipf((700, 400, 5000), (1.1, 1.1, 1.1), 120000, 0, 5)
    else:
        t = make(ca, kind, 5)
    hs = {}
    for key, small, g in (("base", "0", "0"), ("eager", "1", "0"), ("graph", "1", "1")):
        monkeypatch.setenv("ALS_SMALL_UPDATE", small)
        monkeypatch.setenv("ALS_GRAPH", g)
        hs[key] = ca.Als3(t, R=R, threshold=0.03, path=1)
        assert int(hs[key].info.small_update) == (0 if small == "0" else bits)
    monkeypatch.delenv("ALS_SMALL_UPDATE")
    try:
        F = [hs["base"].factor(m) for m in range(3)]
        for rnd in range(2):
            out = {}
            for key, h in hs.items():
                for m in range(3):
                    h.set_factor(m, F[m])
                fit, _, _ = h.run(3)
                out[key] = (fit, [h.factor(m) for m in range(3)])
                h.mttkrp(2)
            for key in ("eager", "graph"):
                assert np.max(np.abs(out[key][0] - out["base"][0])) <= 1e-8, (key, rnd)
                for a_, b_ in zip(out[key][1], out["base"][1]):
                    assert rel_err(a_, b_) <= 1e-6, (key, rnd)
            F = [f * 0.9 for f in out["base"][1]]
    finally:
        for h in hs.values():
            h.close()


def test_graph_recaptured_after_scratch_growth(ca, dev, monkeypatch):
    """A captured iteration holds the addresses of the library's scratch
    buffers (Gram partials, pseudoinverse workspace, reduction partials).
    When another entry point grows one of them (cptc_gram on a wider
    factor reallocates the Gram partials), the next graph-mode run must
    capture the iteration again (cptc_als3_info.graph_captures counts the
    captures) and still match the eager driver from the same factors, within
    the bounds of test_graph_replay_matches_eager."""
    t = make(ca, "clustered", 6)
    R = 32
    hs = {}
    for g in ("1", "0"):
        monkeypatch.setenv("ALS_GRAPH", g)
        hs[g] = ca.Als3(t, R=R, threshold=0.03, path=1)
    try:
        assert int(hs["1"].refresh_info().graph_captures) == 0
        F = [hs["0"].factor(m) for m in range(3)]

        def both():
            out = {}
            for g, h in hs.items():
                for m in range(3):
                    h.set_factor(m, F[m])
                fit, _, _ = h.run(3)
                out[g] = (fit, [h.factor(m) for m in range(3)])
            assert np.max(np.abs(out["1"][0] - out["0"][0])) <= 1e-8
            for a_, b_ in zip(out["1"][1], out["0"][1]):
                assert rel_err(a_, b_) <= 1e-6

        both()
        assert int(hs["1"].refresh_info().graph_captures) == 1
        both()   # the cached graph is replayed: no new capture
        assert int(hs["1"].refresh_info().graph_captures) == 1
        # grow the Gram-partials scratch: 256 partials of 320 x 320 doubles
        rows, Rb = 16384, 320
        Fb = ca.DevBuf.from_numpy(np.random.default_rng(0).random((rows, Rb)))
        Gb = ca.DevBuf.zeros((Rb, Rb))
        assert ca.lib.cptc_gram(Fb.data_ptr(), rows, Rb, Gb.data_ptr(), None) == 0
        ca.sync()
        del Fb, Gb
        both()
        assert int(hs["1"].refresh_info().graph_captures) == 2
    finally:
        for h in hs.values():
            h.close()


def test_cli_runs_and_exports(ca, dev, tmp_path):
    t = make(ca, "zipf", 5)
    path = str(tmp_path / "t.tns")
    ca.write_tns(path, t)
    env = dict(os.environ, ALS_EXPORT_FACTORS=str(tmp_path / "f"))
    out = subprocess.run([ca.CLI_PATH, path, "3", "8"], env=env, capture_output=True, text=True,
                         timeout=300)
    assert out.returncode == 0, out.stderr
    iters = [l for l in out.stdout.splitlines() if l.startswith("[ALS] iter ")]
    assert len(iters) == 3 and "time=" in iters[0] and "fit=" in iters[0]
    lines = open(str(tmp_path / "f.0.out")).read().split("\n")
    assert lines[0] == "matrix" and lines[1] == "2" and lines[2] == f"{t.dims[0]} 8"
    assert len([x for x in lines[3:] if x]) == t.dims[0] * 8
    lam = open(str(tmp_path / "f.lambda.out")).read().split("\n")
    assert lam[:3] == ["vector", "1", "8"]


def test_cli_export_bytes_and_debug(ca, dev, tmp_path):
    """ALS_EXPORT_FACTORS (main.cu:595-621): 'matrix\\n2\\n<dim> <R>' then one
    '%.20lf' line per entry, rows in the input's index order, row-major
    (j * R + i); '<p>.lambda.out' = 'vector\\n1\\n<R>' then '%.20lf' lines.
    The files are byte-for-byte the rendering of their own values, and the
    values are the C-ABI driver's unpermuted factors and lambda after the same
    iteration.  ALS_DEBUG (als.cu:595-603, 731-746) adds its lines."""
    t = make(ca, "zipf", 7)
    fpath = str(tmp_path / "t.tns")
    ca.write_tns(fpath, t)
    R = 8
    env = dict(os.environ, ALS_EXPORT_FACTORS=str(tmp_path / "f"), ALS_DEBUG="1")
    for k in ("ALS_FORCE_CUDA", "ALS_FORCE_WMMA", "ALS_SERIAL"):
        env.pop(k, None)
    out = subprocess.run([ca.CLI_PATH, fpath, "1", str(R)], env=env, capture_output=True,
                         text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    lines = out.stdout.splitlines()
    it = [i for i, l in enumerate(lines) if l.startswith("[ALS] iter 1/1")]
    assert len(it) == 1
    assert lines[it[0] - 1].startswith("[DBG] modeC mttkrp wall = ")
    assert lines[it[0] - 1].endswith(" ms (dual)")
    dbg = lines[it[0] + 1]
    for key in ("[DBG] lambda[0..3]=", " A[0..3]=", " X2=", " iprod=", " model2=",
                " work_r[0..3]=", " FtV[0..3]="):
        assert key in dbg, key
    assert lines[it[0] + 2].startswith("[DBG] exact RMSE=")
    t2 = ca.load_tns3(fpath)
    with ca.Als3(t2, R=R) as h:
        h.run(1)
        F = [h.factor(m, unpermuted=True) for m in range(3)]
        lam = h.lam()
    for m in range(3):
        raw = open(str(tmp_path / f"f.{m}.out"), "rb").read()
        head = f"matrix\n2\n{t.dims[m]} {R}\n".encode()
        assert raw.startswith(head)
        vals = [float(x) for x in raw[len(head):].decode().split("\n") if x]
        assert len(vals) == t.dims[m] * R
        assert raw == head + "".join("%.20lf\n" % x for x in vals).encode()
        got = np.array(vals).reshape(t.dims[m], R)
        assert rel_err(got, F[m]) <= 1e-12, m
    raw = open(str(tmp_path / "f.lambda.out"), "rb").read()
    head = f"vector\n1\n{R}\n".encode()
    vals = [float(x) for x in raw[len(head):].decode().split("\n") if x]
    assert raw == head + "".join("%.20lf\n" % x for x in vals).encode()
    assert rel_err(vals, lam) <= 1e-12


@pytest.mark.parametrize("env_path,path", [({}, -1), ({"ALS_FORCE_CUDA": "1"}, 2),
                                           ({"ALS_FORCE_WMMA": "1"}, 1),
                                           ({"ALS_FORCE_WMMA": "1", "ALS_FUSED": "1"}, 1)])
def test_cli_cpp_flow_matches_driver(ca, dev, tmp_path, env_path, path):
    """The CLI runs main.cu's flow on the C++ interface (load_tns_file,
    compute/apply_cadr_reordering, init_factors_random, create_hybrid_format,
    build_mttkrp_views, build_dense_mttkrp_views, execute_als_decomposition,
    unpermute_factor_matrices).  It must reproduce the C-ABI driver, which
    runs the same CADR, initial factors, layout and kernels."""
    t = clustered(ca, 3)
    fpath = str(tmp_path / "t.tns")
    ca.write_tns(fpath, t)
    env = dict(os.environ, **env_path)
    for k in ("ALS_FORCE_CUDA", "ALS_FORCE_WMMA", "ALS_FUSED"):
        if k not in env_path:
            env.pop(k, None)
    out = subprocess.run([ca.CLI_PATH, fpath, "6", "16"], env=env, capture_output=True,
                         text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    lines = out.stdout.splitlines()
    fits = np.array([float(l.split("fit=")[1]) for l in lines if l.startswith("[ALS] iter ")])
    assert len(fits) == 6
    for s in ("[CADR] Total reordering time", "[Main] density check:", "[Fit Report] final R=16",
              "[ALS] Final RMSE=", "[Main] Final CP weights:", "Unpermutation!"):
        assert any(s in l for l in lines), s
    fused_line = any(l.startswith("[ALS] FUSED path active") for l in lines)
    assert fused_line == ("ALS_FUSED" in env_path)
    t2 = ca.load_tns3(fpath)
    with ca.Als3(t2, R=16, path=path, fused=1 if "ALS_FUSED" in env_path else 0) as h:
        ref, _, _ = h.run(6)
        lam = h.lam()
    # Same layout, factors and kernels; the FP64 atomic adds of the MTTKRP
    # can land in another order in a fresh process (the first launch runs
    # on cold caches), a 1-ulp difference that ALS on this small tensor
    # amplifies about 10x per iteration (~1e-9 by iteration 6).  The CLI
    # prints fits with 10 significant digits.
    assert np.max(np.abs(fits - ref)) <= 1e-7, (fits, ref)
    assert np.max(np.abs(fits[:3] - ref[:3])) <= 1e-10, (fits, ref)
    cli_lam = [l for l in lines if l.startswith("[Main] Final CP weights:")][0].split(":")[1]
    assert np.allclose(np.array([float(x) for x in cli_lam.split()]), lam, rtol=1e-5)


@pytest.mark.parametrize("switch,value", [("ALS_MERGED_NO_SPARSE", "1"),
                                          ("ALS_MERGED_NO_DENSE", "1"),
                                          ("ALS_MERGED_STRIDE", "2"),
                                          ("ALS_MERGED_STRIDE", "7"),
                                          ("ALS_MERGED_STRIDE", "100000")])
def test_merged_switches(ca, orc, dev, tmp_path, switch, value, monkeypatch):
    """The merged grid's experiment switches (dense.cu:2277-2283, 2350-2352)
    on ALS_FUSED: ALS_MERGED_NO_SPARSE leaves only the tile workgroups (the
    MTTKRP is the tiles' alone, MFMA bound 1e-5), ALS_MERGED_NO_DENSE only the
    residual segments (FP64, 1e-10), ALS_MERGED_STRIDE=k puts a tile workgroup
    at every k-th grid position (the whole MTTKRP, 1e-5; k past the grid puts
    the tiles after every segment).  Then the CLI (main.cu's flow on the C++
    interface, compute_mttkrp_merged_async) under the same switch reproduces
    the C-ABI driver's fits."""
    t = clustered(ca, 9)
    perms, p, v = oracle_layout(orc, t, 0.03)
    assert len(p["tiles"]) > 0 and len(p["sp_val"]) > 0
    R = 16
    monkeypatch.setenv(switch, value)
    with ca.Als3(t, R=R, threshold=0.03, path=1, fused=1) as h:
        assert int(h.info.fused) == 1
        F = [h.factor(m).ravel() for m in range(3)]
        for mode in range(3):
            ref = np.zeros(t.dims[mode] * R)
            if switch != "ALS_MERGED_NO_SPARSE":
                ref = ref + orc.mttkrp3_view(v, mode, *F, R, t.dims[mode])
            if switch != "ALS_MERGED_NO_DENSE":
                ref = ref + orc.mttkrp3_tiles(p, mode, *F, R, t.dims)
            tol = 1e-10 if switch == "ALS_MERGED_NO_DENSE" else 1e-5
            err = rel_err(h.mttkrp(mode), ref.reshape(t.dims[mode], R))
            assert err <= tol, (mode, err)
    fpath = str(tmp_path / "t.tns")
    ca.write_tns(fpath, t)
    env = dict(os.environ, ALS_FUSED="1", ALS_FORCE_WMMA="1")
    env[switch] = value
    env.pop("ALS_FORCE_CUDA", None)
    out = subprocess.run([ca.CLI_PATH, fpath, "4", str(R)], env=env, capture_output=True,
                         text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    lines = out.stdout.splitlines()
    assert any(l.startswith("[ALS] FUSED path active") for l in lines)
    fits = np.array([float(l.split("fit=")[1]) for l in lines if l.startswith("[ALS] iter ")])
    t2 = ca.load_tns3(fpath)
    with ca.Als3(t2, R=R, path=1, fused=1) as h:
        ref, _, _ = h.run(4)
    # the same layout, factors and launches; FP64 atomic order only (see
    # test_cli_cpp_flow_matches_driver), the CLI prints 10 significant digits
    assert len(fits) == 4 and np.max(np.abs(fits - ref)) <= 1e-8, (fits, ref)


@pytest.mark.parametrize("fm,path", [("0.99", "FP64 only"), ("0", "MFMA tiles + FP64 residual")])
def test_cli_fill_min(ca, dev, tmp_path, fm, path):
    """ALS_FILL_MIN (main.cu:370-391) replaces the CU-scaled fill_min in the
    density check: a threshold above every fill keeps the tiles in FP64 views,
    0 sends them to the matrix cores."""
    t = make(ca, "clustered", 3)
    fpath = str(tmp_path / "t.tns")
    ca.write_tns(fpath, t)
    env = dict(os.environ, ALS_FILL_MIN=fm)
    out = subprocess.run([ca.CLI_PATH, fpath, "2", "8"], env=env, capture_output=True,
                         text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    line = [l for l in out.stdout.splitlines() if l.startswith("[Main] density check:")]
    assert len(line) == 1 and f"(threshold {float(fm):g}) -> {path}" in line[0], line
    assert "tiles=0 " not in line[0]
    assert "[Main] device=" not in out.stdout   # the CU-scaled default was not consulted


def test_cli_profile_line(ca, dev, tmp_path):
    """ALS_PROFILE (als.cu:748-760): after each '[ALS] iter' line,
    '[ALS][profile] iter k gram=.. mttkrp=.. solve=.. fit=.. (iter=..)' with
    the reference's phases: gram = iteration start to mode C's Hadamard
    (modes A and B whole), mttkrp = mode C's MTTKRP, solve = mode C's update,
    fit = the Gram fit; consecutive event spans, so they add up to at most
    the iteration's time."""
    t = make(ca, "zipf", 5)
    fpath = str(tmp_path / "t.tns")
    ca.write_tns(fpath, t)
    env = dict(os.environ, ALS_PROFILE="1")
    out = subprocess.run([ca.CLI_PATH, fpath, "3", "8"], env=env, capture_output=True,
                         text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    lines = out.stdout.splitlines()
    prof = [l for l in lines if l.startswith("[ALS][profile] iter ")]
    assert len(prof) == 3
    for k, l in enumerate(prof):
        head, rest = l.split(" gram=")
        assert head == f"[ALS][profile] iter {k + 1}"
        vals = {}
        for part in ("gram=" + rest).replace("(", "").replace(")", "").split():
            key, val = part.split("=")
            vals[key] = float(val)
        assert list(vals) == ["gram", "mttkrp", "solve", "fit", "iter"]
        assert all(x >= 0 for x in vals.values()) and vals["mttkrp"] > 0
        parts = vals["gram"] + vals["mttkrp"] + vals["solve"] + vals["fit"]
        assert parts <= vals["iter"] * 1.0001 + 1e-3, vals
        assert lines[lines.index(l) - 1].startswith(f"[ALS] iter {k + 1}/3 ")
