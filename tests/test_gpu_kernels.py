"""Kernel-level parity through the C ABI (device buffers from cptc_dev_*) against
the CPU oracle and numpy closed forms.

Bars: sparse FP64 MTTKRP <= 1e-10 relative; dense-tile FP32-MFMA MTTKRP
<= 1e-5 relative to FP64; Gram / pinv / norms / fit FP64 to ~1e-12 (1e-9 for
the inverse of conditioned systems).
"""
import ctypes as C

import numpy as np
import pytest

from conftest import rel_err

pytestmark = pytest.mark.gpu


def to_dev(ca, a):
    return ca.DevBuf.from_numpy(a)


def zeros(ca, shape, dtype=np.float64):
    return ca.DevBuf.zeros(shape, dtype)


def stream(_ca):
    return None   # the null stream


def zipf_views(ca, orc, dims, nnz, seed, dup=False):
    t = ca.synth_zipf(dims, (1.1, 1.1, 1.1), nnz, 0, seed)
    idx = t.idx.astype(np.int32)
    if dup:
        idx[:, -nnz // 20:] = idx[:, :nnz // 20]
    v = orc.views3(idx[0].astype(np.uint32), idx[1].astype(np.uint32), idx[2].astype(np.uint32),
                   t.val, dims)
    return t, v


@pytest.mark.parametrize("R", [1, 2, 3, 6, 8, 10, 16, 31, 32, 48, 64, 100, 128, 200])
def test_sparse_mttkrp_vs_oracle(ca, orc, dev, R):
    dims = (500, 300, 900)
    t, views = zipf_views(ca, orc, dims, 60000, R, dup=True)
    rng = np.random.default_rng(R)
    F = [rng.standard_normal((d, R)) for d in dims]
    dF = [to_dev(ca, f) for f in F]
    for mode in range(3):
        v = views[mode]
        ref = orc.mttkrp3_view(views, mode, F[0].ravel(), F[1].ravel(), F[2].ravel(), R,
                               dims[mode]).reshape(dims[mode], R)
        dc, dv = to_dev(ca, v["coords"]), to_dev(ca, v["vals"])
        br, bs, bc = (to_dev(ca, v[k]) for k in ("blk_row", "blk_start", "blk_cnt"))
        out = zeros(ca, (dims[mode], R))
        F1 = dF[1] if mode == 0 else dF[0]
        F2 = dF[1] if mode == 2 else dF[2]
        rc = ca.lib.cptc_mttkrp_sparse3(mode, dc.data_ptr(), dv.data_ptr(), br.data_ptr(),
                                        bs.data_ptr(), bc.data_ptr(), len(v["blk_row"]),
                                        F1.data_ptr(), F2.data_ptr(), out.data_ptr(), R,
                                        stream(ca))
        assert rc == 0, ca.lib.cptc_last_error()
        ca.sync()
        assert rel_err(out.numpy(), ref) <= 1e-10, (mode, R)


@pytest.mark.parametrize("R", [8, 16, 30, 32, 64, 128])
@pytest.mark.parametrize("split", ["rows", "random"])
def test_sparse_mttkrp_free_segment_tables(ca, orc, dev, R, split):
    """The C ABI takes any segment table over a row-sorted view: whole rows
    as one segment (hot rows far beyond the 1024 elements of the reference's
    table, so a wave takes several passes) and rows cut at random lengths
    (1 to 3000: ragged shares of the wave's range and of its element slots).
    Every mode within 1e-10 of the oracle."""
    dims = (400, 300, 700)
    t, views = zipf_views(ca, orc, dims, 80000, R + 7)
    rng = np.random.default_rng(R)
    F = [rng.standard_normal((d, R)) for d in dims]
    dF = [to_dev(ca, f) for f in F]
    for mode in range(3):
        v = views[mode]
        ref = orc.mttkrp3_view(views, mode, F[0].ravel(), F[1].ravel(), F[2].ravel(), R,
                               dims[mode]).reshape(dims[mode], R)
        # rows of the view from its reference segment table
        rows = np.repeat(v["blk_row"], v["blk_cnt"]).astype(np.int64)
        starts = np.flatnonzero(np.r_[True, rows[1:] != rows[:-1]])
        ends = np.r_[starts[1:], len(rows)]
        br, bs, bc = [], [], []
        for a, b in zip(starts, ends):
            if split == "rows":
                cuts = [a, b]
            else:
                cuts = [a]
                while cuts[-1] < b:
                    cuts.append(min(b, cuts[-1] + int(rng.integers(1, 3001))))
            for x, y in zip(cuts[:-1], cuts[1:]):
                br.append(rows[a]); bs.append(x); bc.append(y - x)
        assert max(bc) > 1024
        seg = [to_dev(ca, np.asarray(a, np.uint32)) for a in (br, bs, bc)]
        dc, dv = to_dev(ca, v["coords"]), to_dev(ca, v["vals"])
        out = zeros(ca, (dims[mode], R))
        F1 = dF[1] if mode == 0 else dF[0]
        F2 = dF[1] if mode == 2 else dF[2]
        rc = ca.lib.cptc_mttkrp_sparse3(mode, dc.data_ptr(), dv.data_ptr(), seg[0].data_ptr(),
                                        seg[1].data_ptr(), seg[2].data_ptr(), len(br),
                                        F1.data_ptr(), F2.data_ptr(), out.data_ptr(), R,
                                        stream(ca))
        assert rc == 0, ca.lib.cptc_last_error()
        ca.sync()
        assert rel_err(out.numpy(), ref) <= 1e-10, (mode, R, split)


def test_sparse_mttkrp_misaligned_factor_base(ca, orc, dev):
    """Factor bases that are only 8-byte aligned take the scalar path."""
    R, dims = 16, (200, 150, 300)
    t, views = zipf_views(ca, orc, dims, 20000, 4)
    rng = np.random.default_rng(0)
    F = [rng.random((d, R)) for d in dims]
    ref = orc.mttkrp3_view(views, 0, F[0].ravel(), F[1].ravel(), F[2].ravel(), R,
                           dims[0]).reshape(dims[0], R)
    big = to_dev(ca, np.concatenate([[0.0], F[1].ravel(), F[2].ravel()]))
    F1p = big.data_ptr() + 8
    F2p = F1p + F[1].size * 8
    v = views[0]
    dc, dv = to_dev(ca, v["coords"]), to_dev(ca, v["vals"])
    br, bs, bc = (to_dev(ca, v[k]) for k in ("blk_row", "blk_start", "blk_cnt"))
    out = zeros(ca, (dims[0], R))
    assert ca.lib.cptc_mttkrp_sparse3(0, dc.data_ptr(), dv.data_ptr(), br.data_ptr(),
                                      bs.data_ptr(), bc.data_ptr(), len(v["blk_row"]), F1p, F2p,
                                      out.data_ptr(), R, stream(ca)) == 0
    ca.sync()
    assert rel_err(out.numpy(), ref) <= 1e-10


def block_tensor(rng, dims, fill=0.5):
    cells = np.array(np.meshgrid(np.arange(0, 32), np.arange(16, 48), np.arange(0, dims[2]),
                                 indexing="ij")).reshape(3, -1)
    cells = cells[:, (cells[0] < dims[0]) & (cells[1] < dims[1])]
    keep = rng.random(cells.shape[1]) < fill
    bg = np.stack([rng.integers(0, d, 3000) for d in dims])
    idx = np.concatenate([cells[:, keep], bg], axis=1).astype(np.int32)
    lin = np.ravel_multi_index(tuple(idx), dims)
    _, first = np.unique(lin, return_index=True)
    idx = idx[:, np.sort(first)]
    return idx, rng.standard_normal(idx.shape[1])


def tile_groups(ca, hdr, words, slot, G):
    import ctypes as C
    n = hdr.shape[0]
    order = np.zeros(n, np.uint32)
    off = np.zeros(n + 1, np.uint32)
    ng = C.c_size_t()
    assert ca.lib.cptc_dense_groups(np.ascontiguousarray(hdr, np.int32).ctypes.data, words, n,
                                    slot, G, order.ctypes.data, off.ctypes.data,
                                    C.byref(ng)) == 0
    return to_dev(ca, order), to_dev(ca, off[:ng.value + 1].copy()), ng.value


@pytest.mark.parametrize("R,G", [(8, 0), (32, 0), (32, 8), (64, 4), (100, 8), (128, 0), (128, 8)])
def test_merged_mttkrp_vs_oracle(ca, orc, dev, R, G):
    """cptc_mttkrp_merged3 (dense.cu:1914-2058, 2258-2511): tiles and residual
    segments of a mode in one grid = the oracle's tiles + view MTTKRP
    (<= 1e-5, the MFMA bound), grouped (G tiles per wave) and per tile."""
    rng = np.random.default_rng(70 + R + G)
    dims = (40, 45, 37)
    idx, val = block_tensor(rng, dims)
    p = orc.partition3(idx[0], idx[1], idx[2], val, dims, 0.03)
    nt = len(p["tiles"])
    assert nt >= 4 and len(p["sp_val"]) > 500
    v = orc.views3(p["sp_i"], p["sp_j"], p["sp_k"], p["sp_val"], dims)
    F = [rng.random((d, R)) - 0.3 for d in dims]
    dF = [to_dev(ca, f) for f in F]
    tiles = to_dev(ca, p["tiles"].astype(np.int32))
    off, lid, pv = to_dev(ca, p["pool_off"]), to_dev(ca, p["pool_lid"]), to_dev(ca, p["pool_val"])
    tf = zeros(ca, (nt * 4096,), np.float32)
    assert ca.lib.cptc_dense_tiles_pack3(lid.data_ptr(), pv.data_ptr(), off.data_ptr(), nt,
                                         tf.data_ptr(), stream(ca)) == 0
    for mode in range(3):
        ref = orc.mttkrp3_tiles(p, mode, F[0].ravel(), F[1].ravel(), F[2].ravel(), R, dims)
        ref = (ref + orc.mttkrp3_view(v, mode, F[0].ravel(), F[1].ravel(), F[2].ravel(), R,
                                      dims[mode])).reshape(dims[mode], R)
        vm = v[mode]
        dc, dv = to_dev(ca, vm["coords"]), to_dev(ca, vm["vals"])
        br, bs, bc = (to_dev(ca, vm[k]) for k in ("blk_row", "blk_start", "blk_cnt"))
        grp = (None, None, 0)
        if G:
            go, gf, ng = tile_groups(ca, p["tiles"], 4, mode, G)
            grp = (go.data_ptr(), gf.data_ptr(), ng)
        out = zeros(ca, (dims[mode], R))
        rc = ca.lib.cptc_mttkrp_merged3(mode, tiles.data_ptr(), tf.data_ptr(), nt, *grp,
                                        dc.data_ptr(), dv.data_ptr(), br.data_ptr(),
                                        bs.data_ptr(), bc.data_ptr(), len(vm["blk_row"]),
                                        dF[0].data_ptr(), dF[1].data_ptr(), dF[2].data_ptr(),
                                        out.data_ptr(), R, *dims, stream(ca))
        assert rc == 0, ca.lib.cptc_last_error()
        ca.sync()
        assert rel_err(out.numpy(), ref) <= 1e-5, (mode, R, G)
    # only one side present: the grid degenerates to that side
    out = zeros(ca, (dims[0], R))
    assert ca.lib.cptc_mttkrp_merged3(0, tiles.data_ptr(), tf.data_ptr(), nt, None, None, 0, None,
                                      None, None, None, None, 0, dF[0].data_ptr(),
                                      dF[1].data_ptr(), dF[2].data_ptr(), out.data_ptr(), R,
                                      *dims, stream(ca)) == 0
    ca.sync()
    ref = orc.mttkrp3_tiles(p, 0, F[0].ravel(), F[1].ravel(), F[2].ravel(), R, dims)
    assert rel_err(out.numpy(), ref.reshape(dims[0], R)) <= 1e-5


def test_merged_rejects_odd_rank(ca, dev):
    d = zeros(ca, (16,))
    rc = ca.lib.cptc_mttkrp_merged3(0, None, None, 0, None, None, 0, None, None, None, None, None,
                                    0, d.data_ptr(), d.data_ptr(), d.data_ptr(), d.data_ptr(), 33,
                                    4, 4, 4, stream(ca))
    assert rc != 0 and b"even R" in ca.lib.cptc_last_error()


@pytest.mark.parametrize("kern", ["fp32", "bf16x3"])
@pytest.mark.parametrize("R,G", [(8, 0), (16, 0), (20, 0), (32, 0), (128, 0), (8, 3), (32, 8),
                                 (128, 8), (200, 8), (64, 2), (100, 8)])
def test_dense_tiles_mfma_vs_fp64(ca, orc, dev, R, G, kern):
    """FP32 MFMA kernel (cptc_mttkrp_dense_tiles3) and split-bf16 kernel
    (cptc_mttkrp_dense_tiles3_ws) against the FP64 oracle of the tile sum,
    <= 1e-5 relative, boundary tiles in every mode, grouped and per tile."""
    rng = np.random.default_rng(50 + R)
    dims = (40, 45, 37)               # boundary tiles in every mode
    idx, val = block_tensor(rng, dims)
    p = orc.partition3(idx[0], idx[1], idx[2], val, dims, 0.03)
    nt = len(p["tiles"])
    assert nt >= 4
    F = [rng.random((d, R)) - 0.3 for d in dims]
    dF = [to_dev(ca, f) for f in F]
    tiles = to_dev(ca, p["tiles"].astype(np.int32))
    off = to_dev(ca, p["pool_off"])
    lid = to_dev(ca, p["pool_lid"])
    pv = to_dev(ca, p["pool_val"])
    tf = zeros(ca, (nt * 4096,), np.float32)
    assert ca.lib.cptc_dense_tiles_pack3(lid.data_ptr(), pv.data_ptr(), off.data_ptr(), nt,
                                         tf.data_ptr(), stream(ca)) == 0
    for mode in range(3):
        ref = orc.mttkrp3_tiles(p, mode, F[0].ravel(), F[1].ravel(), F[2].ravel(), R,
                                dims).reshape(dims[mode], R)
        out = zeros(ca, (dims[mode], R))
        grp = (None, None, 0)
        if G:
            go, gf, ng = tile_groups(ca, p["tiles"], 4, mode, G)
            grp = (go.data_ptr(), gf.data_ptr(), ng)
        if kern == "fp32":
            rc = ca.lib.cptc_mttkrp_dense_tiles3(mode, tiles.data_ptr(), tf.data_ptr(), nt, *grp,
                                                 dF[0].data_ptr(), dF[1].data_ptr(),
                                                 dF[2].data_ptr(), out.data_ptr(), R, *dims,
                                                 stream(ca))
        else:
            nb = ca.lib.cptc_tile_operands_bytes(max(dims), R)
            ws = zeros(ca, (nb,), np.uint8)
            rc = ca.lib.cptc_mttkrp_dense_tiles3_ws(mode, tiles.data_ptr(), tf.data_ptr(), nt,
                                                    *grp, dF[0].data_ptr(), dF[1].data_ptr(),
                                                    dF[2].data_ptr(), out.data_ptr(), R, *dims,
                                                    ws.data_ptr(), nb, stream(ca))
        assert rc == 0, ca.lib.cptc_last_error()
        ca.sync()
        assert rel_err(out.numpy(), ref) <= 1e-5, (mode, R)


def bf16_rne(x):
    """float32 -> bf16 bits, round to nearest even (finite inputs)."""
    b = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


def split_image(img, slot):
    """numpy restatement of one slot's compacted split image: tile cell
    (a, w, c) of the [i][j][k] image, 4-cell segments (a, w, e), bf16 hi of
    the value clamped to the bf16 range, bf16 lo of the float32 remainder."""
    nt = img.shape[0]
    t = img.reshape(nt, 16, 16, 16)
    A = {0: t.transpose(0, 1, 3, 2), 1: t.transpose(0, 2, 3, 1), 2: t.transpose(0, 3, 2, 1)}[slot]
    cells = np.ascontiguousarray(A).reshape(nt, 1024, 4)
    occ = cells.view(np.uint32).any(axis=2)
    bmax = np.float32(3.38953139e38)
    hi = bf16_rne(np.clip(cells, -bmax, bmax))
    hif = (hi.astype(np.uint32) << 16).view(np.float32)
    lo = bf16_rne((cells - hif).astype(np.float32))
    seg = np.concatenate([hi, lo], axis=2)                    # (nt, 1024, 8) bf16 bits
    return occ, seg


@pytest.mark.parametrize("R,G", [(32, 0), (128, 8), (100, 3), (200, 0)])
def test_dense_tiles_compact_image(ca, orc, dev, R, G):
    """The compacted split image of each target slot
    (cptc_dense_tiles_compact3_mask / _fill): occupancy words, running counts,
    segment offsets and the packed bf16 hi / lo segments equal a numpy
    construction from the dense image (its own round-to-nearest-even bf16
    split); the split-bf16 kernel over it (cptc_mttkrp_dense_tiles3_cws) gives
    the dense-image kernel's results (which split on every launch) up to the
    order of the FP64 atomic adds, every mode, grouped and per tile."""
    rng = np.random.default_rng(90 + R)
    dims = (40, 45, 37)
    idx, val = block_tensor(rng, dims, fill=0.15)
    p = orc.partition3(idx[0], idx[1], idx[2], val, dims, 0.03)
    nt = len(p["tiles"])
    assert nt >= 4
    F = [rng.random((d, R)) - 0.3 for d in dims]
    dF = [to_dev(ca, f) for f in F]
    tiles = to_dev(ca, p["tiles"].astype(np.int32))
    tf = zeros(ca, (nt * 4096,), np.float32)
    pools = [to_dev(ca, p[k]) for k in ("pool_lid", "pool_val", "pool_off")]
    assert ca.lib.cptc_dense_tiles_pack3(*(b.data_ptr() for b in pools), nt, tf.data_ptr(),
                                         stream(ca)) == 0
    ca.sync()
    img = tf.numpy().reshape(nt, 4096)
    nb = ca.lib.cptc_tile_operands_bytes(max(dims), R)
    ws = zeros(ca, (nb,), np.uint8)
    for mode in range(3):
        cm = zeros(ca, (nt * 64,), np.uint32)
        so = zeros(ca, (nt + 1,), np.uint32)
        tot = C.c_uint64()
        assert ca.lib.cptc_dense_tiles_compact3_mask(tf.data_ptr(), nt, mode, cm.data_ptr(),
                                                     so.data_ptr(), C.byref(tot), stream(ca)) == 0
        nseg = tot.value
        seg = zeros(ca, (max(nseg, 1) * 8,), np.uint16)
        assert ca.lib.cptc_dense_tiles_compact3_fill(tf.data_ptr(), nt, mode, cm.data_ptr(),
                                                     so.data_ptr(), seg.data_ptr(),
                                                     stream(ca)) == 0
        ca.sync()
        occ, ref_seg = split_image(img, mode)
        bits = occ.reshape(nt, 32, 32).astype(np.uint64) << np.arange(32, dtype=np.uint64)
        words = bits.sum(axis=2).astype(np.uint32)
        run = np.concatenate([np.zeros((nt, 1), np.uint32),
                              np.cumsum(occ.reshape(nt, 32, 32).sum(axis=2), axis=1)[:, :-1]],
                             axis=1).astype(np.uint32)
        got_m = cm.numpy().reshape(nt, 64)
        assert np.array_equal(got_m[:, :32], words) and np.array_equal(got_m[:, 32:], run), mode
        cnt = occ.sum(axis=1)
        assert nseg == int(cnt.sum()) and 0 < nseg < nt * 1024
        assert np.array_equal(so.numpy(), np.concatenate([[0], np.cumsum(cnt)]).astype(np.uint32))
        assert np.array_equal(seg.numpy()[:nseg * 8].reshape(nseg, 8), ref_seg[occ]), mode
        grp = (None, None, 0)
        if G:
            go, gf, ng = tile_groups(ca, p["tiles"], 4, mode, G)
            grp = (go.data_ptr(), gf.data_ptr(), ng)
        outs = []
        for compact in (False, True):
            out = zeros(ca, (dims[mode], R))
            if compact:
                rc = ca.lib.cptc_mttkrp_dense_tiles3_cws(
                    mode, tiles.data_ptr(), cm.data_ptr(), so.data_ptr(), seg.data_ptr(), nseg,
                    nt, *grp, dF[0].data_ptr(), dF[1].data_ptr(), dF[2].data_ptr(),
                    out.data_ptr(), R, *dims, ws.data_ptr(), nb, stream(ca))
            else:
                rc = ca.lib.cptc_mttkrp_dense_tiles3_ws(
                    mode, tiles.data_ptr(), tf.data_ptr(), nt, *grp, dF[0].data_ptr(),
                    dF[1].data_ptr(), dF[2].data_ptr(), out.data_ptr(), R, *dims, ws.data_ptr(),
                    nb, stream(ca))
            assert rc == 0, ca.lib.cptc_last_error()
            ca.sync()
            outs.append(out.numpy())
        ref = orc.mttkrp3_tiles(p, mode, F[0].ravel(), F[1].ravel(), F[2].ravel(), R,
                                dims).reshape(dims[mode], R)
        assert rel_err(outs[1], ref) <= 1e-5, (mode, R)
        # the same FP64 contributions; only the order of the atomic adds differs
        assert rel_err(outs[1], outs[0]) <= 1e-14, (mode, R)


def test_dense_tiles_bf16x3_split_error(ca, orc, dev):
    """The split-bf16 kernel's error is that of ~16-bit inputs (each operand
    kept to ~2^-17 by its two bf16 terms): inside the 1e-5 bar with
    zero-mean factors, whose sums cancel (measured 4.4-4.6e-6 here), and
    far below plain bf16 (2^-9 per operand); a dropped split term (hi*lo or
    lo*hi) would leave ~1e-3.  A workspace that is too small is an error,
    not a fault."""
    rng = np.random.default_rng(77)
    dims = (48, 40, 44)
    idx, val = block_tensor(rng, dims)
    p = orc.partition3(idx[0], idx[1], idx[2], val, dims, 0.03)
    nt = len(p["tiles"])
    R = 64
    F = [rng.standard_normal((d, R)) for d in dims]
    dF = [to_dev(ca, f) for f in F]
    tiles = to_dev(ca, p["tiles"].astype(np.int32))
    tf = zeros(ca, (nt * 4096,), np.float32)
    pools = [to_dev(ca, p[k]) for k in ("pool_lid", "pool_val", "pool_off")]   # kept alive
    assert ca.lib.cptc_dense_tiles_pack3(*(b.data_ptr() for b in pools), nt, tf.data_ptr(),
                                         stream(ca)) == 0
    nb = ca.lib.cptc_tile_operands_bytes(max(dims), R)
    ws = zeros(ca, (nb,), np.uint8)
    errs = []
    for mode in range(3):
        ref = orc.mttkrp3_tiles(p, mode, F[0].ravel(), F[1].ravel(), F[2].ravel(), R,
                                dims).reshape(dims[mode], R)
        out = zeros(ca, (dims[mode], R))
        assert ca.lib.cptc_mttkrp_dense_tiles3_ws(mode, tiles.data_ptr(), tf.data_ptr(), nt, None,
                                                  None, 0, dF[0].data_ptr(), dF[1].data_ptr(),
                                                  dF[2].data_ptr(), out.data_ptr(), R, *dims,
                                                  ws.data_ptr(), nb, stream(ca)) == 0
        ca.sync()
        errs.append(rel_err(out.numpy(), ref))
    assert max(errs) <= 1e-5, errs
    out = zeros(ca, (dims[0], R))
    rc = ca.lib.cptc_mttkrp_dense_tiles3_ws(0, tiles.data_ptr(), tf.data_ptr(), nt, None, None, 0,
                                            dF[0].data_ptr(), dF[1].data_ptr(), dF[2].data_ptr(),
                                            out.data_ptr(), R, *dims, ws.data_ptr(), nb // 4,
                                            stream(ca))
    assert rc != 0 and b"workspace" in ca.lib.cptc_last_error()


def _bf16_rne(x):
    """float32 -> bf16 bits, round to nearest even (finite values)."""
    b = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint32)


def _operand_images(F, dim, R, Rq):
    """The split-bf16 kernel's operand images of a factor, restated: as the
    contracted factor, 8-row blocks of one rank, each 16-byte entry the bf16
    hi halves of its 8 float32 values (pairs packed low | high << 16), and
    the same for the lo halves bf16(x - hi); as the weight factor, 16-row
    blocks of one rank in float32.  Rows past the factor and ranks >= R are 0."""
    x = np.zeros((((dim + 15) // 16) * 16, Rq), np.float32)
    x[:dim, :R] = F.astype(np.float32)
    hi = _bf16_rne(x)
    lo = _bf16_rne(x - (hi << 16).view(np.float32))
    def pack(h):   # [row / 8][Rq] entries of 4 words: rows 8b + 2s (low), 8b + 2s + 1 (high)
        h = h.reshape(-1, 8, Rq).transpose(0, 2, 1).reshape(-1, 4, 2)
        return (h[..., 0] | (h[..., 1] << 16)).ravel()
    fw = x.reshape(-1, 16, Rq).transpose(0, 2, 1).ravel()
    return pack(hi), pack(lo), fw


def test_dense_tiles_operand_images(ca, orc, dev):
    """The operand images the split-bf16 kernel builds per launch (left in
    its workspace) equal a numpy restatement bit for bit: the contracted
    factor's bf16 hi / lo split (round to nearest even) and the weight
    factor in float32, padded rows and ranks zero (R = 40 pads to 64, dims
    not multiples of 16).  One of the two other factors of the mode must be
    the contracted one and the other the weight."""
    rng = np.random.default_rng(5)
    dims = (40, 37, 50)
    idx, val = block_tensor(rng, dims)
    p = orc.partition3(idx[0], idx[1], idx[2], val, dims, 0.03)
    nt = len(p["tiles"])
    R, Rq = 40, 64
    F = [rng.standard_normal((d, R)) for d in dims]
    dF = [to_dev(ca, f) for f in F]
    tiles = to_dev(ca, p["tiles"].astype(np.int32))
    tf = zeros(ca, (nt * 4096,), np.float32)
    pools = [to_dev(ca, p[k]) for k in ("pool_lid", "pool_val", "pool_off")]   # kept alive
    assert ca.lib.cptc_dense_tiles_pack3(*(b.data_ptr() for b in pools), nt, tf.data_ptr(),
                                         stream(ca)) == 0
    nb = ca.lib.cptc_tile_operands_bytes(max(dims), R)
    imgs = [_operand_images(F[m], dims[m], R, Rq) for m in range(3)]
    for mode in range(3):
        ws = zeros(ca, (nb,), np.uint8)
        out = zeros(ca, (dims[mode], R))
        assert ca.lib.cptc_mttkrp_dense_tiles3_ws(mode, tiles.data_ptr(), tf.data_ptr(), nt, None,
                                                  None, 0, dF[0].data_ptr(), dF[1].data_ptr(),
                                                  dF[2].data_ptr(), out.data_ptr(), R, *dims,
                                                  ws.data_ptr(), nb, stream(ca)) == 0
        ca.sync()
        w = ws.numpy()
        o = [m for m in range(3) if m != mode]
        ok = False
        for c, wt in ((o[0], o[1]), (o[1], o[0])):
            hi, lo, fw = imgs[c]
            n = hi.size * 4
            got_hi = w[:n].view(np.uint32)
            got_lo = w[n:2 * n].view(np.uint32)
            got_fw = w[2 * n:2 * n + imgs[wt][2].size * 4].view(np.float32)
            if (np.array_equal(got_hi, hi) and np.array_equal(got_lo, lo)
                    and np.array_equal(got_fw.view(np.uint32), imgs[wt][2].view(np.uint32))):
                ok = True
        assert ok, mode


def test_dense_tile_pack_last_write_wins(ca, orc, dev):
    rng = np.random.default_rng(1)
    cells = np.array(np.meshgrid(*[np.arange(16)] * 3, indexing="ij")).reshape(3, -1)
    idx = np.concatenate([cells, cells[:, :300]], axis=1).astype(np.int32)
    val = rng.standard_normal(idx.shape[1])
    val[5] = 1e300                                   # clamped to FLT_MAX
    p = orc.partition3(idx[0], idx[1], idx[2], val, (16, 16, 16), 0.5)
    tf = zeros(ca, (4096,), np.float32)
    args = [to_dev(ca, p[k]) for k in ("pool_lid", "pool_val", "pool_off")]
    assert ca.lib.cptc_dense_tiles_pack3(*(a.data_ptr() for a in args), 1, tf.data_ptr(),
                                         stream(ca)) == 0
    ca.sync()
    X = np.zeros((16, 16, 16))
    X[tuple(idx)] = np.clip(val, -np.finfo(np.float32).max, np.finfo(np.float32).max)
    assert np.array_equal(tf.numpy(), X.ravel().astype(np.float32))


@pytest.mark.parametrize("rows,R", [(1, 1), (1000, 7), (28818, 128), (5000, 200), (0, 16),
                                    (300, 65), (9184, 100), (1, 128), (37, 96), (64, 66),
                                    (12092, 128), (129, 512)])
def test_gram(ca, dev, rows, R):
    """cptc_gram against numpy; above R = 64 (the FP64 matrix-core partials)
    only the entries on and above the diagonal are summed and the rest
    mirrored, so G must also be exactly symmetric.  Ragged row ranges (rows
    not a multiple of a batch, fewer rows than one partial) and ragged R."""
    F = np.random.default_rng(rows + R).standard_normal((rows, R))
    dF = to_dev(ca, F)
    G = zeros(ca, (R, R))
    assert ca.lib.cptc_gram(dF.data_ptr(), rows, R, G.data_ptr(), stream(ca)) == 0
    ca.sync()
    assert rel_err(G.numpy(), F.T @ F) < 1e-13 if rows else np.all(G.numpy() == 0)
    assert np.array_equal(G.numpy(), G.numpy().T)


@pytest.mark.parametrize("R,dim", [(64, 100), (65, 1), (65, 77), (100, 1000), (127, 63),
                                   (128, 28818), (128, 17), (129, 300)])
def test_apply_pinv_vs_numpy(ca, dev, R, dim):
    """cptc_apply_pinv: F = Y Ainv / div (the per-entry kernel up to R = 64,
    the 64 x 64 tiled one above) against numpy, with ragged R and row counts
    (partial tiles), with and without the divisor."""
    rng = np.random.default_rng(R * 1000 + dim)
    Y = rng.standard_normal((dim, R))
    A = rng.standard_normal((R, R))
    div = rng.random(R) + 0.5
    dY, dA, dd = to_dev(ca, Y), to_dev(ca, A), to_dev(ca, div)
    for use_div in (True, False):
        out = zeros(ca, (dim, R))
        assert ca.lib.cptc_apply_pinv(dY.data_ptr(), dA.data_ptr(), out.data_ptr(), dim, R,
                                      dd.data_ptr() if use_div else None, stream(ca)) == 0
        ca.sync()
        ref = Y @ A
        if use_div:
            ref = ref / div
        assert rel_err(out.numpy(), ref) < 1e-13, use_div


@pytest.mark.parametrize("R", [1, 5, 16, 17, 32, 33, 63, 64, 65, 100, 128, 129, 200])
def test_solve_pinv_spd(ca, dev, R):
    rng = np.random.default_rng(R)
    Fa, Fb = rng.random((3 * R + 20, R)), rng.random((2 * R + 30, R))
    A = (Fa.T @ Fa) * (Fb.T @ Fb)
    dim = 777
    Y = rng.standard_normal((dim, R))
    lam = rng.random(R) + 0.5
    dA, dY, dl = to_dev(ca, A), to_dev(ca, Y), to_dev(ca, lam)
    out = zeros(ca, (dim, R))
    path = zeros(ca, (1,), np.int32)
    Ainv = zeros(ca, (R, R))
    assert ca.lib.cptc_pinv_sym(dA.data_ptr(), Ainv.data_ptr(), R, path.data_ptr(),
                                stream(ca)) == 0
    assert ca.lib.cptc_solve_pinv(dA.data_ptr(), dY.data_ptr(), out.data_ptr(), dim, R,
                                  dl.data_ptr(), stream(ca)) == 0
    ca.sync()
    assert int(path.numpy()[0]) == 0                    # Cholesky fast path
    inv = np.linalg.inv(A)
    assert rel_err(Ainv.numpy(), inv) < 1e-9
    assert rel_err(out.numpy(), (Y @ inv) / lam) < 1e-9


@pytest.mark.parametrize("R", [24, 64, 100])
def test_pinv_singular_takes_jacobi_path(ca, orc, dev, R):
    """Rank-deficient FtF: the fast path (register sweep for R <= 64, blocked
    Cholesky above) hands over to the Jacobi pseudoinverse."""
    rng = np.random.default_rng(3)
    F = rng.random((max(60, 2 * R), R))
    F[:, 7] = F[:, 3]
    F[:, 11] = 0.0
    F[:, R - 1] = F[:, 0]
    A = F.T @ F
    dA = to_dev(ca, A)
    Ainv = zeros(ca, (R, R))
    path = zeros(ca, (1,), np.int32)
    assert ca.lib.cptc_pinv_sym(dA.data_ptr(), Ainv.data_ptr(), R, path.data_ptr(),
                                stream(ca)) == 0
    ca.sync()
    assert int(path.numpy()[0]) == 1
    P = Ainv.numpy()
    ref, _ = orc.pinv_sym(A.ravel(), R)
    assert rel_err(P, ref.reshape(R, R)) < 1e-8
    assert rel_err(A @ P @ A, A) < 1e-10
    assert rel_err(P @ A @ P, P) < 1e-8


@pytest.mark.parametrize("R,c,scale", [(16, 3.0, 1.0), (32, 1.0, 1.0), (64, 1.0, 1e-3),
                                         (128, 1.0, 1.0), (128, 1.0, 1e6)])
def test_pinv_kahan_type_truncates(ca, orc, dev, R, c, scale):
    """A = s L L^T, L unit lower triangular with every sub-diagonal entry -c:
    every LDL^T pivot is s (no pivot test fires) but one eigenvalue lies far
    below R ulp(sigma_max), so the reference's truncated pseudoinverse
    (solver.cu:900-1002) drops it and the plain inverse (entries ~ (1+c)^(2R))
    is wrong.  The fast path must hand over to the Jacobi pseudoinverse."""
    L = np.eye(R) + np.tril(np.full((R, R), -c), -1)
    A = scale * (L @ L.T)
    w = np.linalg.eigvalsh(A)
    tol = R * np.spacing(w.max())
    assert np.sum(w <= tol) == 1 and np.sort(w)[1] > 1e6 * tol   # one dropped, clear gap
    dA = to_dev(ca, A)
    Ainv = zeros(ca, (R, R))
    path = zeros(ca, (1,), np.int32)
    assert ca.lib.cptc_pinv_sym(dA.data_ptr(), Ainv.data_ptr(), R, path.data_ptr(),
                                stream(ca)) == 0
    ca.sync()
    assert int(path.numpy()[0]) == 1
    P = Ainv.numpy()
    ref, _ = orc.pinv_sym(A.ravel(), R)
    ref = ref.reshape(R, R)
    assert np.linalg.norm(P, 2) < 1.0 / tol                   # truncated, not the inverse
    assert rel_err(P, ref) < 1e-8
    assert rel_err(P @ A @ P, P) < 1e-8
    # the solve entry point takes the same path
    dim = 300
    Y = np.random.default_rng(R).standard_normal((dim, R))
    lam = np.ones(R)
    dY, dl = to_dev(ca, Y), to_dev(ca, lam)
    out = zeros(ca, (dim, R))
    assert ca.lib.cptc_solve_pinv(dA.data_ptr(), dY.data_ptr(), out.data_ptr(), dim, R,
                                  dl.data_ptr(), stream(ca)) == 0
    ca.sync()
    assert rel_err(out.numpy(), Y @ ref) < 1e-8


@pytest.mark.parametrize("R", [32, 128])
def test_pinv_moderately_ill_conditioned_stays_fast(ca, dev, R):
    """kappa ~ 1e8: far from truncation, so the fast path keeps the inverse."""
    rng = np.random.default_rng(40 + R)
    Q, _ = np.linalg.qr(rng.standard_normal((R, R)))
    A = (Q * np.logspace(0, -8, R)) @ Q.T
    A = 0.5 * (A + A.T)
    dA = to_dev(ca, A)
    Ainv = zeros(ca, (R, R))
    path = zeros(ca, (1,), np.int32)
    assert ca.lib.cptc_pinv_sym(dA.data_ptr(), Ainv.data_ptr(), R, path.data_ptr(),
                                stream(ca)) == 0
    ca.sync()
    assert int(path.numpy()[0]) == 0
    # a backward-stable inverse leaves ||P A - I|| ~ kappa * eps * R = 1e8 * 2.2e-16 * R
    assert rel_err(Ainv.numpy() @ A, np.eye(R)) < 1e-4
    assert rel_err(Ainv.numpy(), np.linalg.inv(A)) < 1e-4


def test_norms_normalize_fit(ca, dev):
    rng = np.random.default_rng(8)
    rows, R = 3001, 32
    F = rng.standard_normal((rows, R))
    F[:, 4] = 0.0                                    # zero column: n < 1e-14
    M = rng.standard_normal((rows, R))
    lam = rng.random(R) + 0.1
    dF, dM, dl = to_dev(ca, F), to_dev(ca, M), to_dev(ca, lam)
    n = zeros(ca, (R,))
    assert ca.lib.cptc_colnorms(dF.data_ptr(), rows, R, n.data_ptr(), stream(ca)) == 0
    assert ca.lib.cptc_normalize_absorb(dF.data_ptr(), rows, R, n.data_ptr(), dl.data_ptr(),
                                        stream(ca)) == 0
    ca.sync()
    nr = np.sqrt(np.sum(F * F, axis=0))
    assert rel_err(n.numpy(), nr) < 1e-14
    Fn = np.where(nr < 1e-14, 0.0, F / np.where(nr < 1e-14, 1, nr))
    assert rel_err(dF.numpy(), Fn) < 1e-14
    assert rel_err(dl.numpy(), np.where(nr < 1e-14, 0.0, lam * nr)) < 1e-14
    G = [rng.random((R, R)) for _ in range(3)]
    dG = to_dev(ca, np.concatenate([g.ravel() for g in G]))
    out = zeros(ca, (2,))
    lam2 = dl.numpy()
    assert ca.lib.cptc_fit_gram(dF.data_ptr(), dM.data_ptr(), rows, dl.data_ptr(), dG.data_ptr(),
                                3, R, out.data_ptr(), stream(ca)) == 0
    ca.sync()
    ip = np.sum(lam2 * np.sum(Fn * M, axis=0))
    md = np.sum(np.outer(lam2, lam2) * G[0] * G[1] * G[2])
    o = out.numpy()
    assert abs(o[0] - ip) < 1e-10 * abs(ip) and abs(o[1] - md) < 1e-12 * abs(md)


@pytest.mark.parametrize("R", [8, 128, 200])
def test_gram_normalize_absorb_matches_steps(ca, dev, R):
    """The fused Gram + normalise + absorb equals colnorms, normalize_absorb
    and gram run one after another (zero column included)."""
    rng = np.random.default_rng(R)
    rows = 2003
    F = rng.standard_normal((rows, R))
    F[:, 3] = 0.0
    lam = rng.random(R) + 0.1
    a_F, a_l = to_dev(ca, F), to_dev(ca, lam)
    n1, G1 = zeros(ca, (R,)), zeros(ca, (R, R))
    assert ca.lib.cptc_colnorms(a_F.data_ptr(), rows, R, n1.data_ptr(), stream(ca)) == 0
    assert ca.lib.cptc_normalize_absorb(a_F.data_ptr(), rows, R, n1.data_ptr(), a_l.data_ptr(),
                                        stream(ca)) == 0
    assert ca.lib.cptc_gram(a_F.data_ptr(), rows, R, G1.data_ptr(), stream(ca)) == 0
    b_F, b_l = to_dev(ca, F), to_dev(ca, lam)
    n2, G2 = zeros(ca, (R,)), zeros(ca, (R, R))
    assert ca.lib.cptc_gram_normalize_absorb(b_F.data_ptr(), rows, R, G2.data_ptr(),
                                             n2.data_ptr(), b_l.data_ptr(), stream(ca)) == 0
    ca.sync()
    nr = np.sqrt(np.sum(F * F, axis=0))
    assert rel_err(n2.numpy(), nr) < 1e-14
    assert rel_err(b_F.numpy(), a_F.numpy()) < 1e-14
    assert rel_err(b_l.numpy(), a_l.numpy()) < 1e-14
    assert rel_err(G2.numpy(), G1.numpy()) < 1e-13
    Fn = b_F.numpy()
    assert rel_err(G2.numpy(), Fn.T @ Fn) < 1e-13
    assert np.all(G2.numpy()[3] == 0.0) and np.all(G2.numpy()[:, 3] == 0.0)


@pytest.mark.parametrize("R,rows", [(1, 5), (8, 2003), (17, 64), (32, 512), (32, 1), (33, 700),
                                    (100, 3001), (128, 28818), (128, 1)])
def test_gram_normalize_absorb_next(ca, dev, R, rows):
    """cptc_gram_normalize_absorb_next (one workgroup for R <= 32; above that
    the Gram launches, then the norms, normalisation and FtF in one) gives
    cptc_gram_normalize_absorb's factor, norms, lambda and Gram bit for bit,
    and with d_other the next mode's FtF equal to cptc_hadamard of the new Gram
    and the other one (zero column included)."""
    rng = np.random.default_rng(R * 7 + rows)
    F = rng.standard_normal((rows, R))
    if R > 3:
        F[:, 3] = 0.0
    lam = rng.random(R) + 0.1
    other = rng.standard_normal((R, R))
    a_F, a_l = to_dev(ca, F), to_dev(ca, lam)
    n1, G1, H1 = zeros(ca, (R,)), zeros(ca, (R, R)), zeros(ca, (R, R))
    assert ca.lib.cptc_gram_normalize_absorb(a_F.data_ptr(), rows, R, G1.data_ptr(),
                                             n1.data_ptr(), a_l.data_ptr(), stream(ca)) == 0
    d_o = to_dev(ca, other)
    assert ca.lib.cptc_hadamard(G1.data_ptr(), d_o.data_ptr(), H1.data_ptr(), R * R,
                                stream(ca)) == 0
    for with_next in (True, False):
        b_F, b_l = to_dev(ca, F), to_dev(ca, lam)
        n2, G2, H2 = zeros(ca, (R,)), zeros(ca, (R, R)), zeros(ca, (R, R))
        rc = ca.lib.cptc_gram_normalize_absorb_next(
            b_F.data_ptr(), rows, R, G2.data_ptr(), n2.data_ptr(), b_l.data_ptr(),
            d_o.data_ptr() if with_next else None, H2.data_ptr() if with_next else None,
            stream(ca))
        assert rc == 0, ca.lib.cptc_last_error()
        ca.sync()
        for got, ref in ((b_F, a_F), (n2, n1), (b_l, a_l), (G2, G1)):
            assert np.array_equal(got.numpy(), ref.numpy())
        if with_next:
            assert np.array_equal(H2.numpy(), H1.numpy())
        else:
            assert np.all(H2.numpy() == 0.0)
    assert ca.lib.cptc_gram_normalize_absorb_next(b_F.data_ptr(), rows, 1025, G2.data_ptr(),
                                                  n2.data_ptr(), b_l.data_ptr(), None, None,
                                                  stream(ca)) != 0


@pytest.mark.parametrize("R,rows", [(1, 1), (5, 17), (16, 256), (17, 15), (20, 513),
                                    (31, 1000), (32, 256), (32, 257), (32, 512), (32, 1024),
                                    (3, 129), (32, 4096), (7, 3001), (24, 70), (9, 200)])
def test_update_small3_matches_steps(ca, dev, R, rows):
    """cptc_update_small3 (FP64 matrix cores; up to 256 rows one workgroup
    keeps the factor in registers, above that one 16-row block per wave and
    the last workgroup to finish sums the partials and scales) against the
    separate calls it replaces: cptc_apply_pinv with lambda, then
    cptc_gram_normalize_absorb_next with the next FtF, then cptc_fit_gram on
    the new factor with grams (G_0, G_1, this G), then cptc_pinv_sym of the
    next FtF.  Factor, norms, lambda, G and FtF within 1e-13 (relative,
    2-norm), the fit scalars within 1e-12: the sums run in another order; a
    dropped block, column or rank term shows at 1e-2 and more.  The next
    pinv: `other` SPD makes FtF SPD (Schur product), the one-wave sweep
    accepts it and its inverse equals cptc_pinv_sym of the launch's own FtF
    bit for bit; with a zero row and column in `other` the sweep meets a zero
    pivot and the launch's Jacobi pseudoinverse is within 1e-10 of
    cptc_pinv_sym's.  A zero column of Ainv gives a zero column of F
    (norm < 1e-14): F, lambda and the Gram's row and column are exactly 0.
    FtV[0, nzero) is cleared after its reads and the rest is untouched; a
    call without fit, next FtF or clearing leaves those alone.  Sizes past
    4096 rows or R = 33 are refused.  Calls in a row check that the
    workgroup counter is left at zero."""
    rng = np.random.default_rng(R * 1000 + rows)
    Y = rng.standard_normal((rows, R))
    A = rng.standard_normal((R, R))
    A = A + A.T
    zc = 2 if R > 2 else None
    if zc is not None:
        A[:, zc] = 0.0
    lam = rng.random(R) + 0.1
    B = rng.standard_normal((R, R))
    other = B @ B.T / R + np.eye(R)
    g01 = rng.random((2, R, R))
    dY, dA, do = to_dev(ca, Y), to_dev(ca, A), to_dev(ca, other)
    # the separate calls
    a_F, a_l = zeros(ca, (rows, R)), to_dev(ca, lam)
    n1, G1, H1, out1 = zeros(ca, (R,)), zeros(ca, (R, R)), zeros(ca, (R, R)), zeros(ca, (2,))
    assert ca.lib.cptc_apply_pinv(dY.data_ptr(), dA.data_ptr(), a_F.data_ptr(), rows, R,
                                  a_l.data_ptr(), stream(ca)) == 0
    assert ca.lib.cptc_gram_normalize_absorb_next(a_F.data_ptr(), rows, R, G1.data_ptr(),
                                                  n1.data_ptr(), a_l.data_ptr(), do.data_ptr(),
                                                  H1.data_ptr(), stream(ca)) == 0
    ca.sync()
    g3 = to_dev(ca, np.concatenate([g01.ravel(), G1.numpy().ravel()]))
    assert ca.lib.cptc_fit_gram(a_F.data_ptr(), dY.data_ptr(), rows, a_l.data_ptr(),
                                g3.data_ptr(), 3, R, out1.data_ptr(), stream(ca)) == 0
    # one launch; FtV in a longer buffer, cleared over nzero entries; the
    # next pinv overwrites Ainv
    extra = 40
    Yb = np.concatenate([Y.ravel(), np.full(extra, 7.0)])
    nzero = rows * R + extra // 2
    dYb, dA2 = to_dev(ca, Yb), to_dev(ca, A)
    b_F, b_l = zeros(ca, (rows, R)), to_dev(ca, lam)
    n2, G2, H2, out2 = zeros(ca, (R,)), zeros(ca, (R, R)), zeros(ca, (R, R)), zeros(ca, (2,))
    g01d = to_dev(ca, g01)
    rc = ca.lib.cptc_update_small3(dYb.data_ptr(), dA2.data_ptr(), b_F.data_ptr(), rows, R,
                                   G2.data_ptr(), n2.data_ptr(), b_l.data_ptr(), do.data_ptr(),
                                   H2.data_ptr(), nzero, g01d.data_ptr(), out2.data_ptr(), 1,
                                   stream(ca))
    assert rc == 0, ca.lib.cptc_last_error()
    ca.sync()
    for got, ref in ((b_F, a_F), (n2, n1), (b_l, a_l), (G2, G1), (H2, H1)):
        assert rel_err(got.numpy(), ref.numpy()) <= 1e-13
    o1, o2 = out1.numpy(), out2.numpy()
    assert abs(o2[0] - o1[0]) <= 1e-12 * abs(o1[0]) and abs(o2[1] - o1[1]) <= 1e-12 * abs(o1[1])
    if zc is not None:
        assert np.all(b_F.numpy()[:, zc] == 0.0) and b_l.numpy()[zc] == 0.0
        assert np.all(G2.numpy()[zc] == 0.0) and np.all(G2.numpy()[:, zc] == 0.0)
    assert np.array_equal(G2.numpy(), G2.numpy().T)
    yb = dYb.numpy()
    assert np.all(yb[:nzero] == 0.0) and np.all(yb[nzero:] == 7.0)
    P1 = zeros(ca, (R, R))
    assert ca.lib.cptc_pinv_sym(H2.data_ptr(), P1.data_ptr(), R, None, stream(ca)) == 0
    ca.sync()
    if zc is None:
        assert np.array_equal(dA2.numpy(), P1.numpy())
    else:
        # the zero column of the Gram makes FtF singular: both take Jacobi
        assert rel_err(dA2.numpy(), P1.numpy()) <= 1e-10
    # a zero row and column in `other`: a zero pivot, the launch's Jacobi
    if R > 3:
        o0 = other.copy()
        o0[1, :] = 0.0
        o0[:, 1] = 0.0
        do0, dA3, H3 = to_dev(ca, o0), to_dev(ca, A), zeros(ca, (R, R))
        c_F, c_l, n3, G3 = zeros(ca, (rows, R)), to_dev(ca, lam), zeros(ca, (R,)), zeros(ca, (R, R))
        assert ca.lib.cptc_update_small3(dY.data_ptr(), dA3.data_ptr(), c_F.data_ptr(), rows, R,
                                         G3.data_ptr(), n3.data_ptr(), c_l.data_ptr(),
                                         do0.data_ptr(), H3.data_ptr(), 0, None, None, 1,
                                         stream(ca)) == 0
        P3 = zeros(ca, (R, R))
        assert ca.lib.cptc_pinv_sym(H3.data_ptr(), P3.data_ptr(), R, None, stream(ca)) == 0
        ca.sync()
        assert rel_err(dA3.numpy(), P3.numpy()) <= 1e-10
        assert np.all(dA3.numpy()[1] == 0.0) and np.all(dA3.numpy()[:, 1] == 0.0)
        assert rel_err(c_F.numpy(), a_F.numpy()) <= 1e-13
    # without fit, next FtF, pinv or clearing: those outputs are left alone
    dY2 = to_dev(ca, Y)
    c_l = to_dev(ca, lam)
    n3, G3 = zeros(ca, (R,)), zeros(ca, (R, R))
    assert ca.lib.cptc_update_small3(dY2.data_ptr(), dA.data_ptr(), b_F.data_ptr(), rows, R,
                                     G3.data_ptr(), n3.data_ptr(), c_l.data_ptr(), None, None, 0,
                                     None, None, 0, stream(ca)) == 0
    ca.sync()
    assert rel_err(b_F.numpy(), a_F.numpy()) <= 1e-13
    assert np.array_equal(G3.numpy(), G2.numpy()) and np.array_equal(dY2.numpy(), Y)
    assert np.array_equal(dA.numpy(), A)
    for bad_rows, bad_R, npv in ((4097, R, 0), (rows, 33, 0), (0, R, 0), (rows, R, 1)):
        assert ca.lib.cptc_update_small3(dY2.data_ptr(), dA.data_ptr(), b_F.data_ptr(), bad_rows,
                                         bad_R, G3.data_ptr(), n3.data_ptr(), c_l.data_ptr(),
                                         None, None, 0, None, None, npv, stream(ca)) != 0


@pytest.mark.parametrize("R", [1, 7, 32, 100])
def test_sparse_mttkrp_range(ca, orc, dev, R):
    """compute_sparse_mttkrp_async's sub-range path (sparse.cu:877-955):
    elements [start, start + count) of one mode's view, against a numpy sum
    over the same elements (closed form on the packed coordinates); ranges
    that partition the view add up to the whole-view segment kernel."""
    dims = (500, 300, 900)
    t, views = zipf_views(ca, orc, dims, 30000, 40 + R)
    rng = np.random.default_rng(R)
    F = [rng.standard_normal((d, R)) for d in dims]
    dF = [to_dev(ca, f) for f in F]
    for mode in range(3):
        v = views[mode]
        c = np.asarray(v["coords"], np.uint64)
        i = (c >> np.uint64(30)).astype(np.int64)
        j = ((c >> np.uint64(15)) & np.uint64(0x7FFF)).astype(np.int64)
        k = (c & np.uint64(0x7FFF)).astype(np.int64)
        tgt, o0, o1 = {0: (i, j, k), 1: (j, i, k), 2: (k, i, j)}[mode]
        F1 = F[1] if mode == 0 else F[0]
        F2 = F[1] if mode == 2 else F[2]
        dF1 = dF[1] if mode == 0 else dF[0]
        dF2 = dF[1] if mode == 2 else dF[2]
        dc, dv = to_dev(ca, v["coords"]), to_dev(ca, v["vals"])
        n = len(v["vals"])
        cuts = [0, 1, 977, n // 2, n - 5, n]
        total = zeros(ca, (dims[mode], R))
        for a, b in zip(cuts[:-1], cuts[1:]):
            out = zeros(ca, (dims[mode], R))
            for o in (out, total):
                assert ca.lib.cptc_mttkrp_sparse3_range(mode, dc.data_ptr(), dv.data_ptr(), a,
                                                        b - a, dF1.data_ptr(), dF2.data_ptr(),
                                                        o.data_ptr(), R, stream(ca)) == 0
            ca.sync()
            ref = np.zeros((dims[mode], R))
            np.add.at(ref, tgt[a:b], (np.asarray(v["vals"])[a:b, None] * F1[o0[a:b]]) * F2[o1[a:b]])
            assert rel_err(out.numpy(), ref) <= 1e-12, (mode, a, b)
        full = orc.mttkrp3_view(views, mode, F[0].ravel(), F[1].ravel(), F[2].ravel(), R,
                                dims[mode]).reshape(dims[mode], R)
        assert rel_err(total.numpy(), full) <= 1e-12, mode
