"""Writes the layout fixtures in this folder (run from the repository root:
`python tests/golden/make_golden.py`).

The reference ships no data fixtures and no golden vectors for this path, so
these fixtures are regression pins: small, self-contained inputs (COO index
arrays and values, stored in the fixture) and the layouts the CPU oracle
(oracle/, itself pinned by the independent numpy restatements in
tests/test_oracle_layout.py and tests/test_oracle_nd.py) derives from them
with the reference's rules:

  layout3.npz  order 3 (tensor.cu, cadr.cu, partition.cu): CADR permutations,
               hybrid 16^3 partition (tiles, pools, cutoff) at threshold 0.03,
               the residual's row-sorted views of every mode;
  layoutN.npz  order 4 (generic.cu): HITS (3 rounds) ranks and relabelled
               coordinates, dense units at threshold 0.03 over inner modes
               (0, 1, 2), the per-mode views.

tests/test_golden.py checks that the oracle still produces these bytes;
tests/test_gpu_golden.py checks that the HIP path does.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle", "_build"))


def input3():
    """Zipf-skewed coordinates (dense heads become tiles) plus one planted
    dense block, duplicates removed, element order shuffled."""
    rng = np.random.default_rng(20261202)
    dims = (300, 200, 500)
    n = 12000
    idx = np.stack([np.minimum(rng.zipf(1.6, n) - 1, d - 1) for d in dims])
    blk = np.array(np.meshgrid(np.arange(32, 48), np.arange(16, 32), np.arange(64, 80),
                               indexing="ij")).reshape(3, -1)
    blk = blk[:, rng.random(blk.shape[1]) < 0.3]
    idx = np.unique(np.concatenate([idx, blk], axis=1), axis=1)
    idx = idx[:, rng.permutation(idx.shape[1])].astype(np.uint32)
    val = rng.lognormal(0.0, 1.0, idx.shape[1])
    return dims, idx, val


def inputN():
    rng = np.random.default_rng(4)
    dims = (40, 35, 48, 20)
    cells = np.array(np.meshgrid(np.arange(16), np.arange(16), np.arange(16, 32),
                                 indexing="ij")).reshape(3, -1)
    parts = []
    for o in range(2):
        c = cells[:, rng.random(cells.shape[1]) < 0.25]
        parts.append(np.vstack([c, np.full((1, c.shape[1]), 2 * o + 1)]))
    bg = np.stack([rng.integers(0, d, 1000) for d in dims])
    idx = np.unique(np.concatenate(parts + [bg], axis=1), axis=1)
    idx = idx[:, rng.permutation(idx.shape[1])].astype(np.uint32)
    val = rng.random(idx.shape[1]) + 0.25
    return dims, idx, val


def layout3(orc, dims, idx, val):
    i32 = idx.astype(np.int32)
    perms = orc.cadr3(i32[0], i32[1], i32[2], list(dims))
    r = np.stack([perms[m][i32[m]] for m in range(3)]).astype(np.int32)
    p = orc.partition3(r[0], r[1], r[2], val, list(dims), 0.03)
    v = orc.views3(p["sp_i"], p["sp_j"], p["sp_k"], p["sp_val"], list(dims))
    out = {"perm%d" % m: np.asarray(perms[m]) for m in range(3)}
    for k in ("tiles", "pool_off", "pool_lid", "pool_val"):
        out[k] = np.asarray(p[k])
    out["cutoff"] = np.array(p["cutoff"])
    for m in range(3):
        for k in ("coords", "vals", "blk_row", "blk_start", "blk_cnt"):
            out["view%d_%s" % (m, k)] = np.asarray(v[m][k])
    return out


def layoutN(orc, dims, idx, val):
    ridx, rank = orc.reorder_nd(idx, val, list(dims), "hits", 3, 8000000)
    u = orc.dense_nd(ridx, val, list(dims), 0.03, (0, 1, 2))
    views = orc.views_nd(ridx, val, list(dims), u["is_dense"], True, (0, 1, 2))
    out = {"ridx": np.asarray(ridx)}
    for m in range(len(dims)):
        out["rank%d" % m] = np.asarray(rank[m])
    for k in ("unit6", "outer_coords", "lid", "val", "is_dense"):
        out["unit_" + k] = np.asarray(u[k])
    out["unit_cutoff"] = np.array(u["cutoff"])
    for n in range(len(dims)):
        for k in ("scoords", "vals", "skip", "row", "start", "cnt", "single"):
            out["view%d_%s" % (n, k)] = np.asarray(views[n][k])
    return out


def main():
    import cptc_oracle as orc
    dims, idx, val = input3()
    np.savez_compressed(os.path.join(HERE, "layout3.npz"), dims=np.array(dims), idx=idx,
                        val=val, **layout3(orc, dims, idx, val))
    dims, idx, val = inputN()
    np.savez_compressed(os.path.join(HERE, "layoutN.npz"), dims=np.array(dims), idx=idx,
                        val=val, **layoutN(orc, dims, idx, val))


if __name__ == "__main__":
    main()
