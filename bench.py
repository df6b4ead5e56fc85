"""Benchmark: ms per CP-ALS iteration + sparse MTTKRP HBM GB/s, order-3 R=128.

One "step" = one full ALS iteration (3 x (Gram/Hadamard, MTTKRP, solve,
normalise), Gram fit) of BASELINE config 3 (12092 x 9184 x 28818, 76.9 M nnz,
Zipf(1.1), log-normal values, R = 128, dense threshold 0.03) with every input
resident in HBM.  Prints ONE JSON line on stdout; progress goes to stderr.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 3] [--R 128]
                  [--cpu-iters 4] [--no-cpu] [--fused]

The CPU baseline runs the CPU oracle's OpenMP ALS (the reference's semantics)
on the same row-sorted views, copied from the device, from the same initial
factors, for --cpu-iters iterations on the full tensor; the first iteration
is dropped and the median and mean of the rest are reported.

roofline (the FP64 sparse kernel, per launch): achieved = the algorithmic
bytes of the no-reuse gather model over the launch time measured here with
hipEvents; traffic = the bytes per launch between L2 and memory measured by
rocprofv3 --pmc (profiles/mttkrp_sparse3_<workload>_pmc.json, valid only while
the kernel's sources hash to the value recorded there); the compulsory bytes
and the element-gather floor (a probe kernel that runs the blocked kernel's
element-level row gathers alone, after the timed region) beside them.
--fused runs the merged single-grid MTTKRP (ALS_FUSED).

--config 4 / 5 run the generic N-order path on BASELINE configs 4 and 5
instead (secondary measurements; same JSON shape, the segment MTTKRP as the
roofline kernel and the dense-unit MFMA kernel beside it; the CPU baseline
is the oracle's N-order ALS).  --config 1 / 2 run the order-3 path on the
other two order-3 configs.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

BASELINE_METRIC = "ms per ALS iteration + sparse MTTKRP HBM GB/s (% of peak), order-3 R=128"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, vendor figure
FP32_MFMA_PEAK_TFLOPS = 157.3  # MI355X dense FP32 matrix, vendor figure
BF16_MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 matrix, vendor figure


def tile_roof(info, R, ntiles, launch_ms, where, segments=None):
    """MFMA roofline of the dense-tile kernel over its mean launch time: the
    split-bf16 kernel (three bf16 products per term, 32-rank blocks) against
    the bf16 matrix peak, the FP32 kernel against the FP32 matrix peak; the
    useful flops (8192 R per tile) and the tile image's bytes beside them
    (the compacted split images' 16-byte segments plus 64 header words and
    one offset per tile when `segments` lists them per launch, else the
    dense FP32 image)."""
    b3 = bool(info.tile_bf16x3)
    rq = (R + 31) // 32 * 32
    useful = 8192.0 * R * ntiles
    executed = 3 * 8192.0 * rq * ntiles if b3 else 8192.0 * ((R + 15) // 16 * 16) * ntiles
    peak = BF16_MFMA_PEAK_TFLOPS if b3 else FP32_MFMA_PEAK_TFLOPS
    mean_s = sum(launch_ms) / len(launch_ms) * 1e-3
    if segments and all(segments):
        img_bytes = [int(n) * 16 + ntiles * 260 for n in segments]
    else:
        img_bytes = [ntiles * 4096 * 4] * len(launch_ms)
    ach = executed / mean_s / 1e12
    return {
        "kernel": ("dense_tiles_b3_kernel (16^3 tiles, split-bf16 v_mfma_f32_32x32x16_bf16, "
                   "FP32 weights, FP64 output)" if b3 else
                   "dense_tiles_kernel (16^3 tiles, FP32 MFMA, FP64 output)") + ", " + where,
        "bound": "mfma", "achieved": round(ach, 2), "peak": peak, "unit": "TFLOP/s",
        "frac": round(ach / peak, 4),
        "flops_per_launch": executed, "useful_flops_per_launch": useful,
        "useful_TFLOPs": round(useful / mean_s / 1e12, 2),
        "tile_image_bytes_per_launch": img_bytes,
        "tile_image_GBs": round(sum(img_bytes) / len(img_bytes) / mean_s / 1e9, 1),
        "launch_ms": [round(x, 4) for x in launch_ms],
    }

CONFIG_SPEC = {
    1: dict(R=32, thr=0.03, name="cfg1: order-3 256^3 CP-rank-8 + noise, p=0.9 (~15.1M nnz)"),
    2: dict(R=32, thr=0.03, name="cfg2: order-3 512^3, 2000 16^3 blocks + 2e-4 background"),
    3: dict(R=128, thr=0.03,
            name="cfg3: order-3 12092x9184x28818, 76.9M nnz, Zipf(1.1), log-normal values"),
    4: dict(R=16, thr=0.03,
            name="cfg4: order-4 183x24x1140x1717, 3.3M nnz, HITS(T=3), dense units (0,1,2)"),
    5: dict(R=32, thr=0.03,
            name="cfg5: order-5 64x64x64x32x16, 20M nnz, 4000 dense units + background"),
}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def gather_bytes(nnz: int, dim_n: int, R: int, N: int = 3) -> float:
    """No-reuse gather model: COO stream + (N-1) factor rows per nnz + output rows."""
    return nnz * (4 * N + 8) + nnz * (N - 1) * R * 8 + dim_n * R * 8


SPARSE3_SOURCES = ("cptc_amd/csrc/kernels/mttkrp_sparse.hip", "cptc_amd/csrc/kernels/seg3_body.hpp")
BLK3_SOURCES = ("cptc_amd/csrc/kernels/mttkrp_blk.hip", "cptc_amd/csrc/host/blk3_params.hpp",
                "cptc_amd/csrc/kernels/layout.hip")


def sources_sha(paths) -> str:
    """sha256 (first 16 hex digits) of the kernel's source files, in order."""
    import hashlib

    h = hashlib.sha256()
    for p in paths:
        with open(os.path.join(ROOT, p), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def load_traffic(workload: str, sources=SPARSE3_SOURCES):
    """Measured HBM traffic of one sparse-kernel launch (rocprofv3 --pmc summary
    under profiles/), or None when there is none for this workload or the
    kernel's sources changed since it was measured."""
    path = os.path.join(ROOT, "profiles", f"mttkrp_sparse3_{workload}_pmc.json")
    if not os.path.exists(path):
        return None
    try:
        d = json.load(open(path))
    except (OSError, ValueError):
        return None
    if d.get("workload") != workload or d.get("kernel_src_sha") != sources_sha(sources):
        return None
    return d


SEG_ND_SOURCES = ("cptc_amd/csrc/kernels/seg_keys.hip",)
UNIT_SUMS_SOURCES = ("cptc_amd/csrc/kernels/unit_sums.hip",)
LDS_PEAK_TBS = 78.6   # 256 CUs x 128 B/clk x 2.4 GHz
L1_PEAK_TBS = 39.3    # vector L1 / texture path: 256 CUs x 64 B/clk x 2.4 GHz


def load_traffic_named(name: str, sources, workload: str):
    """A kernel's measured traffic summary profiles/<name>_pmc.json, or None
    when absent or measured on other kernel sources."""
    path = os.path.join(ROOT, "profiles", f"{name}_pmc.json")
    if not os.path.exists(path):
        return None
    try:
        d = json.load(open(path))
    except (OSError, ValueError):
        return None
    if d.get("workload") != workload or d.get("kernel_src_sha") != sources_sha(sources):
        return None
    return d


def load_traffic_seg(workload: str):
    """Measured HBM traffic of one generic segment-kernel launch, as load_traffic."""
    path = os.path.join(ROOT, "profiles", f"mttkrp_seg_nd_{workload}_pmc.json")
    if not os.path.exists(path):
        return None
    try:
        d = json.load(open(path))
    except (OSError, ValueError):
        return None
    if d.get("workload") != workload or d.get("kernel_src_sha") != sources_sha(SEG_ND_SOURCES):
        return None
    return d


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", type=int, default=3, choices=sorted(CONFIG_SPEC))
    ap.add_argument("--R", type=int, default=0)
    ap.add_argument("--cpu-iters", type=int, default=4)
    ap.add_argument("--fused", action="store_true",
                    help="merged single-grid MTTKRP (ALS_FUSED) on the order-3 path")
    ap.add_argument("--sgd", action="store_true",
                    help="CP-SGD (ALS_SGD) on the order-3 residual instead of ALS; default "
                         "R = 32 (the reference's SGD rank), batch 2^20, gamma 1e-9")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calib", action="store_true",
                    help="run only a streaming kernel of known size (PMC scaling)")
    ap.add_argument("--ingest", action="store_true",
                    help="time .tns load + device setup of the workload instead")
    args = ap.parse_args()
    if args.calib:
        return calib()
    if args.ingest:
        return ingest(args)

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (every GPU box here "
              "has one GPU); run with --gpus 1", file=sys.stderr)
        return 2

    import cptc_amd as ca

    if ca.device_count() < 1:
        print("bench.py: no HIP device visible", file=sys.stderr)
        return 1
    spec = CONFIG_SPEC[args.config]
    R = args.R or spec["R"]
    thr = spec["thr"]
    if args.config in (4, 5):
        return bench_generic(ca, args, spec, R)
    if args.sgd:
        return bench_sgd(ca, args, spec, args.R or 32)

    t0 = time.perf_counter()
    t = ca.synth_config(args.config, 42)
    log(f"generated config {args.config}: dims {t.dims} nnz {t.nnz} in "
        f"{time.perf_counter() - t0:.1f} s")

    t0 = time.perf_counter()
    h = ca.Als3(t, R=R, threshold=thr, fused=1 if args.fused else 0)
    info = h.info
    setup_s = time.perf_counter() - t0
    use_mfma = bool(info.use_mfma) and int(info.num_dense_tiles) > 0
    log(f"setup (upload, CADR, partition, views) {setup_s:.2f} s: tiles {info.num_dense_tiles} "
        f"dense_nnz {info.dense_nnz} sparse_nnz {info.sparse_nnz} avg_fill {info.avg_fill:.4f} "
        f"fill_min {info.fill_min:.4f} -> {'MFMA+FP64' if use_mfma else 'FP64'}; "
        f"segments {list(info.segments)} CUs {info.num_cus}")

    # the CPU baseline starts from the same initial factors (lambda = 1)
    F_init = [h.factor(m).ravel().copy() for m in range(3)] if not args.no_cpu else None
    if args.warmup:
        h.run(args.warmup)
        log(f"warmup {args.warmup} iterations done")
    h.kernel_times(reset=True)

    # timed region: exactly K ALS iterations between two device-wide
    # synchronisations (one GPU: no barrier across ranks is needed)
    ca.sync()
    t0 = time.perf_counter()
    fits, ms_iter, ms_mtt = h.run(args.steps)
    ca.sync()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / args.steps
    tile_ms_acc = h.tile_times()
    sp_ms, mt_ms, kit = h.kernel_times(reset=True)
    # a queued run records kernel events on every 8th iteration and its last
    assert kit == sum(1 for it in range(args.steps) if it % 8 == 0 or it == args.steps - 1)
    log(f"timed {args.steps} iterations: {ms_per_step:.3f} ms/iter (host wall), event median "
        f"{float(np.median(ms_iter)):.3f} ms, MTTKRP median {float(np.nanmedian(ms_mtt)) if np.isfinite(ms_mtt).any() else float('nan'):.3f} ms, "
        f"fit {fits[-1]:.6f}")

    dims = t.dims
    nnz = t.nnz
    # all MTTKRP launches of an iteration vs the gather model over all nnz
    b_iter = sum(gather_bytes(nnz, dims[m], R) for m in range(3))
    mtt_ms_iter = float(np.sum(mt_ms)) / kit
    mtt_gbs = b_iter / (mtt_ms_iter * 1e-3) / 1e9
    # dominant kernel: the FP64 residual-view sparse MTTKRP, per launch (one
    # mode); on the FP64-only path with a merged view it reads every nonzero
    merged_fp64 = bool(info.fp64_merged)
    snnz = int(info.nnz) if merged_fp64 else int(info.sparse_nnz)
    b_launch = [gather_bytes(snnz, dims[m], R) for m in range(3)]
    launch_ms = [float(sp_ms[m]) / kit for m in range(3)]
    mean_ms = sum(launch_ms) / 3
    gather_gbs = sum(b_launch) / (sum(launch_ms) * 1e-3) / 1e9 if snnz else 0.0
    blocked = bool(info.sparse_blocked) and not args.fused
    workload = f"cfg{args.config}-R{R}" + ("-fused" if args.fused else "-blocked" if blocked else
                                          "-merged" if merged_fp64 else "")
    # compulsory traffic per launch: the view stream + every factor row once + output rows
    compulsory = [snnz * 20 + sum(dims) * R * 8 + dims[m] * R * 8 for m in range(3)]
    comp_gbs = sum(compulsory) / (sum(launch_ms) * 1e-3) / 1e9 if snnz else 0.0
    prof = load_traffic(workload, BLK3_SOURCES if blocked else SPARSE3_SOURCES)
    # tiles: 8192 R flops per tile per mode (16^3 x R multiply-adds)
    ntiles = int(info.num_dense_tiles)
    tile_ms = [float(x) / kit for x in tile_ms_acc]
    tiles_timed = use_mfma and ntiles and all(x > 0 for x in tile_ms)

    probe_ms = h.gather_probe(3) if blocked else None

    cpu = None
    if not args.no_cpu and args.cpu_iters > 0:
        cpu = cpu_baseline(ca, h, t, R, args.cpu_iters, use_mfma, F_init)

    if snnz:
        traffic = dram = None
        if prof:
            traffic = prof["hbm_bytes_per_launch"]
            dram = traffic / (mean_ms * 1e-3) / 1e9
        roofline = {
            "kernel": ("mttkrp3_merged_kernel (MFMA tiles + FP64 residual in one grid)"
                       if args.fused else
                       "mttkrp3_blk_kernel (FP64 residual, blocked layout, R in (64,128])"
                       if blocked else
                       "mttkrp3_seg_wave_kernel (FP64 residual view, R in (64,128])"
                       if 64 < R <= 128 else
                       ("mttkrp3_seg_lanes_kernel" if R % 2 == 0 and R <= 64
                        else "mttkrp3_seg_kernel") +
                       (" (FP64 view of every nonzero: residual + dense pool)" if merged_fp64
                        else " (FP64 residual view)")) + ", per launch = one mode",
            "bound": "hbm",
            "achieved": round(gather_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gather_gbs / HBM_PEAK_GBS, 4),
            "traffic": int(traffic) if traffic else None,
            "launch_ms": [round(x, 4) for x in launch_ms],
            "algorithmic_bytes_per_launch": [int(b) for b in b_launch],
            "traffic_GBs": round(dram, 1) if dram else None,
            "traffic_frac": round(dram / HBM_PEAK_GBS, 4) if dram else None,
            "compulsory_GBs": round(comp_gbs, 1),
            "compulsory_frac": round(comp_gbs / HBM_PEAK_GBS, 4),
            "compulsory_bytes_per_launch": [int(b) for b in compulsory],
            # the element-level row gathers alone, measured: the probe kernel
            # runs them in the blocked kernel's order and occupancy (None
            # when the layout is not blocked)
            "element_gather_floor_ms": ([round(float(x), 4) for x in probe_ms]
                                        if probe_ms is not None else None),
            "element_gather_floor_basis": "cptc_gather_probe3_blk on the same blocked view and "
                                          "factors: each residual nonzero's R-wide FP64 row of "
                                          "its element-level factor, same chunks, waves and rows "
                                          "in flight, nothing else (mean of 3 launches per mode, "
                                          "after the timed region)",
            # the same rows if every one were an L1 hit: R x 8 B per residual
            # nonzero through the vector L1 at its 64 B per clock per CU
            "l1_floor_model_ms": round(snnz * R * 8 / (L1_PEAK_TBS * 1e12) * 1e3, 4),
            "traffic_source": (f"profiles/mttkrp_sparse3_{workload}_pmc.json "
                               f"(kernel sources sha {prof['kernel_src_sha']})") if prof else
                              "none for these kernel sources: traffic null",
            "note": "achieved = algorithmic bytes per launch (no-reuse gather model: per residual "
                    "nonzero its 20-byte COO entry and one R-wide FP64 row of each of the two "
                    "other factors, plus the output rows) over the launch time measured here "
                    "with hipEvents; L1, L2 and the 256 MB MALL serve most of those row "
                    "gathers, so frac exceeds 1. traffic = bytes per launch between L2 and "
                    "memory measured by rocprofv3 --pmc (read + write, calibrated on a copy "
                    "kernel; MALL hits count, so it bounds the DRAM bytes from above); "
                    "traffic_GBs = traffic over the same launch time. compulsory = view "
                    "stream + every factor row once + output rows.",
        }
    else:
        # no sparse residual (every nonzero in a dense tile): the MFMA tile
        # kernel is the whole MTTKRP
        mt_launch = [float(mt_ms[m]) / kit for m in range(3)]
        if use_mfma and ntiles:
            roofline = tile_roof(info, R, ntiles, mt_launch, "the whole MTTKRP (no residual)",
                                 list(info.tile_segments) if info.tile_compact else None)
        else:
            roofline = {"kernel": "FP64 dense-view MTTKRP", "bound": "hbm", "achieved": None,
                        "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": None,
                        "launch_ms": [round(x, 4) for x in mt_launch]}
        roofline["traffic"] = None
    roofline_tiles = None
    if tiles_timed and snnz:
        where = ("beside the FP64 kernel on a second stream" if info.tiles_beside else
                 "on the main stream before the FP64 kernel")
        roofline_tiles = tile_roof(info, R, ntiles, tile_ms, where,
                                   list(info.tile_segments) if info.tile_compact else None)

    line = {
        "metric": BASELINE_METRIC,
        "value": round(ms_per_step, 4),
        "unit": "ms/iteration",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f64" if not use_mfma else (
            "f64 (dense tiles: split-bf16 MFMA, fp32 weights, f64 output)" if info.tile_bf16x3
            else "f64 (dense tiles: fp32 MFMA, f64 output)"),
        "data": "synthetic (deterministic generator, seed 42)",
        "config": {
            "workload": spec["name"] if R == spec["R"] else f"{spec['name']} (R={R})",
            "R": R, "nnz": nnz, "dims": list(dims), "dense_threshold": thr,
            "dense_tiles": int(info.num_dense_tiles), "dense_nnz": int(info.dense_nnz),
            "sparse_nnz": int(info.sparse_nnz), "fp64_kernel_nnz": snnz,
            "fp64_merged_view": merged_fp64, "path": "mfma+fp64" if use_mfma else "fp64",
            "fused": bool(info.fused), "sparse_blocked": bool(info.sparse_blocked),
            "tile_kernel": "bf16x3" if info.tile_bf16x3 else "fp32",
            "tiles_beside": bool(info.tiles_beside),
            "parallelism": "single GPU",
        },
        "ms_per_iter_event_median": round(float(np.median(ms_iter)), 4),
        "mttkrp_ms_per_iter": round(mtt_ms_iter, 4),
        "mttkrp_gather_model_GBs": round(mtt_gbs, 1),
        "mttkrp_gather_model_frac": round(mtt_gbs / HBM_PEAK_GBS, 4),
        "fit_last": float(fits[-1]),
        "roofline": roofline,
        "roofline_tiles": roofline_tiles,
        "cpu_baseline": cpu,
    }
    h.close()
    print(json.dumps(line), flush=True)
    return 0


def bench_sgd(ca, args, spec, R) -> int:
    """CP-SGD (sgd.cu:302-467): one step = one SGD iteration (sample 2^20
    residual elements, one asynchronous gradient step each; every fifth
    iteration the column normalisation, every tenth the batch loss)."""
    batch, gamma = 1 << 20, 1e-9
    t = ca.synth_config(args.config, 42)
    h = ca.Als3(t, R=R, threshold=spec["thr"])
    snnz = int(h.info.sparse_nnz)
    if args.warmup:
        h.sgd(args.warmup, gamma, batch, 7)
    ca.sync()
    t0 = time.perf_counter()
    rm = h.sgd(args.steps, gamma, batch, 42)
    ca.sync()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    h.close()
    # per element: index + packed coordinate + value, three factor rows read
    # and three rows of atomic steps (read-modify-write counted once each)
    b_elem = 4 + 16 + 6 * R * 8
    log(f"CP-SGD {args.steps} iterations: {ms:.3f} ms/iter, batch rmse {rm[rm > 0].tolist()}")
    print(json.dumps({
        "metric": "ms per CP-SGD iteration (order-3 residual, batch 2^20)",
        "value": round(ms, 4), "unit": "ms/iteration", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "f64",
        "data": "synthetic (deterministic generator, seed 42)",
        "config": {"workload": spec["name"], "R": R, "batch": batch, "gamma": gamma,
                   "sparse_nnz": snnz, "parallelism": "single GPU"},
        "element_steps_per_s": round(batch / (ms * 1e-3), 1),
        "gather_model_GBs": round(batch * b_elem / (ms * 1e-3) / 1e9, 1),
        "batch_rmse": [float(x) for x in rm if x > 0],
    }), flush=True)
    return 0


def bench_generic(ca, args, spec, R) -> int:
    """Configs 4 and 5 through the generic N-order driver (cptc_gen_*)."""
    t0 = time.perf_counter()
    t = ca.synth_config(args.config, 42)
    log(f"generated config {args.config}: dims {t.dims} nnz {t.nnz} in "
        f"{time.perf_counter() - t0:.1f} s")
    t0 = time.perf_counter()
    g = ca.Gen(t, R=R, reorder="hits", rounds=3, threshold=spec["thr"])
    info = g.info
    N = g.N
    knnz = [int(info.kernel_nnz[m]) for m in range(N)]
    log(f"setup {time.perf_counter() - t0:.2f} s: reorder {info.reorder.decode()} units "
        f"{info.n_units} dense_nnz {info.dense_nnz} kernel-view nnz {knnz}")
    if args.warmup:
        g.run(args.warmup)
    g.kernel_times(reset=True)
    ca.sync()
    t0 = time.perf_counter()
    fits, _, _, ms_iter = g.run(args.steps)
    ca.sync()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / args.steps
    # kernel events on every 8th iteration and the last (the driver's sampling)
    seg_ms, unit_ms, kit = g.kernel_times(reset=True)
    assert 1 <= kit <= args.steps
    dims = t.dims
    b_seg = [gather_bytes(knnz[m], dims[m], R, N) for m in range(N)]
    seg_launch = [float(seg_ms[m]) / kit for m in range(N)]
    achieved = sum(b_seg) / (sum(seg_launch) * 1e-3) / 1e9
    workload = f"cfg{args.config}-R{R}"
    usums = bool(info.unit_sums)
    # the inner modes in slot order (the order of unit_segments)
    inner = list(tuple(info.inner)) if info.dense_enabled else []
    outer = [m for m in range(N) if m not in inner]
    unit_launch = [float(unit_ms[m]) / kit for m in inner]
    if usums:
        # outer modes from per-unit sums: one unit_sums_kernel launch per
        # iteration (its time is reported under the first outer mode's unit
        # kernel), then one scatter per outer mode
        us_ms = sum(float(unit_ms[m]) for m in outer) / kit
        n_el = int(info.dense_nnz)
        # algorithmic bytes: every element's 12-byte (lid, value) record and
        # its three R-wide FP64 inner factor rows, plus the unit sums written
        b_us = n_el * 12 + n_el * 3 * R * 8 + int(info.n_units) * R * 8
        ach_us = b_us / (us_ms * 1e-3) / 1e9
        prof = load_traffic_named(f"unit_sums_{workload}", UNIT_SUMS_SOURCES, workload)
        traffic = prof["hbm_bytes_per_launch"] if prof else None
        # the kernel reads RT >= R ranks per row (RT = 8, 16 or 32)
        rt = 8 if R <= 8 else 16 if R <= 16 else 32
        lds_b = n_el * 3 * rt * 8
        roofline = {
            "kernel": "unit_sums_kernel (per-unit FP64 inner sums for the outer modes: every "
                      "element lies in a dense unit), one launch per iteration",
            "bound": "hbm", "achieved": round(ach_us, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(ach_us / HBM_PEAK_GBS, 4),
            "traffic": int(traffic) if traffic else None,
            "launch_ms": [round(us_ms, 4)],
            "algorithmic_bytes_per_launch": [int(b_us)],
            "traffic_GBs": round(traffic / (us_ms * 1e-3) / 1e9, 1) if traffic else None,
            "traffic_frac": round(traffic / (us_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
            if traffic else None,
            "lds_bytes_per_launch": int(lds_b),
            "lds_TBs": round(lds_b / (us_ms * 1e-3) / 1e12, 2),
            "lds_peak_TBs": LDS_PEAK_TBS,
            "lds_frac": round(lds_b / (us_ms * 1e-3) / 1e12 / LDS_PEAK_TBS, 4),
            "scatter_launch_ms": [round(float(seg_ms[m]) / kit, 4) for m in outer],
            "traffic_source": (f"profiles/unit_sums_{workload}_pmc.json (kernel sources sha "
                               f"{prof['kernel_src_sha']})") if prof else
                              "none for these kernel sources: traffic null",
            "note": "achieved = algorithmic bytes per launch (per element its (lid, value) "
                    "record and three R-wide FP64 inner factor rows, plus the unit sums) over "
                    "the launch time measured with hipEvents; the rows come from LDS (each "
                    "workgroup stages its units' three 16-row factor blocks once), so frac "
                    "exceeds 1 and the kernel is bound by the LDS reads: lds_bytes = 3 "
                    "FP64 row values per element and rank, against 256 CUs x 128 B/clk x 2.4 "
                    "GHz.",
        }
    else:
        prof = load_traffic_seg(workload)
        traffic = prof["hbm_bytes_per_launch"] if prof else None
        mean_s = sum(seg_launch) / N * 1e-3
        roofline = {
            "kernel": "seg_keys_kernel / seg_keys_leaf_lds_kernel (FP64 segment MTTKRP over "
                      "packed level keys), per launch = one mode",
            "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": int(traffic) if traffic else None,
            "launch_ms": [round(x, 4) for x in seg_launch],
            "algorithmic_bytes_per_launch": [int(b) for b in b_seg],
            "traffic_GBs": round(traffic / mean_s / 1e9, 1) if traffic else None,
            "traffic_frac": round(traffic / mean_s / 1e9 / HBM_PEAK_GBS, 4) if traffic else None,
            "traffic_source": (f"profiles/mttkrp_seg_nd_{workload}_pmc.json (kernel sources "
                               f"sha {prof['kernel_src_sha']})") if prof else
                              "none for these kernel sources: traffic null",
            "note": "achieved = algorithmic bytes per launch (no-reuse gather model over the "
                    "kernel view's elements) over the launch time measured with hipEvents; "
                    "L1/L2 serve the gathers, so frac exceeds 1; traffic = L2-to-memory bytes "
                    "per launch (rocprofv3 --pmc).",
        }

    log(f"timed {args.steps} iterations: {ms_per_step:.3f} ms/iter; seg launch ms "
        f"{[round(x, 4) for x in seg_launch]}; unit launch ms {[round(x, 4) for x in unit_launch]}")
    cpu = None
    if not args.no_cpu and args.cpu_iters > 0:
        cpu = cpu_baseline_generic(g, t, R, spec["thr"], args.cpu_iters)
    line = {
        "metric": BASELINE_METRIC,
        "value": round(ms_per_step, 4),
        "unit": "ms/iteration",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": ("f64 (dense units: split-bf16 MFMA, fp32 weights, f64 output)"
                  if info.tile_bf16x3 else "f64 (dense units: fp32 MFMA, f64 output)"),
        "data": "synthetic (deterministic generator, seed 42)",
        "config": {"workload": spec["name"] if R == spec["R"] else f"{spec['name']} (R={R})",
                   "R": R, "nnz": t.nnz, "dims": list(dims), "dense_units": int(info.n_units),
                   "dense_nnz": int(info.dense_nnz), "kernel_view_nnz": knnz,
                   "path": "generic N-order", "parallelism": "single GPU",
                   "tile_kernel": "bf16x3" if info.tile_bf16x3 else "fp32"},
        "fit_last": float(fits[-1]),
        "mttkrp_launch_ms": [round(x, 4) for x in seg_launch],
        "roofline": roofline,
        "roofline_units": (tile_roof(info, R, int(info.n_units), unit_launch,
                                     "dense units with FP64 outer weights, per inner mode",
                                     list(info.unit_segments))
                           if unit_launch else None),
        "cpu_baseline": cpu,
    }
    g.close()
    print(json.dumps(line), flush=True)
    return 0


def ingest(args) -> int:
    """The ingest path (.tns text -> device layout): the workload is written
    as a .tns file under $TMPDIR, then timed: the parallel loader
    (load_tns_file / load_tns_generic) and the driver's setup (upload, CADR or
    HITS reorder, partition or dense units, row-sorted views).  The
    reference's published figure for this path: load + init 5.46 s of a
    7.92 s run on NELL-2 (docs/rtx4090_comparison.md:17)."""
    import shutil
    import tempfile

    import cptc_amd as ca

    spec = CONFIG_SPEC[args.config]
    R = args.R or spec["R"]
    t = ca.synth_config(args.config, 42)
    nnz = t.nnz
    tmp = tempfile.mkdtemp(dir=os.environ.get("TMPDIR", "/tmp"))
    try:
        path = os.path.join(tmp, f"cfg{args.config}.tns")
        t0 = time.perf_counter()
        ca.write_tns(path, t)
        write_s = time.perf_counter() - t0
        del t
        size = os.path.getsize(path)
        log(f"wrote {path}: {size / 1e9:.2f} GB in {write_s:.2f} s")
        loads = []
        for _ in range(2):
            t0 = time.perf_counter()
            t2 = ca.load_tns3(path) if args.config <= 3 else ca.load_tns_generic(path)
            loads.append(time.perf_counter() - t0)
            if len(loads) < 2:
                del t2
        log(f"load {[round(x, 3) for x in loads]} s")
        t0 = time.perf_counter()
        if args.config <= 3:
            h = ca.Als3(t2, R=R, threshold=spec["thr"])
        else:
            h = ca.Gen(t2, R=R, reorder="hits", rounds=3, threshold=spec["thr"])
        ca.sync()
        setup_s = time.perf_counter() - t0
        h.close()
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    load_s = min(loads)
    log(f"setup {setup_s:.3f} s")
    print(json.dumps({
        "metric": "ingest: .tns load + device setup (s)",
        "value": round(load_s + setup_s, 3), "unit": "s", "higher_is_better": False,
        "load_s": round(load_s, 3), "load_first_s": round(loads[0], 3),
        "load_GBs": round(size / load_s / 1e9, 2), "file_bytes": size, "nnz": nnz,
        "setup_s": round(setup_s, 3), "host_threads": os.cpu_count(),
        "config": {"workload": spec["name"], "R": R},
        "reference": "load + init 5.46 s, NELL-2 (76.9 M nnz), RTX 4090 host",
    }), flush=True)
    return 0


def calib() -> int:
    """A streaming kernel of known size for scaling rocprofv3 FETCH_SIZE /
    WRITE_SIZE: cptc_hadamard over n doubles reads 16 n and writes 8 n bytes."""
    import cptc_amd as ca

    n = 1 << 25
    a, b, c = (ca.DevBuf.zeros((n,)) for _ in range(3))
    for _ in range(5):
        ca.check(ca.lib.cptc_hadamard(a.data_ptr(), b.data_ptr(), c.data_ptr(), n, None),
                 "cptc_hadamard")
    ca.sync()
    print(json.dumps({"calib": "hadamard_kernel", "n": n, "read_bytes": 16 * n,
                      "write_bytes": 8 * n, "launches": 5}), flush=True)
    return 0


def host_info() -> dict:
    """nproc, the OpenMP thread count and the CPU model of this host."""
    fields = {}
    sockets = set()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                key, _, val = line.partition(":")
                key, val = key.strip(), val.strip()
                if key == "physical id":
                    sockets.add(val)
                if key in ("model name", "cpu family", "model", "stepping", "cpu MHz",
                           "cache size", "cpu cores", "siblings") and key not in fields:
                    fields[key] = val
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "omp_num_threads_env": os.environ.get("OMP_NUM_THREADS"),
            "cpu_model": fields.get("model name"),
            "cpuinfo": dict(fields, sockets=len(sockets) or None)}


def summarize_cpu(ms, extra: dict) -> dict:
    """The CPU timing rule: drop iteration 1 (first-touch and warm-up), report the
    median and mean of the rest."""
    kept = ms[1:] if len(ms) > 1 else ms
    out = {
        "value": round(float(np.median(kept)), 1),
        "unit": "ms/iteration",
        "median_ms": round(float(np.median(kept)), 1),
        "mean_ms": round(float(np.mean(kept)), 1),
        "iterations_ms": [round(float(x), 1) for x in ms],
        "dropped_first": len(ms) > 1,
    }
    out.update(extra)
    return out


def cpu_baseline_generic(g, t, R, thr, iters):
    """The oracle's N-order ALS (C++ with OpenMP MTTKRPs, the reference's
    semantics) on the device-reordered tensor, timed per iteration on this
    host (test infrastructure used as the CPU baseline only)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle", "_build"))
    import cptc_oracle as orc

    coords = g.coords()
    ranks = [g.rank(m) for m in range(g.N)]
    threads = orc.max_threads()
    log(f"CPU baseline: N-order ALS, {iters} iteration(s) with {threads} OpenMP threads "
        f"(setup not timed)")
    _, ms = orc.als_nd_timed(coords, t.val, t.dims, ranks, R, 42, thr, iters)
    ms = [float(x) for x in ms]
    log(f"CPU baseline: {[round(x, 3) for x in ms]} ms/iter")
    return summarize_cpu(ms, {
        "cores": int(threads),
        "kind": "port",
        "sample": f"{iters} full ALS iterations of the same workload (all {t.nnz} nnz, R={R}, "
                  f"HITS-reordered on the GPU, dense units and views built by the oracle), from "
                  f"the reference's initial factors; first iteration dropped",
        "host": host_info(),
    })


def cpu_baseline(ca, h, t, R, iters, use_mfma, F_init):
    """The oracle's OpenMP ALS over the device-built views (test infrastructure
    used as the CPU baseline only), timed on this host from the same initial
    factors as the GPU run (lambda = 1)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle", "_build"))
    import cptc_oracle as orc

    t0 = time.perf_counter()
    views = [h.view(0, m) for m in range(3)]
    dv = None
    tiles = None
    if int(h.info.num_dense_tiles) > 0:
        if use_mfma:
            tl = h.tiles()
            tl["cutoff"] = int(h.info.dense_cutoff)
            tiles = tl
        else:
            dv = [h.view(1, m) for m in range(3)]
    x_sq = float(np.sum(t.val * t.val))
    o = orc.Als3(views, dv, tiles, x_sq, t.dims, R, F_init[0], F_init[1], F_init[2], None)
    del views, dv, tiles
    threads = orc.max_threads()
    log(f"CPU baseline: data staged in {time.perf_counter() - t0:.1f} s; running {iters} "
        f"ALS iteration(s) with {threads} OpenMP threads")
    _, ms, mm = o.iterate(iters)
    ms = [float(x) for x in ms]
    mm = [float(x) for x in mm]
    log(f"CPU baseline: {[round(x, 1) for x in ms]} ms/iter (MTTKRP {[round(x, 1) for x in mm]} ms)")
    kept = mm[1:] if len(mm) > 1 else mm
    return summarize_cpu(ms, {
        "cores": int(threads),
        "kind": "port",
        "sample": f"{iters} full ALS iterations of the same workload (all {t.nnz} nnz, R={R}) "
                  f"from the GPU run's initial factors, views built on the GPU and copied to "
                  f"host; first iteration dropped",
        "mttkrp_ms_median": round(float(np.median(kept)), 1),
        "host": host_info(),
    })


if __name__ == "__main__":
    sys.exit(main())
