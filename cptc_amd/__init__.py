"""MI355X-native CP-ALS engine with cpTC's surface (host-side Python mirror).

The compute path is libcptc.so (hand-written HIP kernels for gfx950 behind a
C ABI); this package only marshals arrays and handles.  ``Als3`` mirrors the
reference's order-3 flow (main.cu:136-672 + execute_als_decomposition,
als.cu:362-821); the module functions mirror the loader, CADR and generators.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from ._lib import (CLI_PATH, LIB_PATH, SIGNATURES, Als3Info, Als3Opts, Coo, CptcError, GenInfo,
                   GenOpts, check, lib)  # noqa: F401  (check is part of the public surface)

__all__ = [
    "lib", "LIB_PATH", "CLI_PATH", "SIGNATURES", "CptcError", "Tensor", "synth_config",
    "synth_zipf", "synth_lowrank3", "synth_blocks3", "synth_units5", "load_tns3",
    "load_tns_generic", "probe_nmodes", "write_tns", "cadr3", "Als3", "device_count", "ptr",
    "DevBuf", "sync", "check", "gen_reorder", "gen_hash", "gen_selftest", "Gen",
]


def device_count() -> int:
    return int(lib.cptc_device_count())


def ptr(x) -> int:
    """Raw address of a DevBuf, numpy array or object with data_ptr() (None -> 0)."""
    if x is None:
        return 0
    if isinstance(x, np.ndarray):
        return x.ctypes.data
    return int(x.data_ptr())


def sync() -> None:
    check(lib.cptc_dev_sync(), "cptc_dev_sync")


class DevBuf:
    """A device allocation made by libcptc's own HIP runtime."""

    def __init__(self, nbytes: int, dtype=np.uint8, shape=None):
        self.dtype = np.dtype(dtype)
        if shape is None:
            shape = (nbytes // self.dtype.itemsize,)
        self.shape = (int(shape),) if np.isscalar(shape) else tuple(shape)
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        check(lib.cptc_dev_malloc(self.nbytes, C.byref(p)), "cptc_dev_malloc")
        self._p = p

    @classmethod
    def from_numpy(cls, a) -> "DevBuf":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes, a.dtype, a.shape)
        check(lib.cptc_dev_upload(b._p, a.ctypes.data, a.nbytes), "cptc_dev_upload")
        return b

    @classmethod
    def zeros(cls, shape, dtype=np.float64) -> "DevBuf":
        dt = np.dtype(dtype)
        n = int(np.prod(shape)) * dt.itemsize
        b = cls(n, dt, shape)
        check(lib.cptc_dev_memset(b._p, 0, n), "cptc_dev_memset")
        return b

    def data_ptr(self) -> int:
        return int(self._p.value or 0)

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        check(lib.cptc_dev_download(out.ctypes.data, self._p, self.nbytes), "cptc_dev_download")
        return out

    def free(self) -> None:
        if getattr(self, "_p", None) is not None and self._p.value:
            lib.cptc_dev_free(self._p)
            self._p = C.c_void_p()

    def __del__(self):
        self.free()


@dataclass
class Tensor:
    """Host COO tensor: idx (nmodes x nnz uint32, 0-based), val (nnz float64)."""

    dims: tuple
    idx: np.ndarray
    val: np.ndarray

    @property
    def nmodes(self) -> int:
        return len(self.dims)

    @property
    def nnz(self) -> int:
        return int(self.val.shape[0])

    def as_coo(self) -> tuple[Coo, tuple]:
        """A cptc_coo view of this tensor (keep the returned arrays alive)."""
        idx = np.ascontiguousarray(self.idx, dtype=np.uint32)
        val = np.ascontiguousarray(self.val, dtype=np.float64)
        c = Coo()
        c.nmodes = self.nmodes
        for m, d in enumerate(self.dims):
            c.dims[m] = int(d)
        c.nnz = self.nnz
        c.idx = idx.ctypes.data_as(C.POINTER(C.c_uint32))
        c.val = val.ctypes.data_as(C.POINTER(C.c_double))
        return c, (idx, val)


class _CooOwner:
    """Owns a library-allocated COO; frees it (cptc_coo_free) when the last
    numpy view of its arrays is gone."""

    def __init__(self, c: Coo):
        self.c = c

    def __del__(self):
        lib.cptc_coo_free(C.byref(self.c))


def _take(c: Coo) -> Tensor:
    """Tensor over the library's arrays without copying them (a 76.9 M-nonzero
    tensor is 1.5 GB)."""
    n, nm = int(c.nnz), int(c.nmodes)
    dims = tuple(int(c.dims[m]) for m in range(nm))
    if not n:
        lib.cptc_coo_free(C.byref(c))
        return Tensor(dims, np.zeros((nm, 0), np.uint32), np.zeros(0, np.float64))
    owner = _CooOwner(c)
    bidx = (C.c_uint32 * (nm * n)).from_address(C.addressof(c.idx.contents))
    bval = (C.c_double * n).from_address(C.addressof(c.val.contents))
    bidx._owner = owner
    bval._owner = owner
    idx = np.frombuffer(bidx, dtype=np.uint32).reshape(nm, n)
    val = np.frombuffer(bval, dtype=np.float64)
    return Tensor(dims, idx, val)


def synth_config(config: int, seed: int = 42) -> Tensor:
    c = Coo()
    check(lib.cptc_synth_config(config, seed, C.byref(c)), f"cptc_synth_config({config})")
    return _take(c)


def synth_zipf(dims, exponents, nnz: int, value_kind: int = 0, seed: int = 42) -> Tensor:
    d = np.asarray(dims, np.uint64)
    e = np.asarray(exponents, np.float64)
    c = Coo()
    check(lib.cptc_synth_zipf(len(d), d.ctypes.data, e.ctypes.data, nnz, value_kind, seed,
                              C.byref(c)), "cptc_synth_zipf")
    return _take(c)


def synth_lowrank3(n: int, rank: int, keep_p: float, noise_sigma: float, seed: int = 42) -> Tensor:
    c = Coo()
    check(lib.cptc_synth_lowrank3(n, rank, keep_p, noise_sigma, seed, C.byref(c)),
          "cptc_synth_lowrank3")
    return _take(c)


def synth_blocks3(n: int, nblocks: int, fill_lo: float, fill_hi: float, bg: float,
                  seed: int = 42) -> Tensor:
    c = Coo()
    check(lib.cptc_synth_blocks3(n, nblocks, fill_lo, fill_hi, bg, seed, C.byref(c)),
          "cptc_synth_blocks3")
    return _take(c)


def synth_units5(dims, nunits: int, fill_lo: float, fill_hi: float, total_nnz: int,
                 signal_rank: int = 4, seed: int = 42) -> Tensor:
    d = np.asarray(dims, np.uint64)
    c = Coo()
    check(lib.cptc_synth_units5(d.ctypes.data, nunits, fill_lo, fill_hi, total_nnz, signal_rank,
                                seed, C.byref(c)), "cptc_synth_units5")
    return _take(c)


def load_tns3(path: str) -> Tensor:
    c = Coo()
    check(lib.cptc_tns_load3(path.encode(), C.byref(c)), "cptc_tns_load3")
    return _take(c)


def load_tns_generic(path: str) -> Tensor:
    c = Coo()
    check(lib.cptc_tns_load_generic(path.encode(), C.byref(c)), "cptc_tns_load_generic")
    return _take(c)


def probe_nmodes(path: str) -> int:
    return int(lib.cptc_tns_probe_nmodes(path.encode()))


def write_tns(path: str, t: Tensor) -> None:
    c, keep = t.as_coo()
    check(lib.cptc_tns_write(path.encode(), C.byref(c)), "cptc_tns_write")
    del keep


def cadr3(t: Tensor, relabel: bool = True):
    """CADR on the device (cadr.cu:23-81): returns (perms, relabelled idx)."""
    idx = np.ascontiguousarray(t.idx, dtype=np.int32).copy()
    dims = np.asarray(t.dims, np.uint64)
    perms = [np.zeros(int(d), np.int32) for d in t.dims]
    check(lib.cptc_cadr3(idx[0].ctypes.data, idx[1].ctypes.data, idx[2].ctypes.data, t.nnz,
                         dims.ctypes.data, perms[0].ctypes.data, perms[1].ctypes.data,
                         perms[2].ctypes.data, int(relabel)), "cptc_cadr3")
    return perms, idx


class Als3:
    """Order-3 CP-ALS on the device (one handle = CADR, partition, views, factors)."""

    def __init__(self, t: Tensor, R: int = 32, threshold: float = 0.03, path: int = -1,
                 fill_min: float = -1.0, cadr: bool = True, seed: int = 42, verbose: bool = False,
                 skip_dense: int = -1, skip_sparse: int = -1, fused: int = -1):
        o = Als3Opts()
        lib.cptc_als3_default_opts(C.byref(o))
        o.R, o.threshold, o.path, o.fill_min = R, threshold, path, fill_min
        o.cadr, o.seed, o.verbose = int(cadr), seed, int(verbose)
        o.skip_dense, o.skip_sparse = skip_dense, skip_sparse
        o.fused = fused
        c, keep = t.as_coo()
        h = C.c_void_p()
        check(lib.cptc_als3_create(C.byref(c), C.byref(o), C.byref(h)), "cptc_als3_create")
        del keep
        self._h = h
        self.R = R
        self.info = Als3Info()
        check(lib.cptc_als3_info_get(h, C.byref(self.info)), "cptc_als3_info_get")
        self.dims = tuple(int(x) for x in self.info.dims)

    def close(self) -> None:
        if getattr(self, "_h", None):
            lib.cptc_als3_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def refresh_info(self):
        """Re-reads cptc_als3_info (graph captures change as runs proceed)."""
        check(lib.cptc_als3_info_get(self._h, C.byref(self.info)), "cptc_als3_info_get")
        return self.info

    def run(self, iters: int):
        fit = np.zeros(iters, np.float64)
        ms = np.zeros(iters, np.float32)
        mt = np.zeros(iters, np.float32)
        check(lib.cptc_als3_run(self._h, iters, fit.ctypes.data, ms.ctypes.data, mt.ctypes.data),
              "cptc_als3_run")
        return fit, ms, mt

    def kernel_times(self, reset: bool = True):
        """(sparse-kernel ms per mode, all-MTTKRP ms per mode, iterations)."""
        out = np.zeros(6, np.float64)
        it = C.c_int()
        check(lib.cptc_als3_kernel_times(self._h, out.ctypes.data, C.byref(it), int(reset)),
              "cptc_als3_kernel_times")
        return out[:3], out[3:], it.value

    def tile_times(self) -> np.ndarray:
        """MFMA tile-kernel ms per mode since the last kernel_times(reset=True)."""
        out = np.zeros(3, np.float64)
        check(lib.cptc_als3_tile_times(self._h, out.ctypes.data), "cptc_als3_tile_times")
        return out

    def gather_probe(self, reps: int = 3) -> np.ndarray:
        """ms per launch, per mode, of the element-gather probe on the blocked
        residual view (the blocked kernel's element-level row gathers alone,
        same order and occupancy): the floor those gathers set."""
        out = np.zeros(3, np.float64)
        check(lib.cptc_als3_gather_probe(self._h, int(reps), out.ctypes.data),
              "cptc_als3_gather_probe")
        return out

    def sgd(self, iters: int, gamma: float = 1e-9, batch: int = 1 << 20,
            seed: int = 42) -> np.ndarray:
        """CP-SGD on the residual (ALS_SGD); batch RMSE per iteration (-1 where
        the loop does not evaluate it)."""
        out = np.zeros(max(iters, 1), np.float64)
        check(lib.cptc_als3_sgd(self._h, iters, gamma, batch, seed, out.ctypes.data),
              "cptc_als3_sgd")
        return out[:iters]

    def mttkrp(self, mode: int) -> np.ndarray:
        out = np.zeros((self.dims[mode], self.R), np.float64)
        check(lib.cptc_als3_mttkrp(self._h, mode, out.ctypes.data), "cptc_als3_mttkrp")
        return out

    def factor(self, mode: int, unpermuted: bool = False) -> np.ndarray:
        out = np.zeros((self.dims[mode], self.R), np.float64)
        check(lib.cptc_als3_factor(self._h, mode, int(unpermuted), out.ctypes.data),
              "cptc_als3_factor")
        return out

    def set_factor(self, mode: int, f: np.ndarray) -> None:
        f = np.ascontiguousarray(f, np.float64)
        assert f.shape == (self.dims[mode], self.R)
        check(lib.cptc_als3_set_factor(self._h, mode, f.ctypes.data), "cptc_als3_set_factor")

    def lam(self) -> np.ndarray:
        out = np.zeros(self.R, np.float64)
        check(lib.cptc_als3_lambda(self._h, out.ctypes.data), "cptc_als3_lambda")
        return out

    def residual(self):
        r, x = C.c_double(), C.c_double()
        check(lib.cptc_als3_residual(self._h, C.byref(r), C.byref(x)), "cptc_als3_residual")
        return r.value, x.value

    def perm(self, mode: int) -> np.ndarray:
        out = np.zeros(self.dims[mode], np.int32)
        check(lib.cptc_als3_perm(self._h, mode, out.ctypes.data), "cptc_als3_perm")
        return out

    def view(self, which: int, mode: int) -> dict:
        """Row-sorted view `which` of `mode`: 0 residual, 1 FP64 dense view, 2
        the FP64-only path's merged view over every nonzero (info.fp64_merged)."""
        i = self.info
        nnz = (int(i.sparse_nnz), int(i.dense_nnz), int(i.nnz))[which]
        nseg = int((i.segments, i.dense_view_segments, i.merged_segments)[which][mode])
        if nseg == 0:
            nnz = 0
        d = {
            "coords": np.zeros(nnz, np.uint64), "vals": np.zeros(nnz, np.float64),
            "blk_row": np.zeros(nseg, np.uint32), "blk_start": np.zeros(nseg, np.uint32),
            "blk_cnt": np.zeros(nseg, np.uint32),
        }
        check(lib.cptc_als3_view(self._h, which, mode, *(d[k].ctypes.data for k in
                                                          ("coords", "vals", "blk_row",
                                                           "blk_start", "blk_cnt"))),
              "cptc_als3_view")
        return d

    def tiles(self) -> dict:
        nt = int(self.info.num_dense_tiles)
        nd = int(self.info.dense_nnz)
        d = {"tiles": np.zeros((nt, 4), np.int32), "pool_off": np.zeros(nt + 1, np.uint64),
             "pool_lid": np.zeros(nd, np.int32), "pool_val": np.zeros(nd, np.float64)}
        check(lib.cptc_als3_tiles(self._h, d["tiles"].ctypes.data, d["pool_off"].ctypes.data,
                                  d["pool_lid"].ctypes.data, d["pool_val"].ctypes.data),
              "cptc_als3_tiles")
        return d


def gen_reorder(t: Tensor, how: str | None = None, rounds: int = 3,
                sample_budget: int = 8000000) -> tuple[Tensor, list, bool]:
    """apply_reordering (generic.cu:1176-1376) on a copy: (relabelled tensor,
    per-mode rank maps new = rank[old], applied)."""
    work = Tensor(tuple(t.dims), np.array(t.idx, dtype=np.uint32, order="C", copy=True), t.val)
    c, keep = work.as_coo()
    rank = np.zeros(int(sum(t.dims)), np.uint32)
    applied = C.c_int()
    check(lib.cptc_gen_reorder(C.byref(c), None if how is None else how.encode(), rounds,
                               sample_budget, rank.ctypes.data, C.byref(applied)),
          "cptc_gen_reorder")
    idx = keep[0].copy()
    ranks, off = [], 0
    for d in t.dims:
        ranks.append(rank[off:off + d].copy())
        off += d
    return Tensor(tuple(t.dims), idx, t.val.copy()), ranks, bool(applied.value)


def gen_hash(x: int) -> int:
    return int(lib.cptc_gen_hash(x))


def gen_selftest(verbose: bool = False) -> int:
    """run_dense_selftest (generic.cu:1389-1637); returns the failure count."""
    f = C.c_int()
    check(lib.cptc_gen_selftest(int(verbose), C.byref(f)), "cptc_gen_selftest")
    return f.value


class Gen:
    """Generic N-order CP-ALS on the device (reorder, units, views, factors)."""

    def __init__(self, t: Tensor, R: int = 16, seed: int = 42, reorder: str | None = None,
                 rounds: int = 3, sample: int = 8000000, dense: bool = True,
                 threshold: float = 0.03, inner=(0, 1, 2), svd: bool = False,
                 profile: bool = False, verbose: bool = False):
        o = GenOpts()
        lib.cptc_gen_default_opts(C.byref(o))
        o.R, o.seed = R, seed
        o.reorder = (reorder or "").encode()
        o.reorder_rounds, o.reorder_sample = rounds, sample
        o.dense, o.threshold = int(dense), threshold
        for q in range(3):
            o.inner[q] = inner[q]
        o.svd, o.profile, o.verbose = int(svd), int(profile), int(verbose)
        c, keep = t.as_coo()
        h = C.c_void_p()
        check(lib.cptc_gen_create(C.byref(c), C.byref(o), C.byref(h)), "cptc_gen_create")
        del keep
        self._h = h
        self.R = R
        self.info = GenInfo()
        check(lib.cptc_gen_info_get(h, C.byref(self.info)), "cptc_gen_info_get")
        self.N = int(self.info.nmodes)
        self.dims = tuple(int(self.info.dims[m]) for m in range(self.N))
        self.nnz = int(self.info.nnz)

    def close(self) -> None:
        if getattr(self, "_h", None):
            lib.cptc_gen_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def run(self, iters: int):
        """(fit, iprod, model2, ms) per iteration."""
        out = [np.zeros(iters, np.float64) for _ in range(4)]
        check(lib.cptc_gen_run(self._h, iters, *(a.ctypes.data for a in out)), "cptc_gen_run")
        return tuple(out)

    def profile(self, reset: bool = True):
        out = np.zeros(5, np.float64)
        it = C.c_int()
        check(lib.cptc_gen_profile(self._h, out.ctypes.data, C.byref(it), int(reset)),
              "cptc_gen_profile")
        return out, it.value

    def kernel_times(self, reset: bool = True):
        """(segment-kernel ms per mode, unit-kernel ms per mode, iterations
        timed).  Queued runs time the kernels on every 8th iteration and on
        the last one; verbose or profiled runs on every iteration.  Outer
        modes on the per-unit-sum path report the scatter as their segment
        kernel and the per-unit sums (where formed) as their unit kernel."""
        out = np.zeros(16, np.float64)
        it = C.c_int()
        check(lib.cptc_gen_kernel_times(self._h, out.ctypes.data, C.byref(it), int(reset)),
              "cptc_gen_kernel_times")
        return out[:self.N], out[8:8 + self.N], it.value

    def mttkrp(self, mode: int) -> np.ndarray:
        out = np.zeros((self.dims[mode], self.R), np.float64)
        check(lib.cptc_gen_mttkrp(self._h, mode, out.ctypes.data), "cptc_gen_mttkrp")
        return out

    def factor(self, mode: int) -> np.ndarray:
        out = np.zeros((self.dims[mode], self.R), np.float64)
        check(lib.cptc_gen_factor(self._h, mode, out.ctypes.data), "cptc_gen_factor")
        return out

    def set_factor(self, mode: int, f: np.ndarray) -> None:
        f = np.ascontiguousarray(f, np.float64)
        assert f.shape == (self.dims[mode], self.R)
        check(lib.cptc_gen_set_factor(self._h, mode, f.ctypes.data), "cptc_gen_set_factor")

    def lam(self) -> np.ndarray:
        out = np.zeros(self.R, np.float64)
        check(lib.cptc_gen_lambda(self._h, out.ctypes.data), "cptc_gen_lambda")
        return out

    def residual(self):
        r, x = C.c_double(), C.c_double()
        check(lib.cptc_gen_residual(self._h, C.byref(r), C.byref(x)), "cptc_gen_residual")
        return r.value, x.value

    def rank(self, mode: int) -> np.ndarray:
        out = np.zeros(self.dims[mode], np.uint32)
        check(lib.cptc_gen_rank(self._h, mode, out.ctypes.data), "cptc_gen_rank")
        return out

    def coords(self) -> np.ndarray:
        out = np.zeros((self.N, self.nnz), np.uint32)
        check(lib.cptc_gen_coords(self._h, out.ctypes.data), "cptc_gen_coords")
        return out

    def view(self, mode: int) -> dict:
        nnz, nseg = self.nnz, int(self.info.nseg[mode])
        d = {"scoords": np.zeros((self.N - 1, nnz), np.uint32),
             "vals": np.zeros(nnz, np.float64), "skip": np.zeros(nnz, np.uint8),
             "row": np.zeros(nseg, np.uint32), "start": np.zeros(nseg, np.uint32),
             "cnt": np.zeros(nseg, np.uint32), "single": np.zeros(nseg, np.uint8)}
        check(lib.cptc_gen_view(self._h, mode, *(d[k].ctypes.data for k in
                                                 ("scoords", "vals", "skip", "row", "start",
                                                  "cnt", "single"))), "cptc_gen_view")
        return d

    def units(self) -> dict:
        nu, nd = int(self.info.n_units), int(self.info.dense_nnz)
        nout = max(self.N - 3, 0)
        d = {"unit6": np.zeros((nu, 6), np.uint32), "outer_coords": np.zeros(nu * nout, np.uint32),
             "lid": np.zeros(nd, np.uint32), "val": np.zeros(nd, np.float64),
             "is_dense": np.zeros(self.nnz, np.uint8)}
        check(lib.cptc_gen_units(self._h, *(d[k].ctypes.data for k in
                                            ("unit6", "outer_coords", "lid", "val",
                                             "is_dense"))), "cptc_gen_units")
        return d

    def dump(self, base: str, input_order: bool = False) -> None:
        """GEN_DUMP to <base>.factors.txt (reordered rows, as the reference),
        or with input_order=True in the input tensor's index order."""
        check(lib.cptc_gen_dump_ex(self._h, base.encode(), int(input_order)), "cptc_gen_dump_ex")
