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

from ._lib import (CLI_PATH, LIB_PATH, SIGNATURES, Als3Info, Als3Opts, Coo, CptcError, check,
                   lib)  # noqa: F401  (check is part of the public surface)

__all__ = [
    "lib", "LIB_PATH", "CLI_PATH", "SIGNATURES", "CptcError", "Tensor", "synth_config",
    "synth_zipf", "synth_lowrank3", "synth_blocks3", "synth_units5", "load_tns3",
    "load_tns_generic", "probe_nmodes", "write_tns", "cadr3", "Als3", "device_count", "ptr",
    "DevBuf", "sync", "check",
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
        self.shape = tuple(shape) if shape is not None else (nbytes // self.dtype.itemsize,)
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


def _take(c: Coo) -> Tensor:
    try:
        n, nm = int(c.nnz), int(c.nmodes)
        if n:
            idx = np.ctypeslib.as_array(c.idx, shape=(nm * n,)).reshape(nm, n).copy()
            val = np.ctypeslib.as_array(c.val, shape=(n,)).copy()
        else:
            idx = np.zeros((nm, 0), np.uint32)
            val = np.zeros(0, np.float64)
        return Tensor(tuple(int(c.dims[m]) for m in range(nm)), idx, val)
    finally:
        lib.cptc_coo_free(C.byref(c))


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
                 skip_dense: int = -1, skip_sparse: int = -1):
        o = Als3Opts()
        lib.cptc_als3_default_opts(C.byref(o))
        o.R, o.threshold, o.path, o.fill_min = R, threshold, path, fill_min
        o.cadr, o.seed, o.verbose = int(cadr), seed, int(verbose)
        o.skip_dense, o.skip_sparse = skip_dense, skip_sparse
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
        """Row-sorted view `which` (0 residual, 1 FP64 dense view) of `mode`."""
        nnz = int(self.info.sparse_nnz) if which == 0 else int(self.info.dense_nnz)
        nseg = int(self.info.segments[mode] if which == 0 else self.info.dense_view_segments[mode])
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
