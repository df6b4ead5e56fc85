"""ctypes binding of libcptc.so (the C ABI declared in include/cptc_hip.h).

The library is loaded from the package's own ``lib/`` directory; if it is
missing the import fails loudly — there is no Python or CPU fallback for any
entry point.
"""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
# CPTC_LIB_PATH overrides the library location (e.g. an alternative build)
LIB_PATH = os.environ.get("CPTC_LIB_PATH") or os.path.join(_HERE, "lib", "libcptc.so")
CLI_PATH = os.path.join(_HERE, "bin", "cptc_opt")

CPTC_MAX_MODES = 8
CPTC_SEG = 1024
OK, ERR_ARG, ERR_HIP, ERR_UNSUPPORTED, ERR_IO, ERR_NUMERIC, ERR_STATE = 0, -1, -2, -3, -4, -5, -6
VAL_LOGNORMAL, VAL_NORMAL, VAL_POISSON1P2 = 0, 1, 2


class CptcError(RuntimeError):
    def __init__(self, where: str, rc: int, msg: str):
        super().__init__(f"{where} failed ({rc}): {msg}")
        self.rc = rc


class Coo(C.Structure):
    _fields_ = [
        ("nmodes", C.c_int),
        ("dims", C.c_uint64 * CPTC_MAX_MODES),
        ("nnz", C.c_uint64),
        ("idx", C.POINTER(C.c_uint32)),
        ("val", C.POINTER(C.c_double)),
    ]


class Als3Opts(C.Structure):
    _fields_ = [
        ("R", C.c_int),
        ("threshold", C.c_double),
        ("path", C.c_int),
        ("fill_min", C.c_double),
        ("skip_dense", C.c_int),
        ("skip_sparse", C.c_int),
        ("cadr", C.c_int),
        ("seed", C.c_uint64),
        ("verbose", C.c_int),
        ("fused", C.c_int),
    ]


class Als3Info(C.Structure):
    _fields_ = [
        ("dims", C.c_uint64 * 3),
        ("nnz", C.c_uint64),
        ("sparse_nnz", C.c_uint64),
        ("dense_nnz", C.c_uint64),
        ("num_dense_tiles", C.c_int64),
        ("dense_cutoff", C.c_int),
        ("avg_fill", C.c_double),
        ("fill_min", C.c_double),
        ("use_mfma", C.c_int),
        ("segments", C.c_uint64 * 3),
        ("dense_view_segments", C.c_uint64 * 3),
        ("num_cus", C.c_int),
        ("fused", C.c_int),
        ("sparse_blocked", C.c_int),
        ("tile_bf16x3", C.c_int),
        ("tiles_beside", C.c_int),
        ("tile_compact", C.c_int),
        ("tile_segments", C.c_uint64 * 3),
        ("graph_mode", C.c_int),
        ("graph_captures", C.c_int),
        ("fp64_merged", C.c_int),
        ("merged_segments", C.c_uint64 * 3),
        ("small_update", C.c_int),
    ]


class GenOpts(C.Structure):
    _fields_ = [
        ("R", C.c_int),
        ("seed", C.c_uint),
        ("reorder", C.c_char * 8),
        ("reorder_rounds", C.c_int),
        ("reorder_sample", C.c_uint64),
        ("dense", C.c_int),
        ("threshold", C.c_double),
        ("inner", C.c_int * 3),
        ("svd", C.c_int),
        ("profile", C.c_int),
        ("verbose", C.c_int),
    ]


class GenInfo(C.Structure):
    _fields_ = [
        ("nmodes", C.c_int),
        ("dims", C.c_uint64 * CPTC_MAX_MODES),
        ("nnz", C.c_uint64),
        ("R", C.c_int),
        ("reorder", C.c_char * 8),
        ("reordered", C.c_int),
        ("dense_enabled", C.c_int),
        ("cutoff", C.c_int),
        ("inner", C.c_int * 3),
        ("n_units", C.c_uint64),
        ("dense_nnz", C.c_uint64),
        ("nseg", C.c_uint64 * CPTC_MAX_MODES),
        ("prep_ms", C.c_double * 3),
        ("kernel_nnz", C.c_uint64 * CPTC_MAX_MODES),
        ("tile_bf16x3", C.c_int),
        ("unit_segments", C.c_uint64 * 3),
        ("unit_sums", C.c_int),
        ("unit_sums_img", C.c_int),
    ]


_P = C.c_void_p
_I = C.c_int
_Z = C.c_size_t
_D = C.c_double
_U64 = C.c_uint64

# name -> (restype, argtypes); every symbol declared in include/cptc_hip.h
SIGNATURES = {
    "cptc_coo_free": (None, [C.POINTER(Coo)]),
    "cptc_version": (C.c_char_p, []),
    "cptc_last_error": (C.c_char_p, []),
    "cptc_device_count": (_I, []),
    "cptc_dev_malloc": (_I, [_Z, C.POINTER(_P)]),
    "cptc_dev_free": (_I, [_P]),
    "cptc_dev_upload": (_I, [_P, _P, _Z]),
    "cptc_dev_download": (_I, [_P, _P, _Z]),
    "cptc_dev_memset": (_I, [_P, _I, _Z]),
    "cptc_dev_sync": (_I, []),
    "cptc_tns_load3": (_I, [C.c_char_p, C.POINTER(Coo)]),
    "cptc_tns_probe_nmodes": (_I, [C.c_char_p]),
    "cptc_tns_load_generic": (_I, [C.c_char_p, C.POINTER(Coo)]),
    "cptc_tns_write": (_I, [C.c_char_p, C.POINTER(Coo)]),
    "cptc_synth_config": (_I, [_I, _U64, C.POINTER(Coo)]),
    "cptc_synth_zipf": (_I, [_I, _P, _P, _U64, _I, _U64, C.POINTER(Coo)]),
    "cptc_synth_lowrank3": (_I, [_U64, _I, _D, _D, _U64, C.POINTER(Coo)]),
    "cptc_synth_blocks3": (_I, [_U64, _I, _D, _D, _D, _U64, C.POINTER(Coo)]),
    "cptc_synth_units5": (_I, [_P, _I, _D, _D, _U64, _I, _U64, C.POINTER(Coo)]),
    "cptc_cadr3": (_I, [_P, _P, _P, _Z, _P, _P, _P, _P, _I]),
    "cptc_unpermute_factor": (_I, [_P, _P, _P, _Z, _I, _P]),
    "cptc_mttkrp_sparse3": (_I, [_I, _P, _P, _P, _P, _P, _Z, _P, _P, _P, _I, _P]),
    "cptc_mttkrp_sparse3_range": (_I, [_I, _P, _P, _Z, _Z, _P, _P, _P, _I, _P]),
    "cptc_mttkrp_dense_tiles3": (_I, [_I, _P, _P, _Z, _P, _P, _Z, _P, _P, _P, _P, _I, _I, _I,
                                      _I, _P]),
    "cptc_tile_operands_bytes": (_Z, [C.c_uint64, _I]),
    "cptc_mttkrp_dense_tiles3_ws": (_I, [_I, _P, _P, _Z, _P, _P, _Z, _P, _P, _P, _P, _I, _I, _I,
                                         _I, _P, _Z, _P]),
    "cptc_dense_tiles_compact3_mask": (_I, [_P, _Z, _I, _P, _P, C.POINTER(C.c_uint64), _P]),
    "cptc_dense_tiles_compact3_fill": (_I, [_P, _Z, _I, _P, _P, _P, _P]),
    "cptc_mttkrp_dense_tiles3_cws": (_I, [_I, _P, _P, _P, _P, C.c_uint64, _Z, _P, _P, _Z, _P, _P,
                                          _P, _P, _I, _I, _I, _I, _P, _Z, _P]),
    "cptc_dense_groups": (_I, [_P, _I, _Z, _I, _I, _P, _P, C.POINTER(_Z)]),
    "cptc_dense_tiles_pack3": (_I, [_P, _P, _P, _Z, _P, _P]),
    "cptc_gram": (_I, [_P, _Z, _I, _P, _P]),
    "cptc_gram_normalize_absorb": (_I, [_P, _Z, _I, _P, _P, _P, _P]),
    "cptc_zero": (_I, [_P, _Z, _P]),
    "cptc_gram_normalize_absorb_next": (_I, [_P, _Z, _I, _P, _P, _P, _P, _P, _P]),
    "cptc_hadamard": (_I, [_P, _P, _P, _Z, _P]),
    "cptc_update_small3": (_I, [_P, _P, _P, _Z, _I, _P, _P, _P, _P, _P, _Z, _P, _P, _I, _P]),
    "cptc_solve_pinv": (_I, [_P, _P, _P, _Z, _I, _P, _P]),
    "cptc_mttkrp_sparse3_blk": (_I, [_I, _P, _P, _P, _P, _P, _P, _P, _P, _Z, _P, _P, _P, _I,
                                     C.c_uint64, C.c_uint64, _P]),
    "cptc_gather_probe3_blk": (_I, [_I, _P, _P, _P, _P, _P, _Z, _P, _I, _P, _P]),
    "cptc_mttkrp_merged3": (_I, [_I, _P, _P, _Z, _P, _P, _Z, _P, _P, _P, _P, _P, _Z, _P, _P, _P,
                                 _P, _I, _I, _I, _I, _P]),
    "cptc_mttkrp_merged3_ex": (_I, [_I, _P, _P, _Z, _P, _P, _Z, _P, _P, _P, _P, _P, _Z, _P, _P,
                                    _P, _P, _I, _I, _I, _I, _I, _I, _P]),
    "cptc_solve_pinv_noalloc": (_I, [_P, _P, _P, _Z, _I, _P, _P]),
    "cptc_pinv_sym": (_I, [_P, _P, _I, _P, _P]),
    "cptc_apply_pinv": (_I, [_P, _P, _P, _Z, _I, _P, _P]),
    "cptc_colnorms": (_I, [_P, _Z, _I, _P, _P]),
    "cptc_normalize_absorb": (_I, [_P, _Z, _I, _P, _P, _P]),
    "cptc_clamp": (_I, [_P, _Z, _D, _D, _P]),
    "cptc_fit_gram": (_I, [_P, _P, _Z, _P, _P, _I, _I, _P, _P]),
    "cptc_residual3_view": (_I, [_P, _P, _Z, _P, _P, _P, _P, _I, _P, _P]),
    "cptc_residual3_tiles": (_I, [_P, _P, _P, _P, _Z, _P, _P, _P, _P, _I, _P, _P]),
    "cptc_als3_default_opts": (None, [C.POINTER(Als3Opts)]),
    "cptc_als3_create": (_I, [C.POINTER(Coo), C.POINTER(Als3Opts), C.POINTER(_P)]),
    "cptc_als3_info_get": (_I, [_P, C.POINTER(Als3Info)]),
    "cptc_als3_run": (_I, [_P, _I, _P, _P, _P]),
    "cptc_als3_mttkrp": (_I, [_P, _I, _P]),
    "cptc_als3_kernel_times": (_I, [_P, _P, C.POINTER(_I), _I]),
    "cptc_als3_tile_times": (_I, [_P, _P]),
    "cptc_als3_gather_probe": (_I, [_P, _I, _P]),
    "cptc_als3_sgd": (_I, [_P, _I, _D, C.c_uint32, C.c_uint64, _P]),
    "cptc_sgd3_sample": (_I, [_P, C.c_uint32, C.c_uint64, C.c_uint64, _P]),
    "cptc_sgd3_update": (_I, [_P, _P, _P, C.c_uint32, _P, _P, _P, _P, _I, _D, _P]),
    "cptc_sgd3_loss": (_I, [_P, _P, _P, C.c_uint32, _P, _P, _P, _P, _I, _P, _P]),
    "cptc_sgd3_normalize": (_I, [_P, _Z, _I, _P, _P]),
    "cptc_sgd3_run": (_I, [_P, _P, C.c_uint64, _P, _P, _P, _P, _P, _I, _I, _D, C.c_uint32,
                           C.c_uint64, _I, _P, _P]),
    "cptc_als3_factor": (_I, [_P, _I, _I, _P]),
    "cptc_als3_set_factor": (_I, [_P, _I, _P]),
    "cptc_als3_lambda": (_I, [_P, _P]),
    "cptc_als3_residual": (_I, [_P, C.POINTER(_D), C.POINTER(_D)]),
    "cptc_als3_perm": (_I, [_P, _I, _P]),
    "cptc_als3_view": (_I, [_P, _I, _I, _P, _P, _P, _P, _P]),
    "cptc_als3_tiles": (_I, [_P, _P, _P, _P, _P]),
    "cptc_als3_destroy": (_I, [_P]),
    "cptc_gen_reorder": (_I, [C.POINTER(Coo), C.c_char_p, _I, _U64, _P, C.POINTER(_I)]),
    "cptc_gen_hash": (_U64, [_U64]),
    "cptc_mttkrp_seg_nd": (_I, [_I, _I, _P, _P, _P, _P, _U64, _P, _P, _P, _P, _U64, _P, _P, _I,
                                _P]),
    "cptc_level_key_bytes": (_I, [_I, _P]),
    "cptc_pack_level_keys": (_I, [_I, _P, _U64, _P, _P, _I, _P]),
    "cptc_mttkrp_seg_nd_keys": (_I, [_I, _I, _P, _I, _P, _P, _P, _U64, _P, _P, _P, _P, _U64, _P,
                                     _P, _I, _P]),
    "cptc_mttkrp_seg_nd_keys_dims": (_I, [_I, _I, _P, _I, _P, _P, _P, _U64, _P, _P, _P, _P,
                                          _U64, _P, _P, _P, _I, _P]),
    "cptc_units_pack_nd": (_I, [_P, _U64, _P, _P, _P, _P]),
    "cptc_units_pack_nd_f64": (_I, [_P, _U64, _P, _P, _P, _P]),
    "cptc_units_weights_nd": (_I, [_P, _U64, _P, _I, _P, _P, _I, _P, _P]),
    "cptc_mttkrp_units_nd": (_I, [_I, _P, _U64, _P, _P, _P, _P, _Z, _P, _P, _P, _I, _I, _I, _P,
                                  _I, _P]),
    "cptc_gen_normalize_gram": (_I, [_P, _Z, _I, _P, _P, _I, _I, _I, _P, _P, _Z, _P]),
    "cptc_mttkrp_units_nd_cws": (_I, [_I, _P, _U64, _P, _P, _P, C.c_uint64, _P, _P, _P, _Z, _P,
                                      _P, _P, _I, _I, _I, _P, _I, _P, _Z, _P]),
    "cptc_mttkrp_units_nd_ws": (_I, [_I, _P, _U64, _P, _P, _P, _P, _Z, _P, _P, _P, _I, _I, _I,
                                     _P, _I, _P, _Z, _P]),
    "cptc_gram_hadamard": (_I, [_P, _I, _I, _I, _P, _P]),
    "cptc_gen_unit_sums": (_I, [_P, _Z, _P, _P, _P, _P, _Z, _P, _P, _P, _I, _I, _I, _I, _P,
                                _P]),
    "cptc_gen_unit_sums_img": (_I, [_P, _Z, _P, _P, _P, _Z, _P, _P, _P, _I, _I, _I, _I, _P,
                                   _P]),
    "cptc_gen_unit_sums_plan": (_I, [_P, _Z, _I, _P, _P, _P]),
    "cptc_gen_unit_scatter": (_I, [_P, _Z, _I, _I, _P, _P, _I, _Z, _P, _P]),
    "cptc_chol_ridge_solve": (_I, [_P, _P, _P, _Z, _I, _P]),
    "cptc_chol_ridge_factor": (_I, [_P, _P, _I, _P]),
    "cptc_chol_ridge_apply": (_I, [_P, _P, _P, _Z, _I, _P]),
    "cptc_gen_normalize": (_I, [_P, _Z, _I, _P, _P]),
    "cptc_residual_nd": (_I, [_I, _P, _P, _U64, _P, _P, _I, _P, _P]),
    "cptc_gen_default_opts": (None, [C.POINTER(GenOpts)]),
    "cptc_gen_create": (_I, [C.POINTER(Coo), C.POINTER(GenOpts), C.POINTER(_P)]),
    "cptc_gen_info_get": (_I, [_P, C.POINTER(GenInfo)]),
    "cptc_gen_run": (_I, [_P, _I, _P, _P, _P, _P]),
    "cptc_gen_profile": (_I, [_P, _P, C.POINTER(_I), _I]),
    "cptc_gen_kernel_times": (_I, [_P, _P, C.POINTER(_I), _I]),
    "cptc_gen_mttkrp": (_I, [_P, _I, _P]),
    "cptc_gen_factor": (_I, [_P, _I, _P]),
    "cptc_gen_set_factor": (_I, [_P, _I, _P]),
    "cptc_gen_lambda": (_I, [_P, _P]),
    "cptc_gen_residual": (_I, [_P, C.POINTER(_D), C.POINTER(_D)]),
    "cptc_gen_rank": (_I, [_P, _I, _P]),
    "cptc_gen_coords": (_I, [_P, _P]),
    "cptc_gen_view": (_I, [_P, _I, _P, _P, _P, _P, _P, _P, _P]),
    "cptc_gen_units": (_I, [_P, _P, _P, _P, _P, _P]),
    "cptc_gen_dump": (_I, [_P, C.c_char_p]),
    "cptc_gen_dump_ex": (_I, [_P, C.c_char_p, _I]),
    "cptc_gen_destroy": (_I, [_P]),
    "cptc_gen_selftest": (_I, [_I, C.POINTER(_I)]),
}


def _load() -> C.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"libcptc.so not built at {LIB_PATH}; run `python -c 'import __graft_entry__ as g; g.build()'`"
        )
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def check(rc: int, where: str) -> None:
    if rc != OK:
        raise CptcError(where, rc, lib.cptc_last_error().decode(errors="replace"))
