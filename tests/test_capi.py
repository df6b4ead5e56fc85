"""The C ABI library: loads, exports every symbol include/cptc_hip.h declares,
and rejects bad arguments with CPTC_ERR_ARG before touching a device (so
these run on a host without a GPU)."""
import ctypes as C
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    syms = set()
    for name in os.listdir(os.path.join(ROOT, "include")):
        if name.endswith(".h"):
            text = open(os.path.join(ROOT, "include", name)).read()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            syms |= set(re.findall(r"\b(cptc_[a-z0-9_]+)\s*\(", text))
    return syms


def test_library_exports_every_declared_symbol(ca):
    lib = C.CDLL(ca.LIB_PATH)
    syms = declared_symbols()
    assert len(syms) >= 30
    for s in sorted(syms):
        assert hasattr(lib, s), f"{s} declared but not exported"
    assert syms == set(ca.SIGNATURES), "Python bindings out of sync with the header"


def test_version_and_no_device_here(ca):
    assert b"gfx950" in ca.lib.cptc_version()
    assert ca.lib.cptc_device_count() >= 0


@pytest.mark.parametrize("call", [
    lambda l: l.cptc_mttkrp_sparse3(3, 0, 0, 0, 0, 0, 10, 0, 0, 0, 32, None),
    lambda l: l.cptc_mttkrp_sparse3(0, 0, 0, 0, 0, 0, 10, 0, 0, 0, 0, None),
    lambda l: l.cptc_mttkrp_sparse3(0, 0, 0, 0, 0, 0, 10, 0, 0, 0, 32, None),
    lambda l: l.cptc_mttkrp_dense_tiles3(5, 0, 0, 1, None, None, 0, 0, 0, 0, 0, 16, 1, 1, 1,
                                         None),
    lambda l: l.cptc_mttkrp_dense_tiles3(0, 0, 0, 1, None, None, 0, 0, 0, 0, 0, 16, 1, 1, 1,
                                         None),
    lambda l: l.cptc_dense_groups(None, 4, 3, 0, 8, None, None, None),
    lambda l: l.cptc_mttkrp_units_nd(3, 0, 1, 0, 0, None, None, 0, 0, 0, 0, 1, 1, 1, 0, 8, None),
    lambda l: l.cptc_gram(0, 10, 8, 0, None),
    lambda l: l.cptc_hadamard(0, 0, 0, 10, None),
    lambda l: l.cptc_solve_pinv(0, 0, 0, 10, 8, 0, None),
    lambda l: l.cptc_solve_pinv_noalloc(0, 0, 0, 10, 8, 0, None),
    lambda l: l.cptc_solve_pinv_noalloc(8, 8, 8, 10, 129, 0, None),
    lambda l: l.cptc_pinv_sym(0, 0, 1024, 0, None),
    lambda l: l.cptc_colnorms(0, 10, 8, 0, None),
    lambda l: l.cptc_normalize_absorb(0, 10, 8, 0, 0, None),
    lambda l: l.cptc_fit_gram(0, 0, 10, 0, 0, 3, 8, 0, None),
    lambda l: l.cptc_residual3_view(0, 0, 10, 0, 0, 0, 0, 8, 0, None),
    lambda l: l.cptc_residual3_tiles(0, 0, 0, 0, 1, 0, 0, 0, 0, 8, 0, None),
    lambda l: l.cptc_unpermute_factor(0, 0, 0, 10, 8, None),
    lambda l: l.cptc_dense_tiles_pack3(0, 0, 0, 4, 0, None),
    lambda l: l.cptc_als3_run(None, 1, None, None, None),
    lambda l: l.cptc_als3_info_get(None, None),
    # odd R, 4-byte keys for 40 bits, a level wider than 32 bits
    lambda l: l.cptc_mttkrp_seg_nd_keys(3, 0, 1, 4, (C.c_int * 2)(1, 2), (C.c_int * 2)(4, 4), 1,
                                        10, 1, 1, 1, None, 1, (C.c_void_p * 3)(16, 16, 16), 1,
                                        7, None),
    lambda l: l.cptc_mttkrp_seg_nd_keys(3, 0, 1, 4, (C.c_int * 2)(1, 2), (C.c_int * 2)(20, 20),
                                        1, 10, 1, 1, 1, None, 1, (C.c_void_p * 3)(16, 16, 16), 1,
                                        8, None),
    lambda l: l.cptc_pack_level_keys(2, 1, 10, (C.c_int * 2)(33, 1), 1, 8, None),
    # one-launch update: rows past 4096, R past 32, no rows, the next pinv
    # without the next FtF, a fit without the Grams, null pointers
    lambda l: l.cptc_update_small3(8, 8, 8, 4097, 8, 8, 8, 8, None, None, 0, None, None, 0, None),
    lambda l: l.cptc_update_small3(8, 8, 8, 100, 33, 8, 8, 8, None, None, 0, None, None, 0, None),
    lambda l: l.cptc_update_small3(8, 8, 8, 0, 8, 8, 8, 8, None, None, 0, None, None, 0, None),
    lambda l: l.cptc_update_small3(8, 8, 8, 100, 8, 8, 8, 8, None, None, 0, None, None, 1, None),
    lambda l: l.cptc_update_small3(8, 8, 8, 100, 8, 8, 8, 8, None, None, 0, None, 8, 0, None),
    lambda l: l.cptc_update_small3(0, 8, 8, 100, 8, 8, 8, 8, None, None, 0, None, None, 0, None),
])
def test_bad_arguments_rejected(ca, call):
    assert call(ca.lib) == -1
    assert ca.lib.cptc_last_error() != b""


def test_empty_work_is_ok(ca):
    # zero segments / tiles: nothing to launch, success
    assert ca.lib.cptc_mttkrp_sparse3(0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 32, None) == 0
    assert ca.lib.cptc_mttkrp_dense_tiles3(0, 0, 0, 0, None, None, 0, 0, 0, 0, 0, 16, 1, 1, 1,
                                           None) == 0
    assert ca.lib.cptc_hadamard(1, 1, 1, 0, None) == 0


def test_als3_create_rejects_non_order3(ca):
    t = ca.Tensor((4, 4, 4, 4), np.zeros((4, 1), np.uint32), np.ones(1))
    with pytest.raises(ca.CptcError):
        ca.Als3(t, R=4)


def test_als3_create_rejects_out_of_range_index(ca):
    t = ca.Tensor((4, 4, 4), np.array([[0, 4], [1, 1], [2, 2]], np.uint32), np.ones(2))
    with pytest.raises(ca.CptcError, match="index"):
        ca.Als3(t, R=4)


def test_cadr3_rejects_out_of_range_index(ca):
    t = ca.Tensor((4, 4, 4), np.array([[0, 1], [1, 9], [2, 2]], np.uint32), np.ones(2))
    with pytest.raises(ca.CptcError, match="index"):
        ca.cadr3(t)


@pytest.mark.parametrize("hdr_words,slot,G", [(4, 0, 8), (4, 1, 8), (4, 2, 3), (6, 1, 16)])
def test_dense_groups(ca, hdr_words, slot, G):
    """Host group builder: the tiles sorted by (target block, others) cut into
    maximal runs of <= G tiles with one target block, the runs ordered
    longest first (stable), covering every tile."""
    import ctypes as C
    rng = np.random.default_rng(slot + G)
    n = 500
    hdr = rng.integers(0, 6, (n, hdr_words)).astype(np.int32)
    order = np.zeros(n, np.uint32)
    off = np.zeros(n + 1, np.uint32)
    ng = C.c_size_t()
    assert ca.lib.cptc_dense_groups(hdr.ctypes.data, hdr_words, n, slot, G, order.ctypes.data,
                                    off.ctypes.data, C.byref(ng)) == 0
    ng = ng.value
    assert np.array_equal(np.sort(order), np.arange(n))
    p, q = (slot + 1) % 3, (slot + 2) % 3
    # the reference partition: maximal runs of <= G over the sorted tiles
    srt = sorted(range(n), key=lambda t: tuple(hdr[t, [slot, p, q]]))
    runs, i = [], 0
    while i < n:
        j = i + 1
        while j < n and j - i < G and hdr[srt[j], slot] == hdr[srt[i], slot]:
            j += 1
        runs.append(srt[i:j])
        i = j
    runs = sorted(runs, key=lambda r: -len(r))   # stable: equal lengths keep block order
    assert off[0] == 0 and off[ng] == n and ng == len(runs)
    for g in range(ng):
        a, b = off[g], off[g + 1]
        assert list(order[a:b]) == runs[g]
        assert 1 <= b - a <= G and len(set(hdr[order[a:b], slot])) == 1
    assert all(off[g + 1] - off[g] >= off[g + 2] - off[g + 1] for g in range(ng - 1))


@pytest.mark.parametrize("chunk", [1, 3, 8])
def test_unit_sums_plan(ca, chunk):
    """Host plan of the unit-sum kernel: the units sorted stably by their
    inner block triple (words 0..2 of the 6-word header), cut into maximal
    chunks of <= `chunk` units that share one triple, covering every unit."""
    import ctypes as C
    rng = np.random.default_rng(chunk)
    n = 700
    hdr = rng.integers(0, 3, (n, 6)).astype(np.uint32)
    hdr[:, 3:] = rng.integers(0, 1000, (n, 3))
    order = np.zeros(n, np.uint32)
    off = np.zeros(n + 1, np.uint32)
    nc = C.c_size_t()
    assert ca.lib.cptc_gen_unit_sums_plan(hdr.ctypes.data, n, chunk, order.ctypes.data,
                                          off.ctypes.data, C.byref(nc)) == 0
    nc = nc.value
    ref = sorted(range(n), key=lambda u: tuple(hdr[u, :3]))   # Python's sort is stable
    assert np.array_equal(order, np.array(ref, np.uint32))
    assert off[0] == 0 and off[nc] == n
    for c in range(nc):
        a, b = off[c], off[c + 1]
        assert 1 <= b - a <= chunk
        assert len({tuple(hdr[u, :3]) for u in order[a:b]}) == 1
    for c in range(1, nc):
        a = off[c]
        if tuple(hdr[order[a], :3]) == tuple(hdr[order[a - 1], :3]):
            assert off[c] - off[c - 1] == chunk
    assert ca.lib.cptc_gen_unit_sums_plan(hdr.ctypes.data, n, 0, order.ctypes.data,
                                          off.ctypes.data, C.byref(C.c_size_t())) == -1


@pytest.mark.parametrize("bits,nbytes", [((6, 6, 6, 4), 4), ((16, 16), 4), ((17, 16), 8),
                                         ((1,), 4), ((32, 32), 8), ((32, 32, 1), 0),
                                         ((0, 5), 0), ((33,), 0)])
def test_level_key_bytes(ca, bits, nbytes):
    """Packed level keys: 4 bytes up to 32 bits, 8 up to 64, none beyond or
    for a field outside 1..32 bits."""
    assert ca.lib.cptc_level_key_bytes(len(bits), (C.c_int * len(bits))(*bits)) == nbytes
