"""The generic driver's environment switches (generic.cu:1647-1663, 1796-1840,
2114-2116; main.cu:127-130), as cptc_gen_default_opts reads them on the host:
GEN_SEED, GEN_REORDER, GEN_REORDER_T, GEN_REORDER_SAMPLE, GEN_DENSE,
GEN_DENSE_THRESHOLD, GEN_DENSE_INNER, GEN_SOLVER=svd, GEN_PROFILE.  Their
effect on a run is in tests/test_gpu_generic.py (test_cli_generic_switches)."""
import ctypes as C

import pytest

SWITCHES = ("GEN_SEED", "GEN_REORDER", "GEN_REORDER_T", "GEN_REORDER_SAMPLE", "GEN_DENSE",
            "GEN_DENSE_THRESHOLD", "GEN_DENSE_INNER", "GEN_SOLVER", "GEN_PROFILE")


def opts(ca):
    o = ca._lib.GenOpts()
    ca.lib.cptc_gen_default_opts(C.byref(o))
    return o


@pytest.fixture
def clean_env(monkeypatch):
    for k in SWITCHES:
        monkeypatch.delenv(k, raising=False)
    return monkeypatch


def test_defaults(ca, clean_env):
    """Unset: R 32, seed 42, no reorder override (the driver then picks hits
    for N >= 4, cadr for N = 3), 3 HITS rounds, an 8 M sample budget, dense
    units on at cutoff 0.03 over inner modes (0, 1, 2), Cholesky, no
    profile."""
    o = opts(ca)
    assert o.R == 32 and o.seed == 42 and o.reorder == b""
    assert o.reorder_rounds == 3 and o.reorder_sample == 8_000_000
    assert o.dense == 1 and o.threshold == 0.03 and list(o.inner) == [0, 1, 2]
    assert o.svd == 0 and o.profile == 0 and o.verbose == 0


def test_every_switch(ca, clean_env):
    env = dict(GEN_SEED="7", GEN_REORDER="none", GEN_REORDER_T="5", GEN_REORDER_SAMPLE="1000",
               GEN_DENSE="0", GEN_DENSE_THRESHOLD="0.05", GEN_DENSE_INNER="1,2,3",
               GEN_SOLVER="svd", GEN_PROFILE="1")
    for k, v in env.items():
        clean_env.setenv(k, v)
    o = opts(ca)
    assert o.seed == 7 and o.reorder == b"none"
    assert o.reorder_rounds == 5 and o.reorder_sample == 1000
    assert o.dense == 0 and o.threshold == 0.05 and list(o.inner) == [1, 2, 3]
    assert o.svd == 1 and o.profile == 1


@pytest.mark.parametrize("val,svd", [("svd", 1), ("chol", 0), ("SVD", 0), ("", 0)])
def test_solver_only_svd(ca, clean_env, val, svd):
    """Only the exact string "svd" selects the pseudoinverse (generic.cu:2114-2116)."""
    clean_env.setenv("GEN_SOLVER", val)
    assert opts(ca).svd == svd


@pytest.mark.parametrize("val,inner", [("0,1,2", [0, 1, 2]), ("2,0,3", [2, 0, 3]),
                                       ("1", [1, 1, 2]), ("4,5", [4, 5, 2])])
def test_dense_inner_list(ca, clean_env, val, inner):
    """GEN_DENSE_INNER is read as up to three comma-separated integers over the
    default (0, 1, 2); whether the set is usable (three distinct modes of the
    tensor) is decided when the driver is created."""
    clean_env.setenv("GEN_DENSE_INNER", val)
    assert list(opts(ca).inner) == inner
