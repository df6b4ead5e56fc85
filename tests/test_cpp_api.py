"""The C++ interface (include/*.hpp, the reference's function names): the
headers compile on their own, and libcptc.so exports every function they
declare.  No GPU needed."""
import os
import re
import subprocess

import pytest

import cptc_amd as ca

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = ["tensor.hpp", "cadr.hpp", "partition.hpp", "sparse.hpp", "dense.hpp", "solver.hpp",
           "sgd.hpp",
           "als.hpp", "common.hpp", "compute_fit.hpp", "generic.hpp"]

# every non-inline function the headers declare (reference names)
FUNCTIONS = [
    "load_tns_file", "free_coo_tensor", "compute_cadr_reordering", "apply_cadr_reordering",
    "unpermute_factor_matrices", "free_cadr_permutation", "partition_tensor_hybrid",
    "partition_tensor_hybrid_gpu", "free_hybrid_tensor", "build_mttkrp_views",
    "build_dense_mttkrp_views", "compute_sparse_mttkrp_async", "compute_sparse_mttkrp",
    "compute_dense_mttkrp_async", "compute_dense_mttkrp", "compute_mttkrp_merged_async",
    "execute_sgd_decomposition",
    "init_svd_workspace", "free_svd_workspace", "solve_als_system_svd",
    "solve_als_system_svd_nosync", "execute_als_decomposition", "debug_device_state",
    "init_factors_random", "clamp_factor_thrust", "calculate_rmse",
    "compute_residual_and_norm_sq", "compute_fit", "print_fit_report", "probe_tns_nmodes",
    "load_tns_generic", "run_dense_selftest", "run_generic_cp",
]


def test_headers_compile_standalone(tmp_path):
    for h in HEADERS:
        src = tmp_path / f"inc_{h}.cpp"
        src.write_text(f'#include "{h}"\n#include "{h}"\nint main() {{ return 0; }}\n')
        r = subprocess.run(["g++", "-std=c++17", "-fsyntax-only", "-Wall", "-Werror",
                            "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROOT, "include"),
                            "-I", "/opt/rocm/include", str(src)], capture_output=True, text=True)
        assert r.returncode == 0, (h, r.stderr[-2000:])


def test_inline_helpers_roundtrip(tmp_path):
    """partition.hpp's block / local-id encodings invert each other."""
    src = tmp_path / "enc.cpp"
    src.write_text(r'''
#include "partition.hpp"
#include <cstdio>
int main() {
    const std::size_t nbj = num_blocks_for_dim(37), nbk = num_blocks_for_dim(64);
    for (int i = 0; i < 50; i += 7) for (int j = 0; j < 37; j += 5) for (int k = 0; k < 64; k += 3) {
        BlockId b; LocalId l; encode_coordinate(i, j, k, nbj, nbk, b, l);
        int a, c, d; decode_coordinate(b, l, nbj, nbk, a, c, d);
        if (a != i || c != j || d != k) { std::printf("bad %d %d %d\n", i, j, k); return 1; }
        if (b != encode_block_id(i / 16, j / 16, k / 16, nbj, nbk)) return 2;
        if (l != (i % 16 * 16 + j % 16) * 16 + k % 16) return 3;
    }
    std::printf("ok\n");
    return 0;
}
''')
    exe = tmp_path / "enc"
    r = subprocess.run(["g++", "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I",
                        os.path.join(ROOT, "include"), "-I", "/opt/rocm/include", str(src), "-o",
                        str(exe)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0 and r.stdout.strip() == "ok", r.stdout


def test_library_exports_cpp_api():
    r = subprocess.run(["nm", "-D", "--defined-only", ca.LIB_PATH], capture_output=True,
                       text=True)
    assert r.returncode == 0
    dem = subprocess.run(["c++filt"], input=r.stdout, capture_output=True, text=True).stdout
    names = set()
    for line in dem.splitlines():
        m = re.match(r"\S+ [TW] ([A-Za-z_][A-Za-z0-9_]*)\(", line)
        if m:
            names.add(m.group(1))
    missing = [f for f in FUNCTIONS if f not in names]
    assert not missing, missing


@pytest.mark.parametrize("h", HEADERS)
def test_header_cites_reference(h):
    text = open(os.path.join(ROOT, "include", h)).read()
    assert re.search(r"\.(hpp|cu):\d+", text), h
