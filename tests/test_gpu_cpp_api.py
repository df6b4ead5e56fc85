"""The C++ interface on the GPU: a small program written against the
reference-named headers (load_tns_file, partition_tensor_hybrid_gpu,
compute_dense_mttkrp) and linked with libcptc.so.  compute_dense_mttkrp
takes the split-bf16 kernel over the compacted tile image when the drivers'
rule (or ALS_TILE_KERNEL) picks it; its result is held to the FP32 MFMA
kernel of the C ABI (1e-5 relative, the dense path's bar) for every mode."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

PROG = r'''
#include <cmath>
#include <cstdio>
#include <vector>
#include "cptc_hip.h"
#include "dense.hpp"
#include "partition.hpp"
#include "tensor.hpp"

int main(int argc, char** argv)
{
    const int R = std::atoi(argv[2]);
    COOTensor t;
    load_tns_file(argv[1], t);
    HybridCOOTensor h;
    partition_tensor_hybrid_gpu(t, h, 0.03, nullptr);
    if (hipDeviceSynchronize() != hipSuccess || h.num_dense_tiles <= 0) return 2;
    double* F[3];
    for (int m = 0; m < 3; ++m)
    {
        std::vector<double> f(h.dims[m] * R);
        for (size_t x = 0; x < f.size(); ++x) f[x] = std::sin(0.37 * double(x) + m) - 0.2;
        if (hipMalloc(&F[m], f.size() * 8) != hipSuccess) return 3;
        if (hipMemcpy(F[m], f.data(), f.size() * 8, hipMemcpyHostToDevice) != hipSuccess) return 3;
    }
    // the FP32 reference kernel reads the same FP32 tile image
    float* img = nullptr;
    if (hipMalloc(&img, size_t(h.num_dense_tiles) * 4096 * 4) != hipSuccess) return 3;
    if (cptc_dense_tiles_pack3(h.d_dense_coords_pool, h.d_dense_values_pool, h.d_pool_off,
                               size_t(h.num_dense_tiles), img, nullptr) != 0) return 4;
    double worst = 0.0;
    for (int mode = 0; mode < 3; ++mode)
    {
        const size_t n = h.dims[mode] * R;
        double *a = nullptr, *b = nullptr;
        if (hipMalloc(&a, n * 8) != hipSuccess || hipMalloc(&b, n * 8) != hipSuccess) return 3;
        if (hipMemset(a, 0, n * 8) != hipSuccess || hipMemset(b, 0, n * 8) != hipSuccess) return 3;
        compute_dense_mttkrp(h, mode, F[0], F[1], F[2], a, nullptr, R);
        if (cptc_mttkrp_dense_tiles3(mode, h.d_tiles4, img, size_t(h.num_dense_tiles), nullptr,
                                     nullptr, 0, F[0], F[1], F[2], b, R, int(h.dims[0]),
                                     int(h.dims[1]), int(h.dims[2]), nullptr) != 0) return 4;
        if (hipDeviceSynchronize() != hipSuccess) return 5;
        std::vector<double> ha(n), hb(n);
        if (hipMemcpy(ha.data(), a, n * 8, hipMemcpyDeviceToHost) != hipSuccess) return 3;
        if (hipMemcpy(hb.data(), b, n * 8, hipMemcpyDeviceToHost) != hipSuccess) return 3;
        double num = 0.0, den = 0.0;
        for (size_t x = 0; x < n; ++x)
        {
            num += (ha[x] - hb[x]) * (ha[x] - hb[x]);
            den += hb[x] * hb[x];
        }
        const double rel = std::sqrt(num / (den > 0 ? den : 1.0));
        worst = rel > worst ? rel : worst;
        (void)hipFree(a);
        (void)hipFree(b);
    }
    std::printf("tiles %lld worst %.3e\n", (long long)h.num_dense_tiles, worst);
    free_hybrid_tensor(h);
    free_coo_tensor(t);
    return worst <= 1e-5 ? 0 : 1;
}
'''


@pytest.fixture(scope="module")
def prog(tmp_path_factory):
    d = tmp_path_factory.mktemp("cppapi")
    src = d / "dense_api.cpp"
    src.write_text(PROG)
    exe = d / "dense_api"
    lib = os.path.join(ROOT, "cptc_amd", "lib")
    r = subprocess.run(["g++", "-std=c++17", "-O1", "-D__HIP_PLATFORM_AMD__", "-I",
                        os.path.join(ROOT, "include"), "-I", "/opt/rocm/include", str(src),
                        "-o", str(exe), "-L", lib, "-lcptc", "-L/opt/rocm/lib", "-lamdhip64",
                        f"-Wl,-rpath,{lib}", "-Wl,-rpath,/opt/rocm/lib"],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    return str(exe)


@pytest.mark.parametrize("kern,R", [("bf16x3", 32), ("bf16x3", 100), ("fp32", 32), (None, 48)])
def test_compute_dense_mttkrp_kernels(ca, dev, tmp_path, prog, kern, R):
    t = ca.synth_blocks3(64, 12, 0.1, 0.6, 2e-3, 5)
    path = str(tmp_path / "t.tns")
    ca.write_tns(path, t)
    env = dict(os.environ)
    env.pop("ALS_TILE_KERNEL", None)
    if kern:
        env["ALS_TILE_KERNEL"] = kern
    out = subprocess.run([prog, path, str(R)], env=env, capture_output=True, text=True,
                         timeout=300)
    assert out.returncode == 0, (out.stdout[-2000:], out.stderr[-2000:])
    assert "worst" in out.stdout
    worst = float(out.stdout.split("worst")[1].split()[0])
    if kern == "bf16x3":   # the split kernel ran: it differs from FP32 in the last bits
        assert 0.0 < worst <= 1e-5
    else:                  # None: 12 blocks give few tiles, below the rule's cut -> FP32 kernel
        assert worst <= 1e-14
