// cptc_opt <tns> [max_iters=20] [R=32] [dense_threshold=0.03]
//
// The reference's CLI (main.cu:22-680) written against this library's C++
// interface (include/*.hpp, the reference's function names): order-3
// tensors run load -> CADR -> factor init -> hybrid partition -> views ->
// fill-rate path selection -> execute_als_decomposition -> unpermute ->
// export; other orders (or ALS_GENERIC_FORCE=1) run the generic N-order
// driver; GEN_SELFTEST=1 runs the dense-unit known-answer test.  Log lines
// keep the reference's formats ("[ALS] iter k/n time=X ms fit=Y").
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "als.hpp"
#include "cadr.hpp"
#include "common.hpp"
#include "cptc_hip.h"
#include "generic.hpp"
#include "partition.hpp"
#include "sgd.hpp"
#include "tensor.hpp"

namespace {

double now_ms()
{
    return std::chrono::duration<double, std::milli>(
               std::chrono::steady_clock::now().time_since_epoch())
        .count();
}

// ALS_EXPORT_FACTORS=<p>: <p>.{0,1,2}.out and <p>.lambda.out (main.cu:595-621)
int export_factors(const char* prefix, double* const d_orig[3], const size_t dims[3],
                   const std::vector<double>& lam, int R)
{
    for (int n = 0; n < 3; ++n)
    {
        const std::string path = std::string(prefix) + "." + std::to_string(n) + ".out";
        FILE* fp = std::fopen(path.c_str(), "w");
        if (!fp) return -1;
        std::fprintf(fp, "matrix\n2\n%zu %d\n", dims[n], R);
        std::vector<double> f(dims[n] * size_t(R));
        CHECK_HIP(hipMemcpy(f.data(), d_orig[n], f.size() * sizeof(double), hipMemcpyDeviceToHost));
        for (double x : f) std::fprintf(fp, "%.20lf\n", x);
        std::fclose(fp);
    }
    FILE* lf = std::fopen((std::string(prefix) + ".lambda.out").c_str(), "w");
    if (!lf) return -1;
    std::fprintf(lf, "vector\n1\n%d\n", R);
    for (double x : lam) std::fprintf(lf, "%.20lf\n", x);
    std::fclose(lf);
    return 0;
}

int run_order3(const std::string& filename, int max_iters, int R, double threshold)
{
    std::printf("[Main] Loading real tensor dataset from file: %s\n", filename.c_str());
    COOTensor tensor;
    double t0 = now_ms();
    load_tns_file(filename, tensor);
    std::printf("%zu non-zero elements.\n", tensor.nnz);
    std::printf("[Main] Load time = %g ms\n", now_ms() - t0);
    std::printf("[Main] Tensor Dimensions: %zu x %zu x %zu | NNZ: %zu\n", tensor.dims[0],
                tensor.dims[1], tensor.dims[2], tensor.nnz);

    // CADR (main.cu:176-192)
    t0 = now_ms();
    TensorPermutation perm = compute_cadr_reordering(tensor);
    apply_cadr_reordering(tensor, perm);
    std::printf("[CADR] Total reordering time = %g ms\n", now_ms() - t0);

    // factors in the relabelled space (main.cu:228-264)
    double* d_factors_perm[3] = {nullptr, nullptr, nullptr};
    for (int m = 0; m < 3; ++m)
        CHECK_HIP(hipMalloc(&d_factors_perm[m], tensor.dims[m] * size_t(R) * sizeof(double)));
    init_factors_random(d_factors_perm, tensor.dims, R);

    // hybrid partition + row-sorted views (main.cu:268-314)
    HybridCOOTensor hybrid, hybrid_dense;
    t0 = now_ms();
    create_hybrid_format(tensor, hybrid, threshold);
    std::printf("[Main] Hybrid partition time = %g ms\n", now_ms() - t0);
    t0 = now_ms();
    build_mttkrp_views(hybrid, nullptr);
    CHECK_HIP(hipDeviceSynchronize());
    std::printf("[Main] MTTKRP views build time = %g ms\n", now_ms() - t0);

    // fill-rate path selection (main.cu:334-426); the SM scaling becomes a
    // CU scaling: fill_min = 0.11 / sqrt(CUs / 24), floored at 0.08
    const double avg_fill =
        hybrid.num_dense_tiles > 0
            ? double(hybrid.dense_nnz) / (double(hybrid.num_dense_tiles) * 4096.0)
            : 0.0;
    double fill_min = 0.08;
    if (const char* fm = std::getenv("ALS_FILL_MIN"))
        fill_min = std::atof(fm);
    else
    {
        int dev = 0;
        CHECK_HIP(hipGetDevice(&dev));
        hipDeviceProp_t prop{};
        CHECK_HIP(hipGetDeviceProperties(&prop, dev));
        fill_min = std::max(0.08, 0.11 / std::sqrt(double(prop.multiProcessorCount) / 24.0));
        std::printf("[Main] device=%s CUs=%d fill_min=%g\n", prop.name, prop.multiProcessorCount,
                    fill_min);
    }
    bool use_mfma = avg_fill >= fill_min;
    if (std::getenv("ALS_FORCE_WMMA"))
        use_mfma = true;
    else if (std::getenv("ALS_FORCE_CUDA"))
        use_mfma = false;
    std::printf("[Main] density check: dense_nnz=%zu sparse_nnz=%zu tiles=%d avg_fill=%g "
                "(threshold %g) -> %s\n",
                hybrid.dense_nnz, hybrid.sparse_nnz, hybrid.num_dense_tiles, avg_fill, fill_min,
                use_mfma ? "MFMA tiles + FP64 residual" : "FP64 only");
    if (!use_mfma && hybrid.num_dense_tiles > 0)
        build_dense_mttkrp_views(hybrid, hybrid_dense, nullptr);

    double* d_lambda = nullptr;
    CHECK_HIP(hipMalloc(&d_lambda, size_t(R) * sizeof(double)));
    CHECK_HIP(hipMemset(d_lambda, 0, size_t(R) * sizeof(double)));
    if (std::getenv("ALS_SGD"))
    {
        // main.cu:466-501: lambda starts at 1; learning rate ALS_SGD_GAMMA
        // (1e-9), batch ALS_SGD_BATCH (2^20), seed 42
        const std::vector<double> ones(static_cast<size_t>(R), 1.0);
        CHECK_HIP(hipMemcpy(d_lambda, ones.data(), ones.size() * sizeof(double),
                            hipMemcpyHostToDevice));
        const char* g = std::getenv("ALS_SGD_GAMMA");
        const char* b = std::getenv("ALS_SGD_BATCH");
        execute_sgd_decomposition(hybrid, d_factors_perm[0], d_factors_perm[1],
                                  d_factors_perm[2], d_lambda, R, max_iters,
                                  g ? std::atof(g) : 1e-9, b ? std::atoi(b) : (1 << 20), 42);
    }
    else
        execute_als_decomposition(tensor, hybrid, hybrid_dense, d_factors_perm[0],
                                  d_factors_perm[1], d_factors_perm[2], d_lambda, R, max_iters,
                                  1e-4);

    // back to the input's index order (main.cu:525-545)
    double* d_factors_orig[3] = {nullptr, nullptr, nullptr};
    for (int m = 0; m < 3; ++m)
        CHECK_HIP(hipMalloc(&d_factors_orig[m], tensor.dims[m] * size_t(R) * sizeof(double)));
    unpermute_factor_matrices(d_factors_perm[0], d_factors_perm[1], d_factors_perm[2],
                              d_factors_orig, perm, tensor.dims, R);
    std::vector<double> lam(static_cast<size_t>(R));
    CHECK_HIP(hipMemcpy(lam.data(), d_lambda, size_t(R) * sizeof(double), hipMemcpyDeviceToHost));
    std::printf("[Main] Final CP weights:");
    for (double x : lam) std::printf(" %g", x);
    std::printf("\n");
    if (const char* exp = std::getenv("ALS_EXPORT_FACTORS"))
    {
        if (export_factors(exp, d_factors_orig, tensor.dims, lam, R) != 0)
            std::fprintf(stderr, "[Main] factor export to %s failed\n", exp);
        else
            std::printf("[Main] factors exported to %s\n", exp);
    }

    free_cadr_permutation(perm);
    free_hybrid_format(hybrid);
    free_hybrid_format(hybrid_dense);
    for (int m = 0; m < 3; ++m)
    {
        CHECK_HIP(hipFree(d_factors_perm[m]));
        CHECK_HIP(hipFree(d_factors_orig[m]));
    }
    CHECK_HIP(hipFree(d_lambda));
    free_coo_tensor(tensor);
    std::printf("[Main] Real tensor execution complete with CADR Reordering & Unpermutation!\n");
    return 0;
}

}  // namespace

int main(int argc, char** argv)
{
    int R = 32, max_iters = 20;
    double threshold = 0.03;
    std::string filename = "nell-2.tns";
    if (argc > 1) filename = argv[1];
    if (argc > 2) max_iters = std::atoi(argv[2]);
    if (argc > 3) R = std::atoi(argv[3]);
    if (argc > 4) threshold = std::atof(argv[4]);
    if (max_iters <= 0) max_iters = 1;
    if (R <= 0) R = 1;

    if (cptc_device_count() <= 0)
    {
        std::fprintf(stderr, "[Error] No HIP devices found!\n");
        return 1;
    }
    debug_device_state();
    if (std::getenv("GEN_SELFTEST")) return run_dense_selftest();

    const int order = probe_tns_nmodes(filename.c_str());
    if (order < 0)
    {
        std::fprintf(stderr, "[Main] cannot determine tensor order of: %s\n", filename.c_str());
        return 1;
    }
    if (order != 3 || std::getenv("ALS_GENERIC_FORCE"))
    {
        std::printf("[Main] order-%d tensor -> generic N-order CP-ALS (pure FP64, MFMA dense "
                    "units for the inner modes)\n",
                    order);
        GTensor gt;
        double load_ms = 0.0;
        if (!load_tns_generic(filename.c_str(), gt, &load_ms)) return 1;
        std::printf("[Main] Load time = %g ms | dims = ", load_ms);
        for (int m = 0; m < gt.nmodes; ++m) std::printf("%s%zu", m ? " x " : "", gt.dims[size_t(m)]);
        std::printf(" | NNZ = %zu\n", gt.nnz);
        const unsigned seed =
            std::getenv("GEN_SEED") ? unsigned(std::atoi(std::getenv("GEN_SEED"))) : 42u;
        return run_generic_cp(gt, max_iters, R, seed) == 0 ? 0 : 1;
    }
    return run_order3(filename, max_iters, R, threshold);
}
