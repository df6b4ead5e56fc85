// cptc_opt <tns> [max_iters=20] [R=32] [dense_threshold=0.03]
//
// The reference's CLI (main.cu:22-680) on the MI355X engine: order-3 tensors
// run the hybrid driver, other orders (or ALS_GENERIC_FORCE=1) the generic
// N-order driver; GEN_SELFTEST=1 runs the dense-unit known-answer test.
// Log lines keep the reference's formats ("[ALS] iter k/n time=X ms fit=Y").
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "cptc_hip.h"

namespace {

double now_ms()
{
    return std::chrono::duration<double, std::milli>(
               std::chrono::steady_clock::now().time_since_epoch())
        .count();
}

int fail(const char* what, int rc)
{
    std::fprintf(stderr, "[Error] %s failed (%d): %s\n", what, rc, cptc_last_error());
    return 1;
}

// ALS_EXPORT_FACTORS=<p>: <p>.{0,1,2}.out and <p>.lambda.out (main.cu:595-621)
int export_factors(void* h, const char* prefix, const uint64_t dims[3], int R)
{
    for (int n = 0; n < 3; ++n)
    {
        const std::string path = std::string(prefix) + "." + std::to_string(n) + ".out";
        FILE* fp = std::fopen(path.c_str(), "w");
        if (!fp) return -1;
        std::fprintf(fp, "matrix\n2\n%llu %d\n", (unsigned long long)dims[n], R);
        std::vector<double> f(dims[n] * size_t(R));
        if (cptc_als3_factor(h, n, 1, f.data()) != CPTC_OK)
        {
            std::fclose(fp);
            return -1;
        }
        for (double x : f) std::fprintf(fp, "%.20lf\n", x);
        std::fclose(fp);
    }
    std::vector<double> lam(static_cast<size_t>(R));
    if (cptc_als3_lambda(h, lam.data()) != CPTC_OK) return -1;
    FILE* lf = std::fopen((std::string(prefix) + ".lambda.out").c_str(), "w");
    if (!lf) return -1;
    std::fprintf(lf, "vector\n1\n%d\n", R);
    for (double x : lam) std::fprintf(lf, "%.20lf\n", x);
    std::fclose(lf);
    return 0;
}

// generic.cu:1639-2366 through the C ABI (run_generic_cp's log lines)
int run_generic(const std::string& filename, int order, int max_iters, int R)
{
    std::printf("[Main] order-%d tensor -> generic N-order CP-ALS (pure FP64, MFMA dense units "
                "for the inner modes)\n",
                order);
    cptc_coo coo{};
    const double t0 = now_ms();
    int rc = cptc_tns_load_generic(filename.c_str(), &coo);
    if (rc != CPTC_OK) return fail("load", rc);
    std::printf("[Main] Load time = %g ms | dims = ", now_ms() - t0);
    for (int m = 0; m < coo.nmodes; ++m)
        std::printf("%s%llu", m ? " x " : "", (unsigned long long)coo.dims[m]);
    std::printf(" | NNZ = %llu\n", (unsigned long long)coo.nnz);
    cptc_gen_opts o;
    cptc_gen_default_opts(&o);
    o.R = R;
    o.verbose = 1;
    void* h = nullptr;
    rc = cptc_gen_create(&coo, &o, &h);
    const uint64_t nnz = coo.nnz;
    cptc_coo_free(&coo);
    if (rc != CPTC_OK)
    {
        std::fprintf(stderr, "%s\n", cptc_last_error());
        return 1;
    }
    std::printf("[GEN] N-order CP-ALS: R=%d iters=%d\n", R, max_iters);
    std::vector<double> fit(static_cast<size_t>(max_iters));
    const double t1 = now_ms();
    rc = cptc_gen_run(h, max_iters, fit.data(), nullptr, nullptr, nullptr);
    if (rc != CPTC_OK)
    {
        cptc_gen_destroy(h);
        return fail("ALS", rc);
    }
    if (const char* base = std::getenv("GEN_DUMP"))
    {
        if (cptc_gen_dump(h, base) == CPTC_OK)
            std::printf("[GEN] factors dumped to %s.factors.txt\n", base);
        else
            std::fprintf(stderr, "[GEN] factor dump to %s.factors.txt failed: %s\n", base,
                         cptc_last_error());
    }
    std::printf("[GEN] ALS total = %g ms\n", now_ms() - t1);
    if (o.profile)
    {
        double p[5];
        int it = 0;
        cptc_gen_profile(h, p, &it, 0);
        const double n = it > 0 ? double(it) : 1.0;
        const double tot = p[0] + p[1] + p[2] + p[3] + p[4];
        std::printf("[GEN][profile] avg/iter over %d iters: gram=%g mttkrp=%g solve=%g norm=%g "
                    "fit=%g (sum=%g ms)\n",
                    it, p[0] / n, p[1] / n, p[2] / n, p[3] / n, p[4] / n, tot / n);
        if (tot > 0.0)
            std::printf("[GEN][profile] share: gram=%g%% mttkrp=%g%% solve=%g%% norm=%g%% "
                        "fit=%g%%\n",
                        100.0 * p[0] / tot, 100.0 * p[1] / tot, 100.0 * p[2] / tot,
                        100.0 * p[3] / tot, 100.0 * p[4] / tot);
    }
    double res2 = 0.0, x2 = 0.0;
    rc = cptc_gen_residual(h, &res2, &x2);
    if (rc != CPTC_OK)
    {
        cptc_gen_destroy(h);
        return fail("residual", rc);
    }
    const double res = std::sqrt(std::max(res2, 0.0)), xn = std::sqrt(x2);
    std::printf("[GEN] exact: ||X-Xhat||_F=%g RMSE=%g fit=%g (||X||_F=%g)\n", res,
                nnz ? res / std::sqrt(double(nnz)) : 0.0, xn > 0.0 ? 1.0 - res / xn : 0.0, xn);
    std::vector<double> lam(static_cast<size_t>(R));
    cptc_gen_lambda(h, lam.data());
    std::printf("[GEN] lambda =");
    for (double x : lam) std::printf(" %g", x);
    std::printf("\n");
    cptc_gen_destroy(h);
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
    if (std::getenv("GEN_SELFTEST"))
    {
        int failures = 0;
        const int rc = cptc_gen_selftest(1, &failures);
        if (rc != CPTC_OK) return fail("self-test", rc);
        return failures ? 1 : 0;
    }
    const int order = cptc_tns_probe_nmodes(filename.c_str());
    if (order < 0)
    {
        std::fprintf(stderr, "[Main] cannot determine tensor order of: %s\n", filename.c_str());
        return 1;
    }
    if (order != 3 || std::getenv("ALS_GENERIC_FORCE"))
        return run_generic(filename, order, max_iters, R);

    std::printf("[Main] Loading real tensor dataset from file: %s\n", filename.c_str());
    cptc_coo coo{};
    const double t0 = now_ms();
    int rc = cptc_tns_load3(filename.c_str(), &coo);
    if (rc != CPTC_OK) return fail("load", rc);
    std::printf("%llu non-zero elements.\n", (unsigned long long)coo.nnz);
    std::printf("[Main] Load time = %g ms\n", now_ms() - t0);
    std::printf("[Main] Tensor Dimensions: %llu x %llu x %llu | NNZ: %llu\n",
                (unsigned long long)coo.dims[0], (unsigned long long)coo.dims[1],
                (unsigned long long)coo.dims[2], (unsigned long long)coo.nnz);

    cptc_als3_opts o;
    cptc_als3_default_opts(&o);
    o.R = R;
    o.threshold = threshold;
    o.verbose = 1;
    void* h = nullptr;
    const double t1 = now_ms();
    rc = cptc_als3_create(&coo, &o, &h);
    cptc_coo_free(&coo);
    if (rc != CPTC_OK) return fail("setup", rc);
    std::printf("[Main] setup (CADR + partition + views) = %g ms\n", now_ms() - t1);
    cptc_als3_info info{};
    cptc_als3_info_get(h, &info);
    std::printf("[Main] CUs=%d fill_threshold=%g avg_fill=%g -> %s\n", info.num_cus, info.fill_min,
                info.avg_fill, info.use_mfma ? "MFMA tiles + FP64 residual" : "FP64 only");

    std::printf("[ALS] Starting CP-ALS: rank=%d, max_iters=%d (pseudoinverse solve, per-iter "
                "normalization)\n",
                R, max_iters);
    std::vector<double> fit(static_cast<size_t>(max_iters));
    std::vector<float> ms(static_cast<size_t>(max_iters)), mt(static_cast<size_t>(max_iters));
    rc = cptc_als3_run(h, max_iters, fit.data(), ms.data(), mt.data());
    if (rc != CPTC_OK) return fail("ALS", rc);
    double res_sq = 0.0, x_sq = 0.0;
    rc = cptc_als3_residual(h, &res_sq, &x_sq);
    if (rc != CPTC_OK) return fail("residual", rc);
    const double rmse = info.nnz ? std::sqrt(std::max(res_sq, 0.0) / double(info.nnz)) : 0.0;
    const double xn = std::sqrt(x_sq);
    double efit = xn > 1e-300 ? 1.0 - std::sqrt(std::max(res_sq, 0.0)) / xn : 0.0;
    if (efit < 0.0 && efit > -1e-10) efit = 0.0;
    if (efit > 1.0 && efit < 1.0 + 1e-10) efit = 1.0;
    std::printf("[Fit] ||X||_F = %g ||X-Xhat||_F = %g RMSE = %g fit = %g\n", xn,
                std::sqrt(std::max(res_sq, 0.0)), rmse, efit);
    std::printf("\n[Fit Report] final R=%d RMSE=%g fit=%g (%g%% Frobenius energy explained)\n\n", R,
                rmse, efit, efit * 100.0);
    std::printf("[ALS] Final RMSE=%g\n", rmse);
    std::vector<double> lam(static_cast<size_t>(R));
    cptc_als3_lambda(h, lam.data());
    std::printf("[Main] Final CP weights:");
    for (double x : lam) std::printf(" %g", x);
    std::printf("\n");
    if (const char* exp = std::getenv("ALS_EXPORT_FACTORS"))
    {
        if (export_factors(h, exp, info.dims, R) != 0)
            std::fprintf(stderr, "[Main] factor export to %s failed\n", exp);
        else
            std::printf("[Main] factors exported to %s\n", exp);
    }
    cptc_als3_destroy(h);
    std::printf("[Main] Real tensor execution complete with CADR Reordering & Unpermutation!\n");
    return 0;
}
