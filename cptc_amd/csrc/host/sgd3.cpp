// CP-SGD driver loop (sgd.cu:302-467; routed by ALS_SGD at main.cu:467-501):
// the kernels are in kernels/sgd3.hip.  One host thread, one stream; the
// batch index buffer and the loss scalar are allocated per call.
#include <hip/hip_runtime_api.h>

#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>

#include "cptc_hip.h"
#include "hip_util.hpp"

extern "C" int cptc_sgd3_run(const uint64_t* d_coords, const double* d_vals, uint64_t nnz,
                             double* d_A, double* d_B, double* d_C, const uint64_t* dims,
                             double* d_lambda, int R, int iters, double gamma, uint32_t batch,
                             uint64_t seed, int verbose, double* batch_rmse, void* stream)
{
    CPTC_REQUIRE(nnz >= 1 && nnz <= 0x7FFFFFFFull && d_coords && d_vals, CPTC_ERR_STATE,
                 "[SGD] sparse views not ready.");
    CPTC_REQUIRE(d_A && d_B && d_C && dims && d_lambda && R >= 1 && R <= 128 && iters >= 0 &&
                     batch >= 1,
                 CPTC_ERR_ARG, "cptc_sgd3_run: bad arguments (R %d, iters %d, batch %u)", R,
                 iters, batch);
    hipStream_t s = cptc::as_stream(stream);
    uint32_t* d_idx = nullptr;
    double* d_loss = nullptr;
    CPTC_HIP(hipMalloc(&d_idx, size_t(batch) * sizeof(uint32_t)));
    if (hipMalloc(&d_loss, sizeof(double)) != hipSuccess)
    {
        (void)hipFree(d_idx);
        CPTC_REQUIRE(false, CPTC_ERR_HIP, "cptc_sgd3_run: hipMalloc failed");
    }
    struct Free
    {
        void* a;
        void* b;
        ~Free()
        {
            (void)hipFree(a);
            (void)hipFree(b);
        }
    } fr{d_idx, d_loss};
    double* F[3] = {d_A, d_B, d_C};
    if (verbose)
        std::printf("[SGD] CP-SGD start: R=%d batch=%u gamma=%g iters=%d sparse_nnz=%llu\n", R,
                    batch, gamma, iters, (unsigned long long)nnz);
    const auto t0 = std::chrono::steady_clock::now();
    for (int it = 0; it < iters; ++it)
    {
        CPTC_TRY(cptc_sgd3_sample(d_idx, batch, nnz, seed + uint64_t(it), s));
        if (verbose && it == 0)
        {
            // the reference's unconditional first-iteration lines (sgd.cu:371-380, 394-398)
            uint32_t hi[4] = {0, 0, 0, 0};
            double ha[4] = {0, 0, 0, 0}, hl[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            const int n4 = batch < 4 ? int(batch) : 4;
            CPTC_HIP(hipMemcpyAsync(hi, d_idx, size_t(n4) * sizeof(uint32_t),
                                    hipMemcpyDeviceToHost, s));
            CPTC_HIP(hipMemcpyAsync(ha, d_A, size_t(R < 4 ? R : 4) * sizeof(double),
                                    hipMemcpyDeviceToHost, s));
            CPTC_HIP(hipMemcpyAsync(hl, d_lambda, size_t(R < 4 ? R : 4) * sizeof(double),
                                    hipMemcpyDeviceToHost, s));
            CPTC_HIP(hipStreamSynchronize(s));
            std::printf("[SGD-DBG] sample[0..3] = %u %u %u %u\n", hi[0], hi[1], hi[2], hi[3]);
            std::printf("[SGD-DBG] before: A[0..3]=%.3e %.3e %.3e %.3e  lam[0..3]=%.3e %.3e %.3e "
                        "%.3e\n",
                        ha[0], ha[1], ha[2], ha[3], hl[0], hl[1], hl[2], hl[3]);
        }
        CPTC_TRY(cptc_sgd3_update(d_coords, d_vals, d_idx, batch, d_A, d_B, d_C, d_lambda, R,
                                  gamma, s));
        if (verbose && it == 0)
        {
            double hl[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            CPTC_HIP(hipMemcpyAsync(hl, d_lambda, size_t(R < 8 ? R : 8) * sizeof(double),
                                    hipMemcpyDeviceToHost, s));
            CPTC_HIP(hipStreamSynchronize(s));
            std::printf("[SGD-DBG] after update lam[0..7]=%.3e %.3e %.3e %.3e %.3e %.3e %.3e "
                        "%.3e\n",
                        hl[0], hl[1], hl[2], hl[3], hl[4], hl[5], hl[6], hl[7]);
        }
        // every fifth iteration: A, then B, then C normalised, lambda = norms
        if (it % 5 == 0)
            for (int m = 0; m < 3; ++m) CPTC_TRY(cptc_sgd3_normalize(F[m], dims[m], R, d_lambda, s));
        if (verbose && it == 0 && std::getenv("ALS_SGD_DBG"))
        {
            double ha[2] = {0, 0}, hl[2] = {0, 0};
            CPTC_HIP(hipMemcpyAsync(ha, d_A, size_t(R < 2 ? R : 2) * sizeof(double),
                                    hipMemcpyDeviceToHost, s));
            CPTC_HIP(hipMemcpyAsync(hl, d_lambda, size_t(R < 2 ? R : 2) * sizeof(double),
                                    hipMemcpyDeviceToHost, s));
            CPTC_HIP(hipStreamSynchronize(s));
            std::printf("[SGD-DBG] it=%d A0=%.3e A1=%.3e lam0=%.3e lam1=%.3e\n", it, ha[0], ha[1],
                        hl[0], hl[1]);
        }
        if (batch_rmse) batch_rmse[it] = -1.0;
        if (it % 10 == 0 || it == iters - 1)
        {
            CPTC_TRY(cptc_sgd3_loss(d_coords, d_vals, d_idx, batch, d_A, d_B, d_C, d_lambda, R,
                                    d_loss, s));
            double loss = 0.0;
            CPTC_HIP(hipMemcpyAsync(&loss, d_loss, sizeof(double), hipMemcpyDeviceToHost, s));
            CPTC_HIP(hipStreamSynchronize(s));
            const double rmse = std::sqrt(loss / double(batch));
            if (batch_rmse) batch_rmse[it] = rmse;
            if (verbose) std::printf("[SGD] iter %d batch-rmse=%g\n", it, rmse);
        }
    }
    CPTC_HIP(hipStreamSynchronize(s));
    if (verbose)
        std::printf("[SGD] done in %g ms\n",
                    std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0)
                        .count());
    return CPTC_OK;
}
