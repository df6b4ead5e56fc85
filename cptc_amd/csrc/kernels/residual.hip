// Exact residual ||X - Xhat||^2 and ||X||^2 over row-sorted views and dense
// tile pools, plus the factor unpermutation of the export path.
//
// The model value of an element follows common.cu:303-334: two accumulators
// over even / odd ranks, each term (a*b*c)*lambda_r, pred = p0 + p1.
// Per-workgroup partials are summed in a fixed order (deterministic).
#include <hip/hip_runtime.h>

#include "../host/hip_util.hpp"

namespace {

constexpr int THREADS = 256;

__device__ double model_value(const double* __restrict__ pa, const double* __restrict__ pb,
                              const double* __restrict__ pc, const double* __restrict__ lam, int R)
{
    double p0 = 0.0, p1 = 0.0;
    int r = 0;
    for (; r + 1 < R; r += 2)
    {
        double x0 = pa[r] * pb[r] * pc[r];
        double x1 = pa[r + 1] * pb[r + 1] * pc[r + 1];
        if (lam)
        {
            x0 *= lam[r];
            x1 *= lam[r + 1];
        }
        p0 += x0;
        p1 += x1;
    }
    for (; r < R; ++r)
    {
        double x = pa[r] * pb[r] * pc[r];
        if (lam) x *= lam[r];
        p0 += x;
    }
    return p0 + p1;
}

__device__ void block_sum2(double a, double b, double* __restrict__ out2)
{
    __shared__ double ra[THREADS], rb[THREADS];
    ra[threadIdx.x] = a;
    rb[threadIdx.x] = b;
    __syncthreads();
    for (int off = THREADS / 2; off > 0; off >>= 1)
    {
        if (int(threadIdx.x) < off)
        {
            ra[threadIdx.x] += ra[threadIdx.x + off];
            rb[threadIdx.x] += rb[threadIdx.x + off];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0)
    {
        out2[0] = ra[0];
        out2[1] = rb[0];
    }
}

__global__ __launch_bounds__(THREADS) void residual_view_kernel(
    const uint64_t* __restrict__ coords, const double* __restrict__ vals, size_t nnz,
    const double* __restrict__ A, const double* __restrict__ B, const double* __restrict__ C,
    const double* __restrict__ lam, int R, double* __restrict__ part)
{
    double res = 0.0, xx = 0.0;
    const size_t stride = size_t(gridDim.x) * THREADS;
    for (size_t e = size_t(blockIdx.x) * THREADS + threadIdx.x; e < nnz; e += stride)
    {
        const uint64_t pc = coords[e];
        const double v = vals[e];
        const uint32_t i = uint32_t(pc >> 30) & 0x7FFFu, j = uint32_t(pc >> 15) & 0x7FFFu,
                       k = uint32_t(pc) & 0x7FFFu;
        const double d =
            v - model_value(A + size_t(i) * R, B + size_t(j) * R, C + size_t(k) * R, lam, R);
        res += d * d;
        xx += v * v;
    }
    block_sum2(res, xx, part + 2 * size_t(blockIdx.x));
}

__global__ __launch_bounds__(THREADS) void residual_tiles_kernel(
    const int32_t* __restrict__ tiles4, const uint64_t* __restrict__ off,
    const int32_t* __restrict__ lid, const double* __restrict__ pval, size_t ntiles,
    const double* __restrict__ A, const double* __restrict__ B, const double* __restrict__ C,
    const double* __restrict__ lam, int R, double* __restrict__ part)
{
    double res = 0.0, xx = 0.0;
    for (size_t t = blockIdx.x; t < ntiles; t += gridDim.x)
    {
        const int b0 = tiles4[4 * t] * 16, b1 = tiles4[4 * t + 1] * 16, b2 = tiles4[4 * t + 2] * 16;
        for (uint64_t e = off[t] + threadIdx.x; e < off[t + 1]; e += THREADS)
        {
            const int l = lid[e];
            const double v = pval[e];
            const size_t i = size_t(b0 + (l >> 8)), j = size_t(b1 + ((l >> 4) & 15)),
                         k = size_t(b2 + (l & 15));
            const double d = v - model_value(A + i * R, B + j * R, C + k * R, lam, R);
            res += d * d;
            xx += v * v;
        }
    }
    block_sum2(res, xx, part + 2 * size_t(blockIdx.x));
}

__global__ void finalize_add_kernel(const double* __restrict__ part, int P,
                                    double* __restrict__ out2)
{
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    double a = 0.0, b = 0.0;
    for (int p = 0; p < P; ++p)
    {
        a += part[2 * p];
        b += part[2 * p + 1];
    }
    out2[0] += a;
    out2[1] += b;
}

__global__ void unpermute_kernel(const double* __restrict__ src, double* __restrict__ dst,
                                 const int32_t* __restrict__ perm, size_t dim, int R)
{
    const size_t total = dim * size_t(R);
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    for (size_t x = size_t(blockIdx.x) * blockDim.x + threadIdx.x; x < total; x += stride)
    {
        const size_t old = x / size_t(R);
        const int r = int(x % size_t(R));
        dst[x] = src[size_t(perm[old]) * R + r];
    }
}

}  // namespace

extern "C" int cptc_residual3_view(const uint64_t* d_coords, const double* d_vals, size_t nnz,
                                   const double* d_A, const double* d_B, const double* d_C,
                                   const double* d_lambda, int R, double* d_out2, void* stream)
{
    CPTC_REQUIRE(R >= 1 && d_A && d_B && d_C && d_out2, CPTC_ERR_ARG,
                 "cptc_residual3_view: bad arguments");
    if (nnz == 0) return CPTC_OK;
    CPTC_REQUIRE(d_coords && d_vals, CPTC_ERR_ARG, "cptc_residual3_view: null view");
    hipStream_t s = cptc::as_stream(stream);
    const int P = int(cptc::grid_for(nnz, THREADS * 8, 2048));
    void* buf = nullptr;
    CPTC_TRY(cptc::scratch_get(cptc::SCR_REDUCE, size_t(P) * 2 * sizeof(double), &buf));
    double* part = static_cast<double*>(buf);
    hipLaunchKernelGGL(residual_view_kernel, dim3(P), dim3(THREADS), 0, s, d_coords, d_vals, nnz,
                       d_A, d_B, d_C, d_lambda, R, part);
    CPTC_LAUNCHED();
    hipLaunchKernelGGL(finalize_add_kernel, dim3(1), dim3(64), 0, s, part, P, d_out2);
    CPTC_LAUNCHED();
    return CPTC_OK;
}

extern "C" int cptc_residual3_tiles(const int32_t* d_tiles, const uint64_t* d_pool_off,
                                    const int32_t* d_pool_lid, const double* d_pool_val,
                                    size_t ntiles, const double* d_A, const double* d_B,
                                    const double* d_C, const double* d_lambda, int R,
                                    double* d_out2, void* stream)
{
    CPTC_REQUIRE(R >= 1 && d_A && d_B && d_C && d_out2, CPTC_ERR_ARG,
                 "cptc_residual3_tiles: bad arguments");
    if (ntiles == 0) return CPTC_OK;
    CPTC_REQUIRE(d_tiles && d_pool_off && d_pool_lid && d_pool_val, CPTC_ERR_ARG,
                 "cptc_residual3_tiles: null pool");
    hipStream_t s = cptc::as_stream(stream);
    const int P = int(ntiles < 2048 ? ntiles : 2048);
    void* buf = nullptr;
    CPTC_TRY(cptc::scratch_get(cptc::SCR_REDUCE, size_t(P) * 2 * sizeof(double), &buf));
    double* part = static_cast<double*>(buf);
    hipLaunchKernelGGL(residual_tiles_kernel, dim3(P), dim3(THREADS), 0, s, d_tiles, d_pool_off,
                       d_pool_lid, d_pool_val, ntiles, d_A, d_B, d_C, d_lambda, R, part);
    CPTC_LAUNCHED();
    hipLaunchKernelGGL(finalize_add_kernel, dim3(1), dim3(64), 0, s, part, P, d_out2);
    CPTC_LAUNCHED();
    return CPTC_OK;
}

extern "C" int cptc_unpermute_factor(const double* d_perm_factor, double* d_orig,
                                     const int32_t* d_perm, size_t dim, int R, void* stream)
{
    CPTC_REQUIRE(R >= 1 && d_perm_factor && d_orig && d_perm, CPTC_ERR_ARG,
                 "cptc_unpermute_factor: bad arguments");
    if (dim == 0) return CPTC_OK;
    hipLaunchKernelGGL(unpermute_kernel, dim3(cptc::grid_for(dim * size_t(R), 256, 4096)),
                       dim3(256), 0, cptc::as_stream(stream), d_perm_factor, d_orig, d_perm, dim,
                       R);
    CPTC_LAUNCHED();
    return CPTC_OK;
}
