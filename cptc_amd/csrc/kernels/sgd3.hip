// CP-SGD on the order-3 sparse residual (sgd.cu:51-288, the reference's
// experimental ALS_SGD path): per iteration a batch of residual elements is
// drawn with a counter-based hash, every drawn element (i, j, k, v) updates
// its three factor rows by one stochastic-gradient step, and every fifth
// iteration the factors are column-normalised with lambda reset to the
// norms.
//
// Semantics kept from the reference:
//   * sample b of iteration `it`: x = (seed + it) + b * 0x9E3779B97F4A7C15,
//     then the SplitMix64 finaliser (xor-shift 30 / multiply / 27 / multiply
//     / 31), index = x mod nnz — over the mode-0 residual view
//     (sgd.cu:195-215);
//   * xhat = sum_r lambda_r a_r b_r c_r, e = v - xhat, then
//     A[i, r] += g e b_r c_r, B[j, r] += g e a_r c_r, C[k, r] += g e a_r b_r
//     with a, b, c the values the element read: the elements of a batch run
//     concurrently and add their steps atomically (asynchronous SGD, as the
//     reference), so elements that share a row see each other's steps in
//     whatever order the hardware runs them;
//   * lambda is not stepped; normalisation sets F[:, r] /= n_r (0 when
//     n_r < 1e-14) and lambda_r = n_r (0 when n_r < 1e-14) for A, then B,
//     then C, so lambda ends as C's column norms (sgd.cu:225-288, 401-417);
//   * the batch loss is sum_b (v - xhat)^2 over the same sample.
//
// MI355X mapping: one wave64 carries 64 / RT elements (RT = the rank tile,
// 8..64; R > 64 loops over 64-rank blocks in the lane), a lane owns one rank
// of its element; xhat is a sum over the element's lanes by xor-shuffles in
// a fixed order.  The reference runs one 32-lane warp per element and
// supports R = 32 only (its lanes index ranks directly); any R works here.
// The loss is reduced deterministically (per-workgroup partials, then one
// ordered sum) instead of one atomic per element.
#include <hip/hip_runtime.h>

#include "../host/hip_util.hpp"

namespace {

constexpr int WAVE = 64;
constexpr int SGD_T = 256;

__device__ __forceinline__ uint32_t sample_index(uint64_t seed, uint32_t b, uint32_t nnz)
{
    uint64_t x = seed + uint64_t(b) * 0x9E3779B97F4A7C15ull;
    x ^= x >> 30;
    x *= 0xBF58476D1CE4E5B9ull;
    x ^= x >> 27;
    x *= 0x94D049BB133111EBull;
    x ^= x >> 31;
    return uint32_t(x % uint64_t(nnz));
}

__global__ __launch_bounds__(SGD_T) void sgd_sample_kernel(uint32_t* __restrict__ idx,
                                                           uint32_t batch, uint32_t nnz,
                                                           uint64_t seed)
{
    const uint32_t b = blockIdx.x * SGD_T + threadIdx.x;
    if (b < batch) idx[b] = sample_index(seed, b, nnz);
}

// Element slot of this lane: EPW = 64 / LPE slots per wave, LPE lanes per
// element (a power of two >= the rank tile).  Ranks r = lane_in_slot,
// lane_in_slot + LPE, ... < R.
template <int LPE>
__device__ __forceinline__ double slot_sum(double x)
{
#pragma unroll
    for (int o = 1; o < LPE; o <<= 1) x += __shfl_xor(x, o, WAVE);
    return x;
}

template <int LPE, bool UPDATE>
__global__ __launch_bounds__(SGD_T) void sgd_kernel(
    const uint64_t* __restrict__ coords, const double* __restrict__ vals,
    const uint32_t* __restrict__ idx, uint32_t batch, double* A, double* B, double* C,
    const double* __restrict__ lambda, int R, double gamma, double* __restrict__ loss_part)
{
    constexpr int EPW = WAVE / LPE;
    // ranks per lane: LPE < 64 means R <= LPE (one rank), else R <= 128 (two)
    constexpr int NR = (LPE < WAVE) ? 1 : 2;
    const int lane = threadIdx.x & (WAVE - 1);
    const int sl = lane % LPE;
    const uint32_t b = (blockIdx.x * (SGD_T / WAVE) + threadIdx.x / WAVE) * EPW + lane / LPE;
    const bool live = b < batch;
    double e2 = 0.0;
    if (live)
    {
        const uint32_t el = idx[b];
        const uint64_t pc = coords[el];
        const double v = vals[el];
        const uint32_t i = uint32_t(pc >> 30) & 0x7FFFu;
        const uint32_t j = uint32_t(pc >> 15) & 0x7FFFu;
        const uint32_t k = uint32_t(pc) & 0x7FFFu;
        double* pa = A + size_t(i) * R;
        double* pb = B + size_t(j) * R;
        double* pcp = C + size_t(k) * R;
        double a[NR], bb[NR], c[NR];
        double xh = 0.0;
#pragma unroll
        for (int q = 0; q < NR; ++q)
        {
            const int r = sl + q * LPE;
            a[q] = bb[q] = c[q] = 0.0;
            if (r < R)
            {
                a[q] = pa[r];
                bb[q] = pb[r];
                c[q] = pcp[r];
                xh += lambda[r] * a[q] * bb[q] * c[q];
            }
        }
        xh = slot_sum<LPE>(xh);
        const double e = v - xh;
        if constexpr (UPDATE)
        {
            const double ge = gamma * e;
#pragma unroll
            for (int q = 0; q < NR; ++q)
            {
                const int r = sl + q * LPE;
                if (r < R)
                {
                    atomicAdd(pa + r, ge * bb[q] * c[q]);
                    atomicAdd(pb + r, ge * a[q] * c[q]);
                    atomicAdd(pcp + r, ge * a[q] * bb[q]);
                }
            }
        }
        else if (sl == 0)
            e2 = e * e;
    }
    if constexpr (!UPDATE)
    {
        // per-workgroup partial: lanes in order, then waves in order
        __shared__ double red[SGD_T / WAVE];
#pragma unroll
        for (int o = WAVE / 2; o >= 1; o >>= 1) e2 += __shfl_xor(e2, o, WAVE);
        if (lane == 0) red[threadIdx.x / WAVE] = e2;
        __syncthreads();
        if (threadIdx.x == 0)
        {
            double t = 0.0;
            for (int w = 0; w < SGD_T / WAVE; ++w) t += red[w];
            loss_part[blockIdx.x] = t;
        }
    }
}

__global__ __launch_bounds__(SGD_T) void sum_parts_kernel(const double* __restrict__ part, int P,
                                                          double* __restrict__ out)
{
    __shared__ double red[SGD_T];
    double t = 0.0;
    for (int p = threadIdx.x; p < P; p += SGD_T) t += part[p];
    red[threadIdx.x] = t;
    __syncthreads();
    if (threadIdx.x == 0)
    {
        double s = 0.0;
        for (int x = 0; x < SGD_T; ++x) s += red[x];
        *out = s;
    }
}

// F[:, r] /= n_r (0 when n_r < 1e-14); lambda_r = n_r (0 when n_r < 1e-14)
__global__ __launch_bounds__(SGD_T) void sgd_normalize_kernel(double* __restrict__ F, size_t rows,
                                                              int R,
                                                              const double* __restrict__ norms,
                                                              double* __restrict__ lambda)
{
    const size_t n = rows * size_t(R);
    const size_t stride = size_t(gridDim.x) * SGD_T;
    for (size_t x = size_t(blockIdx.x) * SGD_T + threadIdx.x; x < n; x += stride)
    {
        const double nr = norms[x % size_t(R)];
        F[x] = nr < 1e-14 ? 0.0 : F[x] / nr;
    }
    if (blockIdx.x == 0)
        for (int r = threadIdx.x; r < R; r += SGD_T) lambda[r] = norms[r] < 1e-14 ? 0.0 : norms[r];
}

template <bool UPDATE>
int sgd_launch(const uint64_t* coords, const double* vals, const uint32_t* idx, uint32_t batch,
               double* A, double* B, double* C, const double* lambda, int R, double gamma,
               double* part, hipStream_t s, unsigned* blocks_out)
{
    // LPE: the smallest power of two >= min(R, 64) (lanes per element)
    int lpe = 8;
    while (lpe < R && lpe < WAVE) lpe <<= 1;
    const unsigned epb = unsigned((SGD_T / WAVE) * (WAVE / lpe));   // elements per workgroup
    const unsigned blocks = unsigned((uint64_t(batch) + epb - 1) / epb);
    if (blocks_out) *blocks_out = blocks;
#define CPTC_SGD_LAUNCH(L)                                                                     \
    hipLaunchKernelGGL((sgd_kernel<L, UPDATE>), dim3(blocks), dim3(SGD_T), 0, s, coords, vals, \
                       idx, batch, A, B, C, lambda, R, gamma, part)
    switch (lpe)
    {
    case 8: CPTC_SGD_LAUNCH(8); break;
    case 16: CPTC_SGD_LAUNCH(16); break;
    case 32: CPTC_SGD_LAUNCH(32); break;
    default: CPTC_SGD_LAUNCH(64); break;
    }
#undef CPTC_SGD_LAUNCH
    CPTC_LAUNCHED();
    return CPTC_OK;
}

}  // namespace

extern "C" int cptc_sgd3_sample(uint32_t* d_idx, uint32_t batch, uint64_t nnz, uint64_t seed,
                                void* stream)
{
    CPTC_REQUIRE(nnz >= 1 && nnz <= 0xFFFFFFFFull && (batch == 0 || d_idx), CPTC_ERR_ARG,
                 "cptc_sgd3_sample: bad arguments (nnz %llu)", (unsigned long long)nnz);
    if (batch == 0) return CPTC_OK;
    hipLaunchKernelGGL(sgd_sample_kernel, dim3((batch + SGD_T - 1) / SGD_T), dim3(SGD_T), 0,
                       cptc::as_stream(stream), d_idx, batch, uint32_t(nnz), seed);
    CPTC_LAUNCHED();
    return CPTC_OK;
}

extern "C" int cptc_sgd3_update(const uint64_t* d_coords, const double* d_vals,
                                const uint32_t* d_idx, uint32_t batch, double* d_A, double* d_B,
                                double* d_C, const double* d_lambda, int R, double gamma,
                                void* stream)
{
    CPTC_REQUIRE(R >= 1 && R <= 128, CPTC_ERR_ARG, "cptc_sgd3_update: R %d (1..128)", R);
    if (batch == 0) return CPTC_OK;
    CPTC_REQUIRE(d_coords && d_vals && d_idx && d_A && d_B && d_C && d_lambda, CPTC_ERR_ARG,
                 "cptc_sgd3_update: null pointer");
    return sgd_launch<true>(d_coords, d_vals, d_idx, batch, d_A, d_B, d_C, d_lambda, R, gamma,
                            nullptr, cptc::as_stream(stream), nullptr);
}

extern "C" int cptc_sgd3_loss(const uint64_t* d_coords, const double* d_vals,
                              const uint32_t* d_idx, uint32_t batch, const double* d_A,
                              const double* d_B, const double* d_C, const double* d_lambda, int R,
                              double* d_loss, void* stream)
{
    CPTC_REQUIRE(R >= 1 && R <= 128 && d_loss, CPTC_ERR_ARG, "cptc_sgd3_loss: R %d (1..128)",
                 R);
    hipStream_t s = cptc::as_stream(stream);
    if (batch == 0)
    {
        CPTC_HIP(hipMemsetAsync(d_loss, 0, sizeof(double), s));
        return CPTC_OK;
    }
    CPTC_REQUIRE(d_coords && d_vals && d_idx && d_A && d_B && d_C && d_lambda, CPTC_ERR_ARG,
                 "cptc_sgd3_loss: null pointer");
    int lpe = 8;
    while (lpe < R && lpe < WAVE) lpe <<= 1;
    const unsigned epb = unsigned((SGD_T / WAVE) * (WAVE / lpe));
    const size_t blocks = (uint64_t(batch) + epb - 1) / epb;
    void* buf = nullptr;
    CPTC_TRY(cptc::scratch_get(cptc::SCR_REDUCE, blocks * sizeof(double), &buf));
    double* part = static_cast<double*>(buf);
    unsigned launched = 0;
    CPTC_TRY(sgd_launch<false>(d_coords, d_vals, d_idx, batch, const_cast<double*>(d_A),
                               const_cast<double*>(d_B), const_cast<double*>(d_C), d_lambda, R,
                               0.0, part, s, &launched));
    hipLaunchKernelGGL(sum_parts_kernel, dim3(1), dim3(SGD_T), 0, s, part, int(launched), d_loss);
    CPTC_LAUNCHED();
    return CPTC_OK;
}

extern "C" int cptc_sgd3_normalize(double* d_F, size_t rows, int R, double* d_lambda,
                                   void* stream)
{
    CPTC_REQUIRE(R >= 1 && d_F && d_lambda, CPTC_ERR_ARG, "cptc_sgd3_normalize: bad arguments");
    hipStream_t s = cptc::as_stream(stream);
    void* buf = nullptr;
    CPTC_TRY(cptc::scratch_get(cptc::SCR_FLAGS, size_t(R) * sizeof(double), &buf));
    double* norms = static_cast<double*>(buf);
    CPTC_TRY(cptc_colnorms(d_F, rows, R, norms, s));
    const unsigned grid = cptc::grid_for(rows * size_t(R), SGD_T, 4096);
    hipLaunchKernelGGL(sgd_normalize_kernel, dim3(grid), dim3(SGD_T), 0, s, d_F, rows, R, norms,
                       d_lambda);
    CPTC_LAUNCHED();
    return CPTC_OK;
}
