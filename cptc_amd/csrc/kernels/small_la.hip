// Small dense FP64 kernels of one ALS mode update: Gram, Hadamard, the R x R
// pseudoinverse solve, column norms, normalisation and the Gram fit.
//
// All reductions are two-stage with a fixed order (per-workgroup partials,
// then one ordered sum), so every result is bit-reproducible run to run.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cfloat>
#include <cmath>
#include <cstdlib>
#include <mutex>

#include "../host/hip_util.hpp"
#include "../host/small_la.hpp"

namespace {

constexpr int WAVE = 64;

// ---------------------------------------------------------------------------
// Gram: G = F^T F.  Stage 1: workgroup p sums rows [p*rpw, (p+1)*rpw) into
// partial[p] (one RT x RT output tile per grid.y); stage 2 sums partials in
// p order.  16 x 16 threads, TPT x TPT outputs per thread (RT = 16 * TPT).
// ---------------------------------------------------------------------------
template <int TPT>
__global__ __launch_bounds__(256) void gram_partial_kernel(const double* __restrict__ F,
                                                           size_t rows, int R, size_t rpw,
                                                           int ntile, double* __restrict__ part)
{
    constexpr int RT = 16 * TPT;
    constexpr int CH = 16;
    __shared__ double sa[CH][RT + 1];
    __shared__ double sb[CH][RT + 1];
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    const int bi = int(blockIdx.y) / ntile, bj = int(blockIdx.y) % ntile;
    const int ci = bi * RT, cj = bj * RT;
    const size_t r_lo = size_t(blockIdx.x) * rpw;
    const size_t r_hi = (r_lo + rpw < rows) ? r_lo + rpw : rows;
    double acc[TPT][TPT];
#pragma unroll
    for (int a = 0; a < TPT; ++a)
#pragma unroll
        for (int b = 0; b < TPT; ++b) acc[a][b] = 0.0;
    for (size_t i0 = r_lo; i0 < r_hi; i0 += CH)
    {
        for (int x = threadIdx.x; x < CH * RT; x += 256)
        {
            const int rr = x / RT, cc = x % RT;
            const size_t i = i0 + rr;
            const bool ok = i < r_hi;
            sa[rr][cc] = (ok && ci + cc < R) ? F[i * R + ci + cc] : 0.0;
            sb[rr][cc] = (ok && cj + cc < R) ? F[i * R + cj + cc] : 0.0;
        }
        __syncthreads();
#pragma unroll 4
        for (int rr = 0; rr < CH; ++rr)
        {
            double va[TPT], vb[TPT];
#pragma unroll
            for (int a = 0; a < TPT; ++a) va[a] = sa[rr][ty + 16 * a];
#pragma unroll
            for (int b = 0; b < TPT; ++b) vb[b] = sb[rr][tx + 16 * b];
#pragma unroll
            for (int a = 0; a < TPT; ++a)
#pragma unroll
                for (int b = 0; b < TPT; ++b) acc[a][b] += va[a] * vb[b];
        }
        __syncthreads();
    }
    double* out = part + size_t(blockIdx.x) * size_t(R) * R;
#pragma unroll
    for (int a = 0; a < TPT; ++a)
#pragma unroll
        for (int b = 0; b < TPT; ++b)
        {
            const int r = ci + ty + 16 * a, s = cj + tx + 16 * b;
            if (r < R && s < R) out[size_t(r) * R + s] = acc[a][b];
        }
}

// Gram partials for R > 64 on the FP64 matrix cores (v_mfma_f64_16x16x4f64):
// grid.x = row range p (rows [p rpw, (p + 1) rpw)), grid.y = one upper-
// triangle pair (bi <= bj) of 64-rank tiles.  Wave w takes tile rows
// 16w .. 16w + 15 against the tile's four 16-column blocks t (all four, so
// the MFMA sequence has no branch) and stores t >= w in diagonal tiles: the
// partials hold every entry r <= c, which is what sum_partials_sym_kernel
// reads.  K runs over the range's rows, 4 per
// step: lane l holds A[l % 16][l / 16] = F[i + l / 16][ci + 16w + l % 16]
// and B_t[l / 16][l % 16] = F[i + l / 16][cj + 16t + l % 16]; the
// accumulator's element v of lane l is D[l / 16 + 4 v][l % 16].  Steps run
// in batches of 8 (40 loads, up to 32 MFMAs), two register sets in turn,
// with scheduling barriers so a batch's loads issue before the previous
// batch's MFMAs.  Loads are unconditional: rows past the range read its
// last row and their A is zeroed when the batch is used; columns past R
// read column R - 1 and are not stored.
typedef double gram_d4 __attribute__((ext_vector_type(4)));
constexpr int GRAM_B = 8;   // K steps (of 4 rows) per batch
#ifndef CPTC_GRAM_MFMA_ROWS
#define CPTC_GRAM_MFMA_ROWS 64   // at least this many rows per partial
#endif

__global__ __launch_bounds__(256) void gram_mfma_partial_kernel(const double* __restrict__ F,
                                                                size_t rows, int R, size_t rpw,
                                                                int ntile,
                                                                double* __restrict__ part)
{
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int li = lane & 15, lk = lane >> 4;
    int rem = int(blockIdx.y), bi = 0;
    while (rem >= ntile - bi)
    {
        rem -= ntile - bi;
        ++bi;
    }
    const int bj = bi + rem;
    const int ca = bi * 64 + 16 * w;          // this wave's 16 G rows
    if (ca >= R) return;                      // wave-uniform; no barrier in the kernel
    const int t0 = (bi == bj) ? w : 0;        // first column block at or above the diagonal
    const size_t r_lo = size_t(blockIdx.x) * rpw;
    const size_t r_hi = (r_lo + rpw < rows) ? r_lo + rpw : rows;
    if (r_lo >= r_hi) return;
    const int colA = (ca + li < R) ? ca + li : R - 1;
    int colB[4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
    {
        const int c = bj * 64 + 16 * t + li;
        colB[t] = c < R ? c : R - 1;
    }
    gram_d4 acc[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[t] = gram_d4{0.0, 0.0, 0.0, 0.0};

    struct Batch
    {
        double a[GRAM_B], b[4][GRAM_B];
    };
    const size_t last = r_hi - 1;
    auto load = [&](size_t i0, Batch& x) {
#pragma unroll
        for (int u = 0; u < GRAM_B; ++u)
        {
            const size_t i = i0 + size_t(4 * u + lk);
            const double* __restrict__ row = F + (i < r_hi ? i : last) * size_t(R);
            x.a[u] = row[colA];
#pragma unroll
            for (int t = 0; t < 4; ++t) x.b[t][u] = row[colB[t]];
        }
    };
    auto compute = [&](size_t i0, const Batch& x) {
#pragma unroll
        for (int u = 0; u < GRAM_B; ++u)
        {
            const size_t i = i0 + size_t(4 * u + lk);
            const double a = (i < r_hi) ? x.a[u] : 0.0;
#pragma unroll
            for (int t = 0; t < 4; ++t)
                acc[t] = __builtin_amdgcn_mfma_f64_16x16x4f64(a, x.b[t][u], acc[t], 0, 0, 0);
        }
    };
    constexpr size_t STEP = 4 * GRAM_B;   // rows per batch
    Batch P, Q;
    load(r_lo, P);
    for (size_t i0 = r_lo; i0 < r_hi; i0 += 2 * STEP)
    {
        load(i0 + STEP, Q);
        __builtin_amdgcn_sched_barrier(0);
        compute(i0, P);
        __builtin_amdgcn_sched_barrier(0);
        load(i0 + 2 * STEP, P);
        __builtin_amdgcn_sched_barrier(0);
        compute(i0 + STEP, Q);   // all-zero A past the range
        __builtin_amdgcn_sched_barrier(0);
    }
    double* __restrict__ out = part + size_t(blockIdx.x) * size_t(R) * R;
#pragma unroll
    for (int t = 0; t < 4; ++t)
    {
        if (t < t0) continue;
        const int c = bj * 64 + 16 * t + li;
        if (c >= R) continue;
#pragma unroll
        for (int v = 0; v < 4; ++v)
        {
            const int r = ca + lk + 4 * v;
            if (r < R) out[size_t(r) * R + c] = acc[t][v];
        }
    }
}

// sum over p of part[p * n + x], in a fixed order: eight interleaved
// accumulators (partials p = k mod 8), combined pairwise, so the loads of
// eight partials are in flight at once and the result is the same on every
// run.
__device__ inline double ordered_sum(const double* __restrict__ part, int P, size_t stride,
                                     size_t x)
{
    double a[8] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
    int p = 0;
    for (; p + 8 <= P; p += 8)
#pragma unroll
        for (int k = 0; k < 8; ++k) a[k] += part[size_t(p + k) * stride + x];
    for (int k = 0; p < P; ++p, ++k) a[k] += part[size_t(p) * stride + x];
    return ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
}

__global__ void sum_partials_kernel(const double* __restrict__ part, int P, size_t n,
                                    double* __restrict__ out)
{
    for (size_t x = size_t(blockIdx.x) * blockDim.x + threadIdx.x; x < n;
         x += size_t(gridDim.x) * blockDim.x)
        out[x] = ordered_sum(part, P, n, x);
}

// sum_partials_kernel over upper-triangle partials (gram_mfma_partial_kernel:
// the partials hold the entries r <= c): those entries are summed (partials
// read in order, coalesced) and written to their own place and, above the
// diagonal, to their mirror's (the one scattered access, once per entry
// rather than once per partial), so the result is symmetric by construction.
__global__ void sum_partials_sym_kernel(const double* __restrict__ part, int P, int R,
                                        double* __restrict__ out)
{
    const size_t n = size_t(R) * R;
    for (size_t x = size_t(blockIdx.x) * blockDim.x + threadIdx.x; x < n;
         x += size_t(gridDim.x) * blockDim.x)
    {
        const int r = int(x / size_t(R)), c = int(x % size_t(R));
        if (r > c) continue;
        const double v = ordered_sum(part, P, n, x);
        out[x] = v;
        if (r < c) out[size_t(c) * R + r] = v;
    }
}

__global__ void hadamard_kernel(const double* A, const double* B, double* C, size_t n)
{
    for (size_t x = size_t(blockIdx.x) * blockDim.x + threadIdx.x; x < n;
         x += size_t(gridDim.x) * blockDim.x)
        C[x] = A[x] * B[x];
}

// ---------------------------------------------------------------------------
// pinv, fast path, one workgroup, A in LDS for R <= 128 (global scratch
// otherwise):
//   1. blocked Cholesky A = L L^T: 16-column panels factored by wave 0
//      (lanes over rows, no workgroup barrier inside a panel), then the
//      trailing update by the whole workgroup;
//   2. X = L^-1 by columns, one 8-lane group per column (the dot products
//      split over the group and reduced with xor-shuffles), X^T stored in
//      the free upper triangle;
//   3. Ainv = X^T X.
// Any pivot <= 1e-10 * max diag (or non-finite), or a computed inverse
// that fails fast_inverse_ok, sets *fallback = 1 and leaves Ainv to the
// Jacobi kernel.
// ---------------------------------------------------------------------------
constexpr int PINV_THREADS = 1024;
constexpr int CHOL_NB = 16;
constexpr int INV_G = 8;

__device__ inline void wave_sync_lds()
{
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

// Fast-path acceptance.  The reference keeps sigma_i > R ulp(sigma_max) and
// drops the rest (solver.cu:957-966), so the truncated pseudoinverse equals
// the inverse exactly when sigma_min > R ulp(sigma_max).  With
// kappa_2 <= ||A||_F ||A^-1||_F and ulp(x) <= DBL_EPSILON x, the product
// ||A||_F ||A^-1||_F < 1 / (64 R DBL_EPSILON) implies
// sigma_min > 64 R ulp(sigma_max); the factor 64 covers the rounding of the
// computed inverse.  Small pivots alone do not show this: A = L L^T with L
// unit lower triangular and every sub-diagonal entry -1 has LDL^T pivots 1
// and kappa ~ 4^R.
__device__ inline bool fast_inverse_ok(double fro2_A, double fro2_inv, int R)
{
    const double lim = 1.0 / (64.0 * double(R) * DBL_EPSILON);
    const double p = sqrt(fro2_A) * sqrt(fro2_inv);
    return isfinite(p) && p < lim;
}

// Sum over a workgroup of NT threads (NT / 64 waves); every thread gets the
// total.  red holds NT / 64 doubles; two barriers.
template <int NT>
__device__ inline double block_sum_all(double v, double* red)
{
#pragma unroll
    for (int o = WAVE / 2; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    if ((threadIdx.x & (WAVE - 1)) == 0) red[threadIdx.x / WAVE] = v;
    __syncthreads();
    double t = 0.0;
#pragma unroll
    for (int w = 0; w < NT / WAVE; ++w) t += red[w];
    __syncthreads();
    return t;
}

__global__ __launch_bounds__(PINV_THREADS) void chol_inverse_kernel(const double* __restrict__ Ain,
                                                                    int R, double* work,
                                                                    double* __restrict__ Ainv,
                                                                    int* fallback, int use_lds)
{
    extern __shared__ double lds[];
    double* A = use_lds ? lds : work;
    __shared__ int ok;
    __shared__ double tau;
    __shared__ double xd[512];   // diagonal of X = L^-1 (R <= 512)
    const int tid = threadIdx.x;
    const int lane = tid & (WAVE - 1);
    const int wave = tid / WAVE;
    const int n2 = R * R;
    __shared__ double red[PINV_THREADS / WAVE];
    double fa = 0.0;
    for (int x = tid; x < n2; x += PINV_THREADS)
    {
        const double v = Ain[x];
        A[x] = v;
        fa += v * v;
    }
    if (tid == 0) *fallback = 0;
    const double fro2_A = block_sum_all<PINV_THREADS>(fa, red);
    if (tid == 0)
    {
        double md = 0.0;
        for (int k = 0; k < R; ++k) md = fmax(md, A[k * R + k]);
        tau = 1e-10 * md;
        ok = (md > 0.0 && isfinite(md)) ? 1 : 0;
    }
    __syncthreads();
    // 1. blocked right-looking Cholesky (lower triangle)
    for (int kb = 0; kb < R; kb += CHOL_NB)
    {
        const int ke = (kb + CHOL_NB < R) ? kb + CHOL_NB : R;
        if (wave == 0 && ok)
        {
            for (int k = kb; k < ke; ++k)
            {
                const double d = A[k * R + k];
                if (!(d > tau) || !isfinite(d))
                {
                    if (lane == 0) ok = 0;   // every lane read the same d: uniform exit
                    break;
                }
                const double lkk = sqrt(d);
                for (int i = k + 1 + lane; i < R; i += WAVE) A[i * R + k] /= lkk;
                wave_sync_lds();
                if (lane == 0) A[k * R + k] = lkk;
                for (int j = k + 1; j < ke; ++j)
                {
                    const double ajk = A[j * R + k];
                    for (int i = j + lane; i < R; i += WAVE) A[i * R + j] -= A[i * R + k] * ajk;
                }
                wave_sync_lds();
            }
        }
        __syncthreads();
        if (!ok) break;
        const int m = R - ke;
        for (int idx = tid; idx < m * m; idx += PINV_THREADS)
        {
            const int ii = idx / m, jj = idx - ii * m;
            if (jj > ii) continue;
            const int i = ke + ii, j = ke + jj;
            double acc = 0.0;
            for (int k = kb; k < ke; ++k) acc += A[i * R + k] * A[j * R + k];
            A[i * R + j] -= acc;
        }
        __syncthreads();
    }
    if (!ok)
    {
        if (tid == 0) *fallback = 1;
        return;
    }
    // 2. X = L^-1: column c by group c; X[j][c] (j > c) at A[c][j], X[c][c] at xd[c]
    const int grp = tid / INV_G, gl = tid % INV_G;
    for (int c = grp; c < R; c += PINV_THREADS / INV_G)
    {
        const double xc = 1.0 / A[c * R + c];
        if (gl == 0) xd[c] = xc;
        for (int j = c + 1; j < R; ++j)
        {
            double s = (gl == 0) ? A[j * R + c] * xc : 0.0;
            for (int q = c + 1 + gl; q < j; q += INV_G) s += A[j * R + q] * A[c * R + q];
            s += __shfl_xor(s, 4, INV_G);
            s += __shfl_xor(s, 2, INV_G);
            s += __shfl_xor(s, 1, INV_G);
            if (gl == 0) A[c * R + j] = -s / A[j * R + j];
            wave_sync_lds();
        }
    }
    __syncthreads();
    // 3. X row-major lower triangular in place (L is no longer needed): each
    //    lower entry is written from its transposed upper entry by one thread
    for (int idx = tid; idx < n2; idx += PINV_THREADS)
    {
        const int r = idx / R, c = idx - r * R;
        if (c < r) A[r * R + c] = A[c * R + r];
    }
    __syncthreads();
    for (int idx = tid; idx < n2; idx += PINV_THREADS)
    {
        const int r = idx / R, c = idx - r * R;
        if (c > r) A[r * R + c] = 0.0;
        if (c == r) A[r * R + r] = xd[r];
    }
    __syncthreads();
    // 4. Ainv = X^T X in 4 x 4 register blocks: Ainv[r][c] = sum_j X[j][r] X[j][c]
    //    (X[j][r] = 0 for j < r, so j starts at the block's smaller index)
    const int nb = (R + 3) / 4;
    double fi = 0.0;
    for (int b = tid; b < nb * nb; b += PINV_THREADS)
    {
        const int r0 = 4 * (b / nb), c0 = 4 * (b % nb);
        double acc[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int k = 0; k < 4; ++k) acc[i][k] = 0.0;
        for (int j = (r0 < c0 ? r0 : c0); j < R; ++j)
        {
            const double* xj = A + size_t(j) * R;
            double xr[4], xc[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
            {
                xr[i] = (r0 + i < R) ? xj[r0 + i] : 0.0;
                xc[i] = (c0 + i < R) ? xj[c0 + i] : 0.0;
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int k = 0; k < 4; ++k) acc[i][k] += xr[i] * xc[k];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (r0 + i < R && c0 + k < R)
                {
                    Ainv[(r0 + i) * R + c0 + k] = acc[i][k];
                    fi += acc[i][k] * acc[i][k];
                }
    }
    // 5. condition check (fast_inverse_ok); on failure the Jacobi kernel
    //    overwrites Ainv with the truncated pseudoinverse
    const double fro2_inv = block_sum_all<PINV_THREADS>(fi, red);
    if (tid == 0 && !fast_inverse_ok(fro2_A, fro2_inv, R)) *fallback = 1;
}

// ---------------------------------------------------------------------------
// pinv, fast path for R <= 64: one workgroup of SWEEP_T threads, the matrix
// in registers.  Symmetric sweep (Beaton's SWEEP operator, i.e.
// Gauss-Jordan elimination without pivoting in its symmetric form):
// sweeping pivot k maps
//   a_kk -> -1 / a_kk,  a_ik -> a_ik / a_kk  (i != k),
//   a_ij -> a_ij - a_ik a_kj / a_kk          (i, j != k),
// and after every pivot the matrix holds -A^-1.  The matrix stays
// symmetric, so pivot row k is column k.  The pivots are the LDL^T pivots
// (the squared Cholesky diagonal), so the fast-path test is the Cholesky
// one: a pivot <= 1e-10 * max diag (or non-finite), or an inverse that
// fails fast_inverse_ok, sets *fallback = 1 and leaves Ainv to the Jacobi
// kernel.
// Thread layout: RT >= R rows (16, 32 or 64), LPR = SWEEP_T / RT threads
// per row, each holding C = RT / LPR consecutive columns: thread = row + RT
// * part, columns part * C .. part * C + C - 1 (C = 1, 4, 16).  Per pivot
// the threads owning column k write it to LDS (one slot per row) and every
// thread reads its row's entry and its C columns' entries back.
// ---------------------------------------------------------------------------
constexpr int SWEEP_T = 256;

template <int T>
__device__ void jacobi_pinv_body(const double* __restrict__ Ain, int R, double* work, double* V,
                                 double* __restrict__ Ainv, int use_lds, double* lds);

// When the fast path declines, the same workgroup runs the Jacobi
// pseudoinverse (jacobi_pinv_body with its 256 threads, A in this kernel's
// LDS, V in `V`), so R <= 64 needs one launch per solve, not two.
template <int RT>
__global__ __launch_bounds__(SWEEP_T) void sweep_inverse_kernel(const double* __restrict__ Ain,
                                                                int R,
                                                                double* __restrict__ Ainv,
                                                                int* fallback, double* V)
{
    __shared__ double jA[RT * RT];   // the Jacobi path's A
    constexpr int LPR = SWEEP_T / RT;
    constexpr int C = RT / LPR;
    static_assert(C >= 1 && C <= 16, "sweep layout");
    __shared__ double col[RT];
    __shared__ double wmax[SWEEP_T / WAVE];
    __shared__ double wsum[SWEEP_T / WAVE];
    const int tid = threadIdx.x;
    const int row = tid % RT;
    const int part = tid / RT;
    const int c0 = part * C;
    double a[C];
#pragma unroll
    for (int c = 0; c < C; ++c)
        a[c] = (row < R && c0 + c < R) ? Ain[size_t(row) * R + c0 + c] : 0.0;
    // largest diagonal entry (the thread holding (row, row) contributes it)
    // and ||A||_F^2
    double md = 0.0, fa = 0.0;
#pragma unroll
    for (int c = 0; c < C; ++c)
    {
        if (c0 + c == row) md = a[c];
        fa += a[c] * a[c];
    }
#pragma unroll
    for (int o = WAVE / 2; o >= 1; o >>= 1)
    {
        md = fmax(md, __shfl_xor(md, o));
        fa += __shfl_xor(fa, o);
    }
    if ((tid & (WAVE - 1)) == 0)
    {
        wmax[tid / WAVE] = md;
        wsum[tid / WAVE] = fa;
    }
    __syncthreads();
    double fro2_A = 0.0;
#pragma unroll
    for (int w = 0; w < SWEEP_T / WAVE; ++w)
    {
        md = fmax(md, wmax[w]);
        fro2_A += wsum[w];
    }
    const double tau = 1e-10 * md;
    int ok = (md > 0.0 && isfinite(md)) ? 1 : 0;
#pragma unroll 1
    for (int kp = 0; kp < LPR && kp * C < R && ok; ++kp)
    {
#pragma unroll
        for (int kc = 0; kc < C; ++kc)
        {
            const int k = kp * C + kc;
            if (k >= R || !ok) continue;   // uniform
            if (part == kp) col[row] = a[kc];
            __syncthreads();
            const double p = col[k];
            if (!(p > tau) || !isfinite(p))
            {
                ok = 0;   // every thread read the same pivot: uniform exit
                continue;
            }
            const double ip = 1.0 / p;
            const double f = col[row] * ip;    // a_ik / a_kk (1 on row k)
            const bool prow = row == k;
            const double g = prow ? 0.0 : f;
            const double h = prow ? ip : 1.0;
            double cj[C];
#pragma unroll
            for (int c = 0; c < C; ++c) cj[c] = col[c0 + c];
#pragma unroll
            for (int c = 0; c < C; ++c)
            {
                const double up = fma(-g, cj[c], a[c] * h);
                a[c] = (c == kc && part == kp) ? (prow ? -ip : f) : up;
            }
            __syncthreads();
        }
    }
    // both declines below are uniform over the workgroup
    if (!ok)
    {
        if (tid == 0) *fallback = 1;
        jacobi_pinv_body<SWEEP_T>(Ain, R, nullptr, V, Ainv, 1, jA);
        return;
    }
    // condition check (fast_inverse_ok); padding entries are 0
    double fi = 0.0;
#pragma unroll
    for (int c = 0; c < C; ++c) fi += a[c] * a[c];
    const double fro2_inv = block_sum_all<SWEEP_T>(fi, wsum);
    if (!fast_inverse_ok(fro2_A, fro2_inv, R))
    {
        if (tid == 0) *fallback = 1;
        jacobi_pinv_body<SWEEP_T>(Ain, R, nullptr, V, Ainv, 1, jA);
        return;
    }
    if (tid == 0) *fallback = 0;
    if (row < R)
#pragma unroll
        for (int c = 0; c < C; ++c)
            if (c0 + c < R) Ainv[size_t(row) * R + c0 + c] = -a[c];
}

// ---------------------------------------------------------------------------
// pinv, exact path (runs only when *fallback != 0): parallel cyclic Jacobi
// (round-robin pair ordering, Brent & Luk 1985) on A = V diag(l) V^T, then
// Ainv = sum_{|l_i| > R ulp(max|l|)} v_i v_i^T / l_i — the truncated SVD
// pseudoinverse of a symmetric matrix (solver.cu:764-775, 900-1002).
// A in LDS (R <= 128) or global scratch; V in global scratch.
// ---------------------------------------------------------------------------
constexpr int JACOBI_SWEEPS = 15;
constexpr double JACOBI_TOL = 1e-14;

template <int T>
__device__ void jacobi_pinv_body(const double* __restrict__ Ain, int R, double* work, double* V,
                                 double* __restrict__ Ainv, int use_lds, double* lds)
{
    double* A = use_lds ? lds : work;
    __shared__ double red[T / WAVE];
    __shared__ double s_off, s_fro;
    __shared__ int pair_p[256], pair_q[256];
    __shared__ double rot_c[256], rot_s[256];
    const int tid = threadIdx.x;
    const int n2 = R * R;
    const int Rp = R + (R & 1);  // even with a dummy index R when R is odd
    const int npairs = Rp / 2;
    for (int x = tid; x < n2; x += T)
    {
        A[x] = Ain[x];
        V[x] = ((x / R) == (x % R)) ? 1.0 : 0.0;
    }
    __syncthreads();
    auto block_sum = [&](double v) -> double {
        for (int off = WAVE / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, WAVE);
        if ((tid & (WAVE - 1)) == 0) red[tid / WAVE] = v;
        __syncthreads();
        double t = 0.0;
        for (int w = 0; w < T / WAVE; ++w) t += red[w];
        __syncthreads();
        return t;
    };
    {
        double f = 0.0;
        for (int x = tid; x < n2; x += T) f += A[x] * A[x];
        f = block_sum(f);
        if (tid == 0) s_fro = sqrt(f);
    }
    __syncthreads();
    // gesvdj's settings in the reference (solver.cu:837-838): at most 15
    // sweeps, stop once the off-diagonal norm is <= 1e-14 of the Frobenius norm
    for (int sweep = 0; sweep < JACOBI_SWEEPS; ++sweep)
    {
        double o = 0.0;
        for (int x = tid; x < n2; x += T)
            if ((x / R) != (x % R)) o += A[x] * A[x];
        o = block_sum(o);
        if (tid == 0) s_off = sqrt(o);
        __syncthreads();
        if (!(s_off > JACOBI_TOL * s_fro)) break;
        for (int round = 0; round < Rp - 1; ++round)
        {
            // round-robin: index 0 fixed, others rotate
            for (int k = tid; k < npairs; k += T)
            {
                auto at = [&](int pos) { return pos == 0 ? 0 : 1 + (pos - 1 + round) % (Rp - 1); };
                int p = at(k), q = at(Rp - 1 - k);
                if (p > q) { const int t = p; p = q; q = t; }
                double c = 1.0, s = 0.0;
                if (q < R)
                {
                    const double apq = A[p * R + q];
                    if (apq != 0.0)
                    {
                        const double theta = (A[q * R + q] - A[p * R + p]) / (2.0 * apq);
                        const double t = (theta >= 0.0 ? 1.0 : -1.0) /
                                         (fabs(theta) + sqrt(theta * theta + 1.0));
                        c = 1.0 / sqrt(t * t + 1.0);
                        s = t * c;
                    }
                }
                pair_p[k] = p;
                pair_q[k] = q;
                rot_c[k] = c;
                rot_s[k] = s;
            }
            __syncthreads();
            // A <- J^T A J, one 2 x 2 block (rows of pair a, columns of pair
            // b) per item, in place: the column rotation of pair b, then the
            // row rotation of pair a on the column-rotated values, the same
            // operations on every entry as a pass over all columns followed
            // by a pass over all rows, with one barrier per round fewer
            for (int x = tid; x < npairs * npairs; x += T)
            {
                const int a = x / npairs, b = x % npairs;
                const int i0 = pair_p[a], i1 = pair_q[a], j0 = pair_p[b], j1 = pair_q[b];
                const bool ra = i1 < R && rot_s[a] != 0.0, rb = j1 < R && rot_s[b] != 0.0;
                if (!ra && !rb) continue;
                const bool has_i1 = i1 < R, has_j1 = j1 < R;
                double a00 = A[i0 * R + j0];
                double a01 = has_j1 ? A[i0 * R + j1] : 0.0;
                double a10 = has_i1 ? A[i1 * R + j0] : 0.0;
                double a11 = (has_i1 && has_j1) ? A[i1 * R + j1] : 0.0;
                if (rb)
                {
                    const double c = rot_c[b], sn = rot_s[b];
                    const double t00 = c * a00 - sn * a01, t01 = sn * a00 + c * a01;
                    const double t10 = c * a10 - sn * a11, t11 = sn * a10 + c * a11;
                    a00 = t00;
                    a01 = t01;
                    a10 = t10;
                    a11 = t11;
                }
                if (ra)
                {
                    const double c = rot_c[a], sn = rot_s[a];
                    const double t00 = c * a00 - sn * a10, t10 = sn * a00 + c * a10;
                    const double t01 = c * a01 - sn * a11, t11 = sn * a01 + c * a11;
                    a00 = t00;
                    a01 = t01;
                    a10 = t10;
                    a11 = t11;
                }
                A[i0 * R + j0] = a00;
                if (has_j1) A[i0 * R + j1] = a01;
                if (has_i1) A[i1 * R + j0] = a10;
                if (has_i1 && has_j1) A[i1 * R + j1] = a11;
            }
            // V <- V J, V in global memory: a thread's VB column pairs are
            // loaded together, then rotated and stored, so a round waits on
            // one memory round trip per VB pairs instead of one per pair
            // (the same operations on every entry as a pair-at-a-time loop)
            constexpr int VB = 8;
            for (int x0 = 0; x0 < npairs * R; x0 += VB * T)
            {
                double vp[VB], vq[VB], cc[VB], ss[VB];
                int ip[VB], iq[VB];
                bool on[VB];
#pragma unroll
                for (int j = 0; j < VB; ++j)
                {
                    const int x = x0 + j * T + tid;
                    const int k = x / R, r = x % R;
                    on[j] = x < npairs * R;
                    const int kk = on[j] ? k : 0;
                    const int p = pair_p[kk], q = pair_q[kk];
                    on[j] = on[j] && q < R && rot_s[kk] != 0.0;
                    cc[j] = rot_c[kk];
                    ss[j] = rot_s[kk];
                    ip[j] = on[j] ? r * R + p : 0;
                    iq[j] = on[j] ? r * R + q : 0;
                    vp[j] = on[j] ? V[ip[j]] : 0.0;
                    vq[j] = on[j] ? V[iq[j]] : 0.0;
                }
#pragma unroll
                for (int j = 0; j < VB; ++j)
                    if (on[j])
                    {
                        V[ip[j]] = cc[j] * vp[j] - ss[j] * vq[j];
                        V[iq[j]] = ss[j] * vp[j] + cc[j] * vq[j];
                    }
            }
            __syncthreads();
        }
    }
    __shared__ double s_tol;
    if (tid == 0)
    {
        double smax = 0.0;
        for (int k = 0; k < R; ++k) smax = fmax(smax, fabs(A[k * R + k]));
        s_tol = double(R) * (nextafter(smax, smax + 1.0) - smax);
    }
    __syncthreads();
    for (int x = tid; x < n2; x += T)
    {
        const int r = x / R, c = x % R;
        double s = 0.0;
        for (int k = 0; k < R; ++k)
        {
            const double l = A[k * R + k];
            if (fabs(l) > s_tol) s += V[r * R + k] * (1.0 / l) * V[c * R + k];
        }
        Ainv[x] = s;
    }
}

__global__ __launch_bounds__(PINV_THREADS) void jacobi_pinv_kernel(const double* __restrict__ Ain,
                                                                   int R, double* work,
                                                                   double* V,
                                                                   double* __restrict__ Ainv,
                                                                   const int* fallback,
                                                                   int use_lds)
{
    if (*fallback == 0) return;
    extern __shared__ double lds[];
    jacobi_pinv_body<PINV_THREADS>(Ain, R, work, V, Ainv, use_lds, lds);
}

// ---------------------------------------------------------------------------
// F = FtV * Ainv (row-major dim x R times R x R), then F[:, r] /= div[r],
// for R > 64, on the FP64 matrix cores (v_mfma_f64_16x16x4f64).
//
// A workgroup of 4 waves takes 16 rows x 128 columns (grid.y walks 128-wide
// column blocks when R > 128); wave w takes columns 32w .. 32w + 31 of the
// block as two 16 x 16 tiles.  K advances 4 per step.  Operand layout of the
// instruction: lane l holds A[l % 16][l / 16] = Y[row0 + l % 16][k + l / 16]
// and B[l / 16][l % 16] = Ainv[k + l / 16][col + l % 16]; the accumulator's
// element v of lane l is D[l / 16 + 4 v][l % 16] (measured: the FP32
// instructions' 4 (l / 16) + v order does not hold for this one).
//
// On this GPU the FP64 matrix rate equals the FP64 vector rate; the matrix
// form pays because each operand in a register feeds 16 products.  The
// workgroup's 16 rows of Y are staged in LDS, 128 columns of K at a time
// (an A operand read from global memory touches 16 rows, i.e. 16 cache
// lines, per instruction, and the four waves would each read it), zero
// from R to the pass's 128 columns; batches never run past them.  Steps run in batches of 8 (16 B-operand
// loads, 8 LDS reads, 16 MFMAs), two register sets in turn: a batch's loads
// are issued before the previous batch's MFMAs.  The B loads are
// unconditional (a column past R reads column R - 1 and is not stored; a K
// step past R reads row R - 1 and meets a zero A), so no branch sits
// between a load and its use.
// ---------------------------------------------------------------------------
typedef double apply_d4 __attribute__((ext_vector_type(4)));
constexpr int APPLY_B = 8;            // K steps (of 4) per batch
constexpr int APPLY_KC = 128;         // K columns of Y staged per pass
constexpr int APPLY_LD = APPLY_KC + 1;   // LDS row stride (odd: rows on distinct banks)

__global__ __launch_bounds__(256) void apply_mfma_kernel(const double* __restrict__ Y,
                                                         const double* __restrict__ Ainv,
                                                         double* __restrict__ F, size_t dim, int R,
                                                         const double* __restrict__ div)
{
    __shared__ double sA[16 * APPLY_LD];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int li = lane & 15, lk = lane >> 4;
    const size_t row0 = size_t(blockIdx.x) * 16;
    const int cb = int(blockIdx.y) * 128 + wave * 32;
    const bool active = cb < R;   // wave-uniform: waves past R stage and wait only
    const int c0 = cb + li, c1 = cb + 16 + li;
    const bool c0_ok = c0 < R, c1_ok = c1 < R;
    const int c0c = c0_ok ? c0 : R - 1, c1c = c1_ok ? c1 : R - 1;
    apply_d4 acc0 = {0.0, 0.0, 0.0, 0.0}, acc1 = {0.0, 0.0, 0.0, 0.0};

    struct Batch
    {
        double b0[APPLY_B], b1[APPLY_B];
    };
    // B operands of batch bt of the pass at K offset kc (K rows clamped to R)
    auto load = [&](int kc, int bt, Batch& x) {
#pragma unroll
        for (int u = 0; u < APPLY_B; ++u)
        {
            const int k = kc + 4 * (APPLY_B * bt + u) + lk;
            const double* __restrict__ ak = Ainv + size_t(k < R ? k : R - 1) * size_t(R);
            x.b0[u] = ak[c0c];
            x.b1[u] = ak[c1c];
        }
    };
    auto compute = [&](int bt, const Batch& x) {
        const double* __restrict__ arow = sA + li * APPLY_LD + 4 * APPLY_B * bt + lk;
#pragma unroll
        for (int u = 0; u < APPLY_B; ++u)
        {
            const double a = arow[4 * u];
            acc0 = __builtin_amdgcn_mfma_f64_16x16x4f64(a, x.b0[u], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f64_16x16x4f64(a, x.b1[u], acc1, 0, 0, 0);
        }
    };

    for (int kc = 0; kc < R; kc += APPLY_KC)
    {
        const int kn = R - kc < APPLY_KC ? R - kc : APPLY_KC;
        if (kc > 0) __syncthreads();   // the previous pass's LDS reads are done
        // the first batch's B operands load while Y is staged (inactive
        // waves load them too, from clamped addresses, and never use them)
        Batch P, Q;
        load(kc, 0, P);
        __builtin_amdgcn_sched_barrier(0);
        {
            // 16 x 128 entries, 8 per thread: row 2j + tid / 128, column
            // tid % 128; loads from clamped addresses, all issued before
            // the first store
            constexpr int PER = 16 * APPLY_KC / 256;
            const int c = tid & (APPLY_KC - 1);
            const int cc = kc + (c < kn ? c : kn - 1);
            double v[PER];
#pragma unroll
            for (int j = 0; j < PER; ++j)
            {
                const size_t i = row0 + size_t(2 * j + (tid >> 7));
                v[j] = Y[(i < dim ? i : dim - 1) * size_t(R) + cc];
            }
#pragma unroll
            for (int j = 0; j < PER; ++j)
            {
                const int r = 2 * j + (tid >> 7);
                const bool ok = c < kn && row0 + size_t(r) < dim;
                sA[r * APPLY_LD + c] = ok ? v[j] : 0.0;
            }
        }
        __syncthreads();
        if (!active) continue;
        // batches of this pass, taken in pairs; an odd count (kn <= 96) runs
        // one more batch, over the staged zeros between kn and 128
        const int nb = (kn + 4 * APPLY_B - 1) / (4 * APPLY_B);
        // the scheduling barriers keep each batch's loads ahead of the other
        // batch's MFMAs (left alone, the scheduler sinks every load to its use)
        for (int bt = 0; bt < nb; bt += 2)
        {
            load(kc, bt + 1, Q);
            __builtin_amdgcn_sched_barrier(0);
            compute(bt, P);
            __builtin_amdgcn_sched_barrier(0);
            load(kc, bt + 2 < nb ? bt + 2 : bt, P);   // the last pass's reload is not used
            __builtin_amdgcn_sched_barrier(0);
            compute(bt + 1, Q);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    if (!active) return;

    const double d0 = (div && c0_ok) ? div[c0] : 1.0;
    const double d1 = (div && c1_ok) ? div[c1] : 1.0;
#pragma unroll
    for (int v = 0; v < 4; ++v)
    {
        const size_t i = row0 + size_t(lk + 4 * v);
        if (i >= dim) continue;
        double* __restrict__ out = F + i * size_t(R);
        if (c0_ok) out[c0] = div ? acc0[v] / d0 : acc0[v];
        if (c1_ok) out[c1] = div ? acc1[v] / d1 : acc1[v];
    }
}

// F = FtV * Ainv for R <= 64: Ainv staged in LDS, one thread per output
// entry (row x / R, column x % R); the R threads of a row read the same FtV
// row; each entry is one k-ascending FMA chain.
constexpr int APPLY_SMALL_R = 64;
__global__ __launch_bounds__(256) void apply_small_kernel(const double* __restrict__ Y,
                                                          const double* __restrict__ Ainv,
                                                          double* __restrict__ F, size_t dim,
                                                          int R, const double* __restrict__ div)
{
    __shared__ double sa[APPLY_SMALL_R * APPLY_SMALL_R];
    for (int x = threadIdx.x; x < R * R; x += 256) sa[x] = Ainv[x];
    __syncthreads();
    const size_t n = dim * size_t(R);
    for (size_t x = size_t(blockIdx.x) * 256 + threadIdx.x; x < n;
         x += size_t(gridDim.x) * 256)
    {
        const size_t i = x / size_t(R);
        const int c = int(x - i * size_t(R));
        const double* __restrict__ y = Y + i * size_t(R);
        double acc = 0.0;
        for (int k = 0; k < R; ++k) acc = fma(y[k], sa[k * R + c], acc);
        F[x] = div ? acc / div[c] : acc;
    }
}

// ---------------------------------------------------------------------------
// Column reductions: partial[p][r] over a row range, then ordered sums.
// mode 0: sum F^2;  mode 1: sum F * M.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void col_partial_kernel(const double* __restrict__ F,
                                                          const double* __restrict__ M,
                                                          size_t rows, int R, size_t rpw,
                                                          double* __restrict__ part)
{
    // thread t handles ranks r = t % R' ... with R' = min(R, 256) lanes per row
    const int lanes = R < 256 ? R : 256;
    const int rows_per_pass = 256 / lanes;
    const int sub = threadIdx.x / lanes;
    const int rl = threadIdx.x % lanes;
    const size_t r_lo = size_t(blockIdx.x) * rpw;
    const size_t r_hi = (r_lo + rpw < rows) ? r_lo + rpw : rows;
    __shared__ double red[256];
    for (int rb = 0; rb < R; rb += lanes)
    {
        const int r = rb + rl;
        // eight independent chains over rows i = r_lo + sub + k * rows_per_pass
        // (eight rows' loads in flight per thread)
        double s8[8] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
        if (sub < rows_per_pass && r < R)
        {
            size_t i = r_lo + sub;
            const size_t step = size_t(rows_per_pass);
            for (; i + 7 * step < r_hi; i += 8 * step)
#pragma unroll
                for (int k = 0; k < 8; ++k)
                {
                    const size_t ii = i + size_t(k) * step;
                    const double f = F[ii * R + r];
                    s8[k] += M ? f * M[ii * R + r] : f * f;
                }
            for (int k = 0; i < r_hi; i += step, ++k)
            {
                const double f = F[i * R + r];
                s8[k] += M ? f * M[i * R + r] : f * f;
            }
        }
        red[threadIdx.x] = ((s8[0] + s8[1]) + (s8[2] + s8[3])) + ((s8[4] + s8[5]) + (s8[6] + s8[7]));
        __syncthreads();
        if (threadIdx.x < lanes && rb + threadIdx.x < R)
        {
            double t = 0.0;
            for (int q = 0; q < rows_per_pass; ++q) t += red[q * lanes + threadIdx.x];
            part[size_t(blockIdx.x) * R + rb + threadIdx.x] = t;
        }
        __syncthreads();
    }
}

__global__ void norms_finalize_kernel(const double* __restrict__ part, int P, int R,
                                      double* __restrict__ norms)
{
    for (int r = threadIdx.x; r < R; r += blockDim.x) norms[r] = sqrt(ordered_sum(part, P, R, r));
}

// als.cu:308-342
__global__ void normalize_absorb_kernel(double* __restrict__ F, size_t rows, int R,
                                        const double* __restrict__ norms,
                                        double* __restrict__ lambda)
{
    const size_t total = rows * size_t(R);
    for (size_t x = size_t(blockIdx.x) * blockDim.x + threadIdx.x; x < total;
         x += size_t(gridDim.x) * blockDim.x)
    {
        const int r = int(x % size_t(R));
        const double n = norms[r];
        F[x] = (n < 1e-14) ? 0.0 : F[x] / n;
    }
    if (blockIdx.x == 0)
        for (int r = threadIdx.x; r < R; r += blockDim.x)
        {
            const double n = norms[r];
            lambda[r] = (n < 1e-14) ? 0.0 : lambda[r] * n;
        }
}

// iprod and model^2 of the Gram fit (als.cu:659-715), one 1024-thread block
// (R <= 1024): iprod_r = lambda_r * sum_p part[p][r] with the partials split
// over 1024 / R thread chunks, model^2 = sum lambda lambda^T o G_1 o ... o
// G_ngram; fixed-order tree reductions.
constexpr int FIT_T = 1024;

__device__ inline double block_sum(double v, double* red)
{
    red[threadIdx.x] = v;
    __syncthreads();
    for (int w = FIT_T / 2; w > 0; w >>= 1)
    {
        if (int(threadIdx.x) < w) red[threadIdx.x] += red[threadIdx.x + w];
        __syncthreads();
    }
    const double t = red[0];
    __syncthreads();
    return t;
}

__global__ __launch_bounds__(FIT_T) void fit_finalize_kernel(const double* __restrict__ part,
                                                             int P, int R,
                                                             const double* __restrict__ lambda,
                                                             const double* __restrict__ grams,
                                                             int ngram, double* __restrict__ out2)
{
    __shared__ double red[FIT_T];
    __shared__ double lam[FIT_T];
    const int tid = threadIdx.x;
    if (tid < R) lam[tid] = lambda[tid];
    const int C = FIT_T / R;   // chunks of partials per rank
    const int r = tid % R, c = tid / R;
    // eight independent accumulators (partials p, p + C, ... loaded together)
    double d8[8] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
    if (c < C)
    {
        int p = c;
        for (; p + 7 * C < P; p += 8 * C)
#pragma unroll
            for (int q = 0; q < 8; ++q) d8[q] += part[size_t(p + q * C) * R + r];
        for (int q = 0; p < P; p += C, ++q) d8[q] += part[size_t(p) * R + r];
    }
    const double d = ((d8[0] + d8[1]) + (d8[2] + d8[3])) + ((d8[4] + d8[5]) + (d8[6] + d8[7]));
    red[tid] = (c < C) ? d : 0.0;
    __syncthreads();
    double ip = 0.0;
    if (tid < R)
    {
        double t = 0.0;
        for (int q = 0; q < C; ++q) t += red[q * R + tid];
        ip = lam[tid] * t;
    }
    __syncthreads();
    const double iprod = block_sum(ip, red);
    // thread t: column c = t % R of rows t / R, t / R + T / R, ... (no index
    // division per entry), four independent accumulators
    double m4[4] = {0.0, 0.0, 0.0, 0.0};
    const size_t RR = size_t(R) * R;
    const int rpp = FIT_T / R;
    const int cc = tid % R, r0 = tid / R;
    if (r0 < rpp)
    {
        const double lc = lam[cc];
        auto term = [&](int i) {
            const size_t x = size_t(i) * R + cc;
            double v = lam[i] * lc;
            for (int g = 0; g < ngram; ++g) v *= grams[size_t(g) * RR + x];
            return v;
        };
        int i = r0;
        for (; i + 3 * rpp < R; i += 4 * rpp)
#pragma unroll
            for (int q = 0; q < 4; ++q) m4[q] += term(i + q * rpp);
        for (int q = 0; i < R; i += rpp, ++q) m4[q] += term(i);
    }
    const double md = (m4[0] + m4[1]) + (m4[2] + m4[3]);
    const double model2 = block_sum(md, red);
    if (tid == 0)
    {
        out2[0] = iprod;
        out2[1] = model2;
    }
}

// The Gram of the normalised factor from the Gram of the unnormalised one
// (als.cu:308-342 with the Gram refresh after it): n_r = sqrt(G_rr);
// lambda_r *= n_r and G_rs /= n_r n_s, with a column of norm < 1e-14 set to
// zero (its lambda and its Gram row / column too); when `other` is given,
// also the next mode's FtF = G .* other (hadamard_kernel's product, bit for
// bit).  One block; thread t keeps column t % R of rows t / R, t / R + T / R,
// ... (no index division per entry), the norms in LDS.
__global__ __launch_bounds__(FIT_T) void gram_norms_absorb_kernel(double* __restrict__ G, int R,
                                                                  double* __restrict__ norms,
                                                                  double* __restrict__ lambda,
                                                                  const double* __restrict__ other,
                                                                  double* __restrict__ FtF)
{
    __shared__ double nl[FIT_T];
    for (int r = threadIdx.x; r < R; r += FIT_T)
    {
        const double n = sqrt(G[size_t(r) * R + r]);
        norms[r] = n;
        nl[r] = n;
        lambda[r] = (n < 1e-14) ? 0.0 : lambda[r] * n;
    }
    __syncthreads();
    const int rpp = FIT_T / R;   // rows per pass (R <= FIT_T)
    const int c = int(threadIdx.x) % R, r0 = int(threadIdx.x) / R;
    if (r0 >= rpp) return;
    const double nj = nl[c];
    // entry i of column c: G /= n_i n_j (0 when either norm is below
    // 1e-14), the division by 1 of a masked 0 standing for the select, so
    // that neither the load nor the division sits under a branch
    auto scaled = [&](int i, double g) {
        const double ni = nl[i];
        const bool keep = !(ni < 1e-14 || nj < 1e-14);
        long long m = keep ? -1LL : 0LL;
        asm volatile("" : "+v"(m));
        return __longlong_as_double(__double_as_longlong(g) & m) / (keep ? ni * nj : 1.0);
    };
    auto one = [&](int i) {
        const size_t x = size_t(i) * R + c;
        const double v = scaled(i, G[x]);
        G[x] = v;
        if (other) FtF[x] = v * other[x];
    };
    // four rows per round, their loads issued before any store (G is
    // updated in place, so a load after a store would wait for it)
    int i = r0;
    for (; i + 3 * rpp < R; i += 4 * rpp)
    {
        double g4[4], o4[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
        {
            const size_t x = size_t(i + q * rpp) * R + c;
            g4[q] = G[x];
            o4[q] = other ? other[x] : 0.0;
        }
#pragma unroll
        for (int q = 0; q < 4; ++q)
        {
            const size_t x = size_t(i + q * rpp) * R + c;
            const double v = scaled(i + q * rpp, g4[q]);
            G[x] = v;
            if (other) FtF[x] = v * o4[q];
        }
    }
    for (; i < R; i += rpp) one(i);
}

// R <= 32, one workgroup: the partial Gram sums of cptc_gram (the same
// ordered sums), then gram_norms_absorb_kernel's norms, lambda and
// normalisation, then, when `other` is given, the next mode's FtF = G .*
// other (hadamard_kernel; the product commutes bit for bit).  Two and, with
// the product, three launches in one.
__global__ __launch_bounds__(FIT_T) void gram_finish_small_kernel(
    const double* __restrict__ part, int P, int R, double* __restrict__ G,
    double* __restrict__ norms, double* __restrict__ lambda, const double* __restrict__ other,
    double* __restrict__ FtF)
{
    __shared__ double g_l[32 * 32];
    __shared__ double n_l[32];
    const int RR = R * R;
    const int x = threadIdx.x;
    if (x < RR) g_l[x] = ordered_sum(part, P, size_t(RR), size_t(x));
    __syncthreads();
    if (x < R)
    {
        const double n = sqrt(g_l[x * R + x]);
        n_l[x] = n;
        norms[x] = n;
        lambda[x] = (n < 1e-14) ? 0.0 : lambda[x] * n;
    }
    __syncthreads();
    if (x < RR)
    {
        const double ni = n_l[x / R], nj = n_l[x % R];
        const double v = (ni < 1e-14 || nj < 1e-14) ? 0.0 : g_l[x] / (ni * nj);
        G[x] = v;
        if (other) FtF[x] = v * other[x];
    }
}

__global__ void zero_kernel(double* __restrict__ p, size_t n)
{
    for (size_t x = size_t(blockIdx.x) * blockDim.x + threadIdx.x; x < n;
         x += size_t(gridDim.x) * blockDim.x)
        p[x] = 0.0;
}

// F[:, r] /= n_r (0 when n_r < 1e-14).  The driver's update tail also
// hands this last launch of a mode's update two jobs for the next mode
// (cptc::TailJobs): zero z[0, nz) (the next MTTKRP's output, once the apply
// has read it) and form C = A .* B over n2 entries (the next mode's FtF,
// hadamard_kernel's product bit for bit), so neither needs a launch.
__global__ void scale_columns_kernel(double* __restrict__ F, size_t rows, int R,
                                     const double* __restrict__ norms, double* __restrict__ z,
                                     size_t nz, const double* __restrict__ A,
                                     const double* __restrict__ B, double* __restrict__ C,
                                     size_t n2)
{
    const size_t total = rows * size_t(R);
    const size_t n = total > nz ? (total > n2 ? total : n2) : (nz > n2 ? nz : n2);
    for (size_t x = size_t(blockIdx.x) * blockDim.x + threadIdx.x; x < n;
         x += size_t(gridDim.x) * blockDim.x)
    {
        if (x < total)
        {
            const double nr = norms[x % size_t(R)];
            F[x] = (nr < 1e-14) ? 0.0 : F[x] / nr;
        }
        if (x < nz) z[x] = 0.0;
        if (x < n2) C[x] = A[x] * B[x];
    }
}

int scale_launch(double* F, size_t rows, int R, const double* norms, const cptc::TailJobs* t,
                 hipStream_t s)
{
    double* z = t ? t->zero : nullptr;
    const size_t nz = z ? t->nzero : 0;
    const bool had = t && t->ftf;
    const size_t n2 = had ? size_t(R) * R : 0;
    const size_t n = std::max({rows * size_t(R), nz, n2});
    if (n == 0) return CPTC_OK;
    hipLaunchKernelGGL(scale_columns_kernel, dim3(cptc::grid_for(n, 256, 4096)), dim3(256), 0, s,
                       F, rows, R, norms, z, nz, had ? t->ga : nullptr, had ? t->gb : nullptr,
                       had ? t->ftf : nullptr, n2);
    CPTC_LAUNCHED();
    return CPTC_OK;
}

// ---------------------------------------------------------------------------
// A small factor's whole update in one launch (rows <= UPD3_MAX_ROWS, R <=
// 16 NT <= 32) on the FP64 matrix cores (v_mfma_f64_16x16x4f64), the six
// launches of apply + Gram + norms + scaling (+ fit) in one:
//   F = (FtV Ainv) / lambda                      (apply_small_kernel)
//   G = F^T F; n_r = sqrt(G_rr); lambda_r *= n_r, 0 when n_r < 1e-14;
//   G_rs /= n_r n_s (0 at a tiny norm); FtF = G .* other when other is given
//                                                (gram_finish_small_kernel)
//   F[:, r] /= n_r (0 at a tiny norm)            (scale_columns_kernel)
// With fit_out (the iteration's last mode), also the Gram fit scalars of
// fit_finalize_kernel: fit_out[0] = sum_r lambda_r <F[:, r], FtV[:, r]>,
// fit_out[1] = sum_{r,s} lambda_r lambda_s G_0 G_1 G_2 [r][s] (grams holds
// G_0 and G_1; G_2 is this launch's G).  Last, Z[0, nz) is cleared (Z is
// FtV).
// Stage 1, every workgroup: wave w takes the 16-row block 4 blockIdx + w
// (and every 4 gridDim-th after it); the apply's accumulator element v of
// lane l is F[16 b + l / 16 + 4 v][16 t + l % 16], stored unscaled, and it
// is also the Gram's A operand (F^T, ranks 16 t .. + 15 against rows 16 b +
// 4 v .. + 3) and B operand, so the Gram partial needs no data movement;
// the workgroup's Gram (and, for the fit, per-rank <F, FtV>) partial goes
// to part[blockIdx] after the four waves' sums in wave order.  Stage 2, the
// workgroup that finishes last (a device counter taken after a release
// fence; no workgroup waits for another): the partials in workgroup order,
// the norms, lambda, G, FtF and the fit, then the factor scaled in place
// and FtV cleared (every workgroup's reads of FtV precede its count).  The
// last workgroup resets the counter, so launches on one device must not
// overlap (the library's scratch buffers have the same rule).  The sums run
// in the matrix cores' order, not the separate kernels'.
// ---------------------------------------------------------------------------
// Loads that may be padding are zeroed by an AND with a mask made opaque
// by an empty asm, not by a select: the compiler turns `cond ? load : 0`
// into a branch around the load, with a wait of its own per load.
__device__ __forceinline__ long long upd3_mask(bool keep)
{
    long long m = keep ? -1LL : 0LL;
    asm volatile("" : "+v"(m));
    return m;
}
__device__ __forceinline__ double upd3_and(double v, long long m)
{
    return __longlong_as_double(__double_as_longlong(v) & m);
}
// A value as an operand of an empty asm: a load before it cannot be moved
// past this point (placed where the load has completed anyway).
__device__ __forceinline__ double upd3_keep(double v)
{
    asm volatile("" : "+v"(v));
    return v;
}

// The pinv fast path of sweep_inverse_kernel run by one wave, with no
// workgroup barrier (the rest of the workgroup does other work meanwhile):
// A (R x R, row stride ld) read from LDS, lane l keeps row l % RT, columns
// C (l / RT) .. + C - 1 (C = RT^2 / 64), the pivot column goes through the
// LDS row colb (a wave's LDS accesses run in order).  Per entry the same
// operations as sweep_inverse_kernel, so an accepted inverse is the same
// bits.  Returns 1 with -(swept A) = A^-1 stored to Ainv, or 0 when a pivot
// is <= 1e-10 max diag (or not finite) or fast_inverse_ok fails: the
// caller then runs the Jacobi pseudoinverse.  Uniform over the wave.
template <int RT>
__device__ int sweep_wave(const double* As, int ld, int R, double* __restrict__ Ainv,
                          double* colb)
{
    constexpr int LPR = WAVE / RT;
    constexpr int C = RT / LPR;
    const int l = int(threadIdx.x) % WAVE;
    const int row = l % RT, part = l / RT, c0 = part * C;
    double a[C];
#pragma unroll
    for (int c = 0; c < C; ++c) a[c] = (row < R && c0 + c < R) ? As[row * ld + c0 + c] : 0.0;
    double md = 0.0, fa = 0.0;
#pragma unroll
    for (int c = 0; c < C; ++c)
    {
        if (c0 + c == row) md = a[c];
        fa += a[c] * a[c];
    }
#pragma unroll
    for (int o = WAVE / 2; o >= 1; o >>= 1)
    {
        md = fmax(md, __shfl_xor(md, o));
        fa += __shfl_xor(fa, o);
    }
    const double tau = 1e-10 * md;
    int ok = (md > 0.0 && isfinite(md)) ? 1 : 0;
#pragma unroll 1
    for (int kp = 0; kp < LPR && kp * C < R && ok; ++kp)
    {
#pragma unroll
        for (int kc = 0; kc < C; ++kc)
        {
            const int k = kp * C + kc;
            if (k >= R || !ok) continue;   // uniform
            if (part == kp) colb[row] = a[kc];
            __builtin_amdgcn_wave_barrier();
            const double p = colb[k];
            if (!(p > tau) || !isfinite(p))
            {
                ok = 0;
                continue;
            }
            const double ip = 1.0 / p;
            const double f = colb[row] * ip;
            const bool prow = row == k;
            const double g = prow ? 0.0 : f;
            const double h = prow ? ip : 1.0;
            double cj[C];
#pragma unroll
            for (int c = 0; c < C; ++c) cj[c] = colb[c0 + c];
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int c = 0; c < C; ++c)
            {
                const double up = fma(-g, cj[c], a[c] * h);
                a[c] = (c == kc && part == kp) ? (prow ? -ip : f) : up;
            }
        }
    }
    if (!ok) return 0;
    double fi = 0.0;
#pragma unroll
    for (int c = 0; c < C; ++c) fi += a[c] * a[c];
#pragma unroll
    for (int o = WAVE / 2; o >= 1; o >>= 1) fi += __shfl_xor(fi, o);
    if (!fast_inverse_ok(fa, fi, R)) return 0;
    if (row < R)
#pragma unroll
        for (int c = 0; c < C; ++c)
            if (c0 + c < R) Ainv[size_t(row) * R + c0 + c] = -a[c];
    return 1;
}

constexpr int UPD3_T = 256;
constexpr int UPD3_WAVES = UPD3_T / WAVE;
constexpr int UPD3_MAX_ROWS = 4096;
constexpr int UPD3_MAX_P = UPD3_MAX_ROWS / (16 * UPD3_WAVES);   // 64 workgroups
__device__ unsigned int upd3_count;   // zero at load; the last workgroup resets it

template <int NT>
__global__ __launch_bounds__(UPD3_T) void update3_small_kernel(
    const double* Y, const double* __restrict__ Ainv, double* F, int rows, int R,
    double* __restrict__ G, double* __restrict__ norms, double* lambda,
    const double* __restrict__ other, double* __restrict__ FtF, double* Z, int nz,
    const double* __restrict__ grams, double* __restrict__ fit_out, double* part,
    double* __restrict__ Anext, double* __restrict__ Vw)
{
    constexpr int NP = NT * (NT + 1) / 2;   // tile pairs (a <= c) of the Gram
    constexpr int KS = 4 * NT;              // K steps of 4 over R padded to 16 NT
    __shared__ double gl[UPD3_WAVES][NP][256];
    __shared__ double g_s[32][33], f_s[32][33];
    __shared__ double n_s[32], lamn_s[32], fit_s[UPD3_WAVES][32], fs_s[32], colb[32];
    __shared__ double red2[UPD3_WAVES];
    __shared__ int last_s, decl_s;
    const int tid = threadIdx.x, w = tid / WAVE, l = tid % WAVE;
    const int lr = l % 16, lk = l / 16;
    const int RR = R * R;
    const int P = int(gridDim.x);
    const int stride = R * (R + 1);   // one partial: RR Gram entries, then R fit sums
    // ---- stage 1 -------------------------------------------------------
    double bop[KS][NT];
#pragma unroll
    for (int kk = 0; kk < KS; ++kk)
#pragma unroll
        for (int t = 0; t < NT; ++t)
        {
            const int k = 4 * kk + lk, c = 16 * t + lr;
            bop[kk][t] = upd3_and(Ainv[min(k, R - 1) * R + min(c, R - 1)],
                                  upd3_mask(k < R && c < R));
        }
    // (padding columns: any divisor; their entries are not kept)
    double dv[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) dv[t] = lambda[min(16 * t + lr, R - 1)];
    const int nb = (rows + 15) / 16;
    gram_d4 gacc[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) gacc[p] = gram_d4{0.0, 0.0, 0.0, 0.0};
    double sp[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) sp[t] = 0.0;
    for (int blk = UPD3_WAVES * int(blockIdx.x) + w; blk < nb; blk += UPD3_WAVES * P)
    {
        const int row0 = 16 * blk;
        const int ar = min(row0 + lr, rows - 1);
        double aop[KS];
#pragma unroll
        for (int kk = 0; kk < KS; ++kk)
        {
            const int k = 4 * kk + lk;
            aop[kk] = upd3_and(Y[size_t(ar) * R + min(k, R - 1)],
                               upd3_mask(row0 + lr < rows && k < R));
        }
        // the fit's FtV entries at the accumulator's positions (loaded on
        // every path, pinned after the products; used only with fit_out)
        double ym[NT][4];
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int v = 0; v < 4; ++v)
                ym[t][v] = Y[size_t(min(row0 + lk + 4 * v, rows - 1)) * R +
                             min(16 * t + lr, R - 1)];
        gram_d4 f[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t)
        {
            gram_d4 acc = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
            for (int kk = 0; kk < KS; ++kk)
                acc = __builtin_amdgcn_mfma_f64_16x16x4f64(aop[kk], bop[kk][t], acc, 0, 0, 0);
            const int c = 16 * t + lr;
#pragma unroll
            for (int v = 0; v < 4; ++v)
            {
                const int row = row0 + lk + 4 * v;
                const bool in = row < rows && c < R;
                const double x = in ? acc[v] / dv[t] : 0.0;
                f[t][v] = x;
                if (in) F[size_t(row) * R + c] = x;
                const double y = upd3_keep(ym[t][v]);
                if (fit_out) sp[t] += in ? x * y : 0.0;
            }
        }
        int p = 0;
#pragma unroll
        for (int a = 0; a < NT; ++a)
#pragma unroll
            for (int c = a; c < NT; ++c, ++p)
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    gacc[p] = __builtin_amdgcn_mfma_f64_16x16x4f64(f[a][v], f[c][v], gacc[p], 0,
                                                                   0, 0);
    }
    // the workgroup's partial: Gram tiles summed in wave order, the upper
    // triangle mirrored (exactly symmetric), then the fit's per-rank sums
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int v = 0; v < 4; ++v) gl[w][p][(lk + 4 * v) * 16 + lr] = gacc[p][v];
    if (fit_out)
#pragma unroll
        for (int t = 0; t < NT; ++t)
        {
            sp[t] += __shfl_xor(sp[t], 16);
            sp[t] += __shfl_xor(sp[t], 32);
            if (lk == 0) fit_s[w][16 * t + lr] = sp[t];
        }
    __syncthreads();
    double* my = part + size_t(blockIdx.x) * stride;
    for (int x = tid; x < NP * 256; x += UPD3_T)
    {
        const int p = x / 256, e = x % 256, m = e / 16, n = e % 16;
        const int a = (p == 2) ? 1 : 0, c = (p == 0) ? 0 : 1;
        double s = 0.0;
#pragma unroll
        for (int q = 0; q < UPD3_WAVES; ++q) s += gl[q][p][e];
        const int i = 16 * a + m, j = 16 * c + n;
        if ((a != c || m <= n) && i < R && j < R)
        {
            my[i * R + j] = s;
            my[j * R + i] = s;
        }
    }
    if (fit_out && tid < R)
    {
        double s = 0.0;
#pragma unroll
        for (int q = 0; q < UPD3_WAVES; ++q) s += fit_s[q][tid];
        my[RR + tid] = s;
    }
    // every thread's stores (factor and partial) visible device-wide, then
    // one count per workgroup
    __threadfence();
    __syncthreads();
    if (tid == 0) last_s = (atomicAdd(&upd3_count, 1u) == unsigned(P - 1)) ? 1 : 0;
    __syncthreads();
    if (!last_s) return;
    // ---- stage 2: the last workgroup --------------------------------------
    __threadfence();   // acquire: the other workgroups' stores are seen
    // every load that does not depend on the sums is issued first: the
    // factor's first SB entries of this thread's column (scaling thread t:
    // column t % R, rows t / R + k rpp; with Anext wave 0 runs the sweep
    // instead and waves 1.. scale), the next FtF's other Gram and the fit's
    // two Grams (entries tid + q T, RR <= 4 T)
    constexpr int SB = 32;
    const int nsc = Anext ? UPD3_T - WAVE : UPD3_T;
    const int st = Anext ? tid - WAVE : tid;
    const int stc = st < 0 ? 0 : st;
    const int c0 = stc % R, rpp = nsc / R, r0 = stc / R;
    double fv[SB];
#pragma unroll
    for (int k = 0; k < SB; ++k) fv[k] = F[size_t(min(r0 + k * rpp, rows - 1)) * R + c0];
    // (a null operand reads the partials instead: valid memory, unused)
    const double* osrc = other ? other : part;
    const double* gsrc = fit_out ? grams : part;
    double ot[4], ga[4], gb[4];
#pragma unroll
    for (int q = 0; q < 4; ++q)
    {
        const int xc = min(tid + q * UPD3_T, RR - 1);
        ot[q] = osrc[xc];
        ga[q] = gsrc[xc];
        gb[q] = gsrc[(fit_out ? size_t(RR) : 0) + xc];
    }
    // partial sums in workgroup order: the thread's Gram entries tid + q T
    // (q < 4) and, for tid < R, the fit sum of rank tid; all loads of eight
    // partials issued together
    double gs[4] = {0.0, 0.0, 0.0, 0.0}, fsum = 0.0;
    for (int q0 = 0; q0 < P; q0 += 8)
    {
        double v[8][5];
#pragma unroll
        for (int u = 0; u < 8; ++u)
        {
            const double* pp = part + size_t(min(q0 + u, P - 1)) * stride;
#pragma unroll
            for (int q = 0; q < 4; ++q) v[u][q] = pp[min(tid + q * UPD3_T, RR - 1)];
            v[u][4] = pp[RR + min(tid, R - 1)];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u)
            if (q0 + u < P)
            {
#pragma unroll
                for (int q = 0; q < 4; ++q) gs[q] += v[u][q];
                fsum += fit_out ? v[u][4] : 0.0;
            }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q)
    {
        const int x = tid + q * UPD3_T;
        if (x < RR) g_s[x / R][x % R] = gs[q];
    }
    // the early loads, issued before the partials', have landed: pin them here
#pragma unroll
    for (int k = 0; k < SB; ++k) fv[k] = upd3_keep(fv[k]);
#pragma unroll
    for (int q = 0; q < 4; ++q)
    {
        ot[q] = upd3_keep(ot[q]);
        ga[q] = upd3_keep(ga[q]);
        gb[q] = upd3_keep(gb[q]);
    }
    __syncthreads();
    if (tid < R)
    {
        const double n = sqrt(g_s[tid][tid]);
        n_s[tid] = n;
        norms[tid] = n;
        const double lm = (n < 1e-14) ? 0.0 : lambda[tid] * n;
        lamn_s[tid] = lm;
        lambda[tid] = lm;
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 4; ++q)
    {
        const int x = tid + q * UPD3_T;
        if (x < RR)
        {
            const int i = x / R, j = x % R;
            const double ni = n_s[i], nj = n_s[j];
            const double v = (ni < 1e-14 || nj < 1e-14) ? 0.0 : g_s[i][j] / (ni * nj);
            g_s[i][j] = v;   // each entry read and written by its own thread only
            G[x] = v;
            if (other)
            {
                const double h = v * ot[q];
                FtF[x] = h;
                f_s[i][j] = h;
            }
        }
    }
    if (fit_out)   // uniform (a kernel argument)
    {
        // <F[:, r], FtV[:, r]> = <F_unscaled[:, r], FtV[:, r]> / n_r for the
        // fit wave, and this thread's share of model^2, per wave
        if (tid < R) fs_s[tid] = (n_s[tid] < 1e-14) ? 0.0 : fsum / n_s[tid];
        double md = 0.0;
#pragma unroll
        for (int q = 0; q < 4; ++q)
        {
            const int x = tid + q * UPD3_T;
            if (x < RR)
            {
                const int i = x / R, j = x % R;
                md += lamn_s[i] * lamn_s[j] * ga[q] * gb[q] * g_s[i][j];
            }
        }
#pragma unroll
        for (int o = WAVE / 2; o >= 1; o >>= 1) md += __shfl_xor(md, o);
        if (l == 0) red2[w] = md;
    }
    __syncthreads();   // FtF in f_s; the fit's sums
    if (st < 0)
    {
        // wave 0: the next mode's pinv (one-wave sweep)
        const int okp = sweep_wave<16 * NT>(&f_s[0][0], 33, R, Anext, colb);
        if (l == 0) decl_s = !okp;
    }
    else
    {
        if (fit_out && w == 1)
        {
            double ip = (l < R) ? lamn_s[l] * fs_s[l] : 0.0;
#pragma unroll
            for (int o = WAVE / 2; o >= 1; o >>= 1) ip += __shfl_xor(ip, o);
            if (l == 0)
            {
                double m2 = 0.0;
#pragma unroll
                for (int q = 0; q < UPD3_WAVES; ++q) m2 += red2[q];
                fit_out[0] = ip;
                fit_out[1] = m2;
            }
        }
        // the factor scaled in place, SB rows of the thread's column at a time
        if (r0 < rpp)
        {
            const double n = n_s[c0];
            const bool zero = n < 1e-14;
#pragma unroll
            for (int k = 0; k < SB; ++k)
            {
                const int i = r0 + k * rpp;
                if (i < rows) F[size_t(i) * R + c0] = zero ? 0.0 : fv[k] / n;
            }
            for (int i0 = r0 + SB * rpp; i0 < rows; i0 += SB * rpp)
            {
#pragma unroll
                for (int k = 0; k < SB; ++k)
                    fv[k] = F[size_t(min(i0 + k * rpp, rows - 1)) * R + c0];
#pragma unroll
                for (int k = 0; k < SB; ++k)
                {
                    const int i = i0 + k * rpp;
                    if (i < rows) F[size_t(i) * R + c0] = zero ? 0.0 : fv[k] / n;
                }
            }
        }
        for (int x = st; x < nz; x += nsc) Z[x] = 0.0;
    }
    if (Anext)   // uniform (a kernel argument)
    {
        __syncthreads();
        // a declined sweep: the Jacobi pseudoinverse of FtF by the whole
        // workgroup (A in the Gram tiles' LDS, V in global scratch)
        if (decl_s) jacobi_pinv_body<UPD3_T>(FtF, R, nullptr, Vw, Anext, 1, &gl[0][0][0]);
    }
    if (tid == 0) upd3_count = 0u;
}

// The same update in one workgroup of UPD1_T threads for rows <= 16
// UPD1_WAVES MAXB: no partials, counter or rescaling pass.  Wave w owns the
// blocks w, w + UPD1_WAVES, ... and keeps their factor entries in registers
// from the product to the scaled store; the waves' Gram tiles are summed in
// wave order.  All matrix-core work runs on one CU, so it is the form for a
// few hundred rows (two memory round trips instead of five).
constexpr int UPD1_T = 512;
constexpr int UPD1_WAVES = UPD1_T / WAVE;

template <int NT, int MAXB>
__global__ __launch_bounds__(UPD1_T) void update3_one_kernel(
    const double* Y, const double* __restrict__ Ainv, double* __restrict__ F, int rows, int R,
    double* __restrict__ G, double* __restrict__ norms, double* __restrict__ lambda,
    const double* __restrict__ other, double* __restrict__ FtF, double* Z, int nz,
    const double* __restrict__ grams, double* __restrict__ fit_out, double* __restrict__ Anext,
    double* __restrict__ Vw)
{
    constexpr int NP = NT * (NT + 1) / 2;
    constexpr int KS = 4 * NT;
    __shared__ double gl[UPD1_WAVES][NP][256];
    __shared__ double g_s[32][33], f_s[32][33];
    __shared__ double n_s[32], lamn_s[32], fit_s[UPD1_WAVES][32], colb[32];
    __shared__ double red2[UPD1_WAVES];
    __shared__ int decl_s;
    const int tid = threadIdx.x, w = tid / WAVE, l = tid % WAVE;
    const int lr = l % 16, lk = l / 16;
    const int RR = R * R;
    const int nb = (rows + 15) / 16;
    double bop[KS][NT];
#pragma unroll
    for (int kk = 0; kk < KS; ++kk)
#pragma unroll
        for (int t = 0; t < NT; ++t)
        {
            const int k = 4 * kk + lk, c = 16 * t + lr;
            bop[kk][t] = upd3_and(Ainv[min(k, R - 1) * R + min(c, R - 1)],
                                  upd3_mask(k < R && c < R));
        }
    double dv[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) dv[t] = lambda[min(16 * t + lr, R - 1)];
    // the next FtF's other Gram and the fit's two Grams (entries tid + q T,
    // RR <= 2 T); a null operand reads Ainv instead (valid, unused)
    const double* osrc = other ? other : Ainv;
    const double* gsrc = fit_out ? grams : Ainv;
    double ot[2], ga[2], gb[2];
#pragma unroll
    for (int q = 0; q < 2; ++q)
    {
        const int xc = min(tid + q * UPD1_T, RR - 1);
        ot[q] = osrc[xc];
        ga[q] = gsrc[xc];
        gb[q] = gsrc[(fit_out ? size_t(RR) : 0) + xc];
    }
    gram_d4 f[MAXB][NT];
    gram_d4 gacc[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) gacc[p] = gram_d4{0.0, 0.0, 0.0, 0.0};
    // A operands of every block the wave owns, loaded together
    double aop[MAXB][KS];
#pragma unroll
    for (int b = 0; b < MAXB; ++b)
    {
        const int row0 = 16 * (w + UPD1_WAVES * b);
        const int ar = max(0, min(row0 + lr, rows - 1));
#pragma unroll
        for (int kk = 0; kk < KS; ++kk)
        {
            const int k = 4 * kk + lk;
            aop[b][kk] = upd3_and(Y[size_t(ar) * R + min(k, R - 1)],
                                  upd3_mask(row0 + lr < rows && k < R));
        }
    }
#pragma unroll
    for (int b = 0; b < MAXB; ++b)
    {
        const int row0 = 16 * (w + UPD1_WAVES * b);
#pragma unroll
        for (int t = 0; t < NT; ++t) f[b][t] = gram_d4{0.0, 0.0, 0.0, 0.0};
        if (row0 >= rows) continue;   // uniform over the wave
#pragma unroll
        for (int t = 0; t < NT; ++t)
        {
            gram_d4 acc = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
            for (int kk = 0; kk < KS; ++kk)
                acc = __builtin_amdgcn_mfma_f64_16x16x4f64(aop[b][kk], bop[kk][t], acc, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 4; ++v)
                f[b][t][v] =
                    (row0 + lk + 4 * v < rows && 16 * t + lr < R) ? acc[v] / dv[t] : 0.0;
        }
        int p = 0;
#pragma unroll
        for (int a = 0; a < NT; ++a)
#pragma unroll
            for (int c = a; c < NT; ++c, ++p)
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    gacc[p] = __builtin_amdgcn_mfma_f64_16x16x4f64(f[b][a][v], f[b][c][v],
                                                                   gacc[p], 0, 0, 0);
    }
    // the fit's FtV entries at the accumulator positions, in flight during
    // the Gram's reduction (used only with fit_out)
    double ym[MAXB][NT][4];
#pragma unroll
    for (int b = 0; b < MAXB; ++b)
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int v = 0; v < 4; ++v)
                ym[b][t][v] = Y[size_t(max(0, min(16 * (w + UPD1_WAVES * b) + lk + 4 * v,
                                                  rows - 1))) * R +
                                min(16 * t + lr, R - 1)];
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int v = 0; v < 4; ++v) gl[w][p][(lk + 4 * v) * 16 + lr] = gacc[p][v];
    __syncthreads();
    for (int x = tid; x < NP * 256; x += UPD1_T)
    {
        const int p = x / 256, e = x % 256, m = e / 16, n = e % 16;
        const int a = (p == 2) ? 1 : 0, c = (p == 0) ? 0 : 1;
        double s = 0.0;
#pragma unroll
        for (int q = 0; q < UPD1_WAVES; ++q) s += gl[q][p][e];
        if (a != c || m <= n)
        {
            g_s[16 * a + m][16 * c + n] = s;
            g_s[16 * c + n][16 * a + m] = s;
        }
    }
    __syncthreads();
    if (tid < R)
    {
        const double n = sqrt(g_s[tid][tid]);
        n_s[tid] = n;
        norms[tid] = n;
        const double lm = (n < 1e-14) ? 0.0 : lambda[tid] * n;
        lamn_s[tid] = lm;
        lambda[tid] = lm;
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 2; ++q)
    {
        const int x = tid + q * UPD1_T;
        if (x < RR)
        {
            const int i = x / R, j = x % R;
            const double ni = n_s[i], nj = n_s[j];
            const double v = (ni < 1e-14 || nj < 1e-14) ? 0.0 : g_s[i][j] / (ni * nj);
            g_s[i][j] = v;   // each entry read and written by its own thread only
            G[x] = v;
            if (other)
            {
                const double h = v * ot[q];
                FtF[x] = h;
                f_s[i][j] = h;
            }
        }
    }
    double nr[NT], sp[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t)
    {
        nr[t] = (16 * t + lr < R) ? n_s[16 * t + lr] : 1.0;
        sp[t] = 0.0;
    }
#pragma unroll
    for (int b = 0; b < MAXB; ++b)
    {
        const int row0 = 16 * (w + UPD1_WAVES * b);
        if (row0 >= rows) continue;
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int v = 0; v < 4; ++v)
            {
                const int row = row0 + lk + 4 * v, c = 16 * t + lr;
                const double x = (nr[t] < 1e-14) ? 0.0 : f[b][t][v] / nr[t];
                const bool in = row < rows && c < R;
                if (in) F[size_t(row) * R + c] = x;
                if (fit_out) sp[t] += in ? x * ym[b][t][v] : 0.0;
            }
    }
    if (fit_out)   // uniform (a kernel argument)
    {
        // <F, FtV> per rank (the four lanes of a column, then per wave) and
        // this thread's share of model^2, per wave
#pragma unroll
        for (int t = 0; t < NT; ++t)
        {
            sp[t] += __shfl_xor(sp[t], 16);
            sp[t] += __shfl_xor(sp[t], 32);
            if (lk == 0) fit_s[w][16 * t + lr] = sp[t];
        }
        double md = 0.0;
#pragma unroll
        for (int q = 0; q < 2; ++q)
        {
            const int x = tid + q * UPD1_T;
            if (x < RR)
            {
                const int i = x / R, j = x % R;
                md += lamn_s[i] * lamn_s[j] * ga[q] * gb[q] * g_s[i][j];
            }
        }
#pragma unroll
        for (int o = WAVE / 2; o >= 1; o >>= 1) md += __shfl_xor(md, o);
        if (l == 0) red2[w] = md;
    }
    __syncthreads();   // FtF in f_s, the fit partials; every wave's FtV loads are consumed
    // wave 0: the next mode's pinv (one-wave sweep); wave 1: the fit
    // scalars; waves 2.. : FtV cleared for the next MTTKRP
    if (w == 0)
    {
        if (Anext)
        {
            const int okp = sweep_wave<16 * NT>(&f_s[0][0], 33, R, Anext, colb);
            if (l == 0) decl_s = !okp;
        }
    }
    else if (w == 1)
    {
        if (fit_out)
        {
            double ip = 0.0;
            if (l < R)
            {
                double sr = 0.0;
#pragma unroll
                for (int q = 0; q < UPD1_WAVES; ++q) sr += fit_s[q][l];
                ip = lamn_s[l] * sr;
            }
#pragma unroll
            for (int o = WAVE / 2; o >= 1; o >>= 1) ip += __shfl_xor(ip, o);
            if (l == 0)
            {
                double m2 = 0.0;
#pragma unroll
                for (int q = 0; q < UPD1_WAVES; ++q) m2 += red2[q];
                fit_out[0] = ip;
                fit_out[1] = m2;
            }
        }
    }
    else
    {
        for (int x = tid - 2 * WAVE; x < nz; x += UPD1_T - 2 * WAVE) Z[x] = 0.0;
    }
    if (Anext)   // uniform (a kernel argument)
    {
        __syncthreads();
        // a declined sweep: the Jacobi pseudoinverse of FtF by the whole
        // workgroup (A in the Gram tiles' LDS, V in global scratch)
        if (decl_s) jacobi_pinv_body<UPD1_T>(FtF, R, nullptr, Vw, Anext, 1, &gl[0][0][0]);
    }
}

int partials_for(size_t rows, size_t min_rows)
{
    size_t p = (rows + min_rows - 1) / min_rows;
    if (p < 1) p = 1;
    if (p > 256) p = 256;
    return int(p);
}

}  // namespace

extern "C" int cptc_gram(const double* d_F, size_t rows, int R, double* d_G, void* stream)
{
    CPTC_REQUIRE(R >= 1 && d_F && d_G, CPTC_ERR_ARG, "cptc_gram: bad arguments");
    hipStream_t s = cptc::as_stream(stream);
    const size_t RR = size_t(R) * R;
    if (rows == 0)
    {
        CPTC_HIP(hipMemsetAsync(d_G, 0, RR * sizeof(double), s));
        return CPTC_OK;
    }
    const int P = partials_for(rows, R > 64 ? CPTC_GRAM_MFMA_ROWS : 64);
    const size_t rpw = (rows + P - 1) / P;
    void* part = nullptr;
    CPTC_TRY(cptc::scratch_get(cptc::SCR_GRAM, size_t(P) * RR * sizeof(double), &part));
    double* pd = static_cast<double*>(part);
    if (R <= 16)
    {
        hipLaunchKernelGGL(gram_partial_kernel<1>, dim3(P, 1), dim3(256), 0, s, d_F, rows, R, rpw,
                           1, pd);
    }
    else if (R <= 32)
    {
        hipLaunchKernelGGL(gram_partial_kernel<2>, dim3(P, 1), dim3(256), 0, s, d_F, rows, R, rpw,
                           1, pd);
    }
    else if (R <= 64)
    {
        hipLaunchKernelGGL(gram_partial_kernel<4>, dim3(P, 1), dim3(256), 0, s, d_F, rows, R, rpw,
                           1, pd);
    }
    else
    {
        // the FP64 matrix cores over 64 x 64 tiles, upper triangle only
        const int nt = (R + 63) / 64;
        hipLaunchKernelGGL(gram_mfma_partial_kernel, dim3(P, nt * (nt + 1) / 2), dim3(256), 0, s,
                           d_F, rows, R, rpw, nt, pd);
        CPTC_LAUNCHED();
        hipLaunchKernelGGL(sum_partials_sym_kernel, dim3(cptc::grid_for(RR, 256, 1024)),
                           dim3(256), 0, s, pd, P, R, d_G);
        CPTC_LAUNCHED();
        return CPTC_OK;
    }
    CPTC_LAUNCHED();
    hipLaunchKernelGGL(sum_partials_kernel, dim3(cptc::grid_for(RR, 256, 1024)), dim3(256), 0, s,
                       pd, P, RR, d_G);
    CPTC_LAUNCHED();
    return CPTC_OK;
}

namespace cptc {

int gram_normalize_absorb_tail(double* d_F, size_t rows, int R, double* d_G, double* d_norms,
                               double* d_lambda, const TailJobs* t, hipStream_t s)
{
    CPTC_REQUIRE(R >= 1 && R <= FIT_T && d_F && d_G && d_norms && d_lambda, CPTC_ERR_ARG,
                 "cptc_gram_normalize_absorb: bad arguments");
    CPTC_TRY(cptc_gram(d_F, rows, R, d_G, s));
    hipLaunchKernelGGL(gram_norms_absorb_kernel, dim3(1), dim3(FIT_T), 0, s, d_G, R, d_norms,
                       d_lambda, nullptr, nullptr);
    CPTC_LAUNCHED();
    return scale_launch(d_F, rows, R, d_norms, t, s);
}

int gram_normalize_absorb_next_tail(double* d_F, size_t rows, int R, double* d_G,
                                    double* d_norms, double* d_lambda, const double* d_other,
                                    double* d_FtF, const TailJobs* t, hipStream_t s)
{
    CPTC_REQUIRE(R >= 1 && R <= FIT_T && d_F && d_G && d_norms && d_lambda && rows >= 1 &&
                     (d_other == nullptr) == (d_FtF == nullptr),
                 CPTC_ERR_ARG, "cptc_gram_normalize_absorb_next: bad arguments (R <= %d)", FIT_T);
    if (R > 32)
    {
        // cptc_gram, then the norms, normalisation and the next mode's FtF in
        // one launch (cptc_gram_normalize_absorb + cptc_hadamard, same bits)
        CPTC_TRY(cptc_gram(d_F, rows, R, d_G, s));
        hipLaunchKernelGGL(gram_norms_absorb_kernel, dim3(1), dim3(FIT_T), 0, s, d_G, R, d_norms,
                           d_lambda, d_other, d_FtF);
        CPTC_LAUNCHED();
        return scale_launch(d_F, rows, R, d_norms, t, s);
    }
    const size_t RR = size_t(R) * R;
    const int P = partials_for(rows, 64);
    const size_t rpw = (rows + P - 1) / P;
    void* part = nullptr;
    CPTC_TRY(cptc::scratch_get(cptc::SCR_GRAM, size_t(P) * RR * sizeof(double), &part));
    double* pd = static_cast<double*>(part);
    if (R <= 16)
        hipLaunchKernelGGL(gram_partial_kernel<1>, dim3(P, 1), dim3(256), 0, s, d_F, rows, R, rpw,
                           1, pd);
    else
        hipLaunchKernelGGL(gram_partial_kernel<2>, dim3(P, 1), dim3(256), 0, s, d_F, rows, R, rpw,
                           1, pd);
    CPTC_LAUNCHED();
    hipLaunchKernelGGL(gram_finish_small_kernel, dim3(1), dim3(FIT_T), 0, s, pd, P, R, d_G,
                       d_norms, d_lambda, d_other, d_FtF);
    CPTC_LAUNCHED();
    return scale_launch(d_F, rows, R, d_norms, t, s);
}

int update3_small(double* d_FtV, double* d_Ainv, double* d_F, size_t rows, int R, double* d_G,
                  double* d_norms, double* d_lambda, const double* d_other, double* d_FtF,
                  size_t nzero, const double* d_grams, double* d_fit, int next_pinv,
                  hipStream_t s)
{
    CPTC_REQUIRE(R >= 1 && R <= 32 && rows >= 1 && rows <= UPDATE3_SMALL_MAX_ROWS,
                 CPTC_ERR_ARG, "cptc_update_small3: rows %zu R %d (1..%zu rows, R <= 32)", rows,
                 R, UPDATE3_SMALL_MAX_ROWS);
    CPTC_REQUIRE(d_FtV && d_Ainv && d_F && d_G && d_norms && d_lambda &&
                     (d_other == nullptr) == (d_FtF == nullptr) && (!d_fit || d_grams) &&
                     (!next_pinv || d_FtF) && nzero < (size_t(1) << 31),
                 CPTC_ERR_ARG, "cptc_update_small3: bad arguments");
    static_assert(UPDATE3_SMALL_MAX_ROWS == size_t(UPD3_MAX_ROWS), "row limit");
    const int nb = int((rows + 15) / 16);
    const int P = (nb + UPD3_WAVES - 1) / UPD3_WAVES;   // one 16-row block per wave
    const size_t RR = size_t(R) * R;
    void* buf = nullptr;
    CPTC_TRY(cptc::scratch_get(cptc::SCR_GRAM, size_t(UPD3_MAX_P) * 32 * (32 + 1) * sizeof(double),
                               &buf));
    double* part = static_cast<double*>(buf);
    // the Jacobi fallback's V (pinv_launch's scratch layout: [work][V][flag])
    double* Vw = nullptr;
    double* Anext = next_pinv ? d_Ainv : nullptr;
    if (next_pinv)
    {
        void* pb = nullptr;
        CPTC_TRY(cptc::scratch_get(cptc::SCR_PINV, (2 * RR + 2) * sizeof(double), &pb));
        Vw = static_cast<double*>(pb) + RR;
    }
    const int nr = int(rows), nz = int(nzero);
    // one workgroup up to 256 rows, the multi-workgroup form above that
    // (CPTC_UPD3_ONE_ROWS overrides the limit, at most 512; 0 = never).
    // Per launch at R = 32: 256 rows 13.0 us in one workgroup against 15.0
    // in four; 512 rows 22.0 us against 19.2 in eight.
    static const int one_rows = [] {
        const char* e = std::getenv("CPTC_UPD3_ONE_ROWS");
        return e ? std::atoi(e) : 256;
    }();
    if (nr <= one_rows && nr <= 16 * UPD1_WAVES * 4)
    {
        const bool two = nr <= 16 * UPD1_WAVES * 2;
        auto go = [&](auto kern) {
            hipLaunchKernelGGL(kern, dim3(1), dim3(UPD1_T), 0, s, d_FtV, d_Ainv, d_F, nr, R, d_G,
                               d_norms, d_lambda, d_other, d_FtF, d_FtV, nz, d_grams, d_fit, Anext,
                               Vw);
        };
        if (R <= 16) two ? go(update3_one_kernel<1, 2>) : go(update3_one_kernel<1, 4>);
        else two ? go(update3_one_kernel<2, 2>) : go(update3_one_kernel<2, 4>);
        CPTC_LAUNCHED();
        return CPTC_OK;
    }
    if (R <= 16)
        hipLaunchKernelGGL(update3_small_kernel<1>, dim3(P), dim3(UPD3_T), 0, s, d_FtV, d_Ainv,
                           d_F, nr, R, d_G, d_norms, d_lambda, d_other, d_FtF, d_FtV, nz, d_grams,
                           d_fit, part, Anext, Vw);
    else
        hipLaunchKernelGGL(update3_small_kernel<2>, dim3(P), dim3(UPD3_T), 0, s, d_FtV, d_Ainv,
                           d_F, nr, R, d_G, d_norms, d_lambda, d_other, d_FtF, d_FtV, nz, d_grams,
                           d_fit, part, Anext, Vw);
    CPTC_LAUNCHED();
    return CPTC_OK;
}

}  // namespace cptc

extern "C" int cptc_update_small3(double* d_FtV, double* d_Ainv, double* d_F, size_t rows,
                                  int R, double* d_G, double* d_norms, double* d_lambda,
                                  const double* d_other, double* d_FtF, size_t nzero,
                                  const double* d_grams, double* d_fit, int next_pinv,
                                  void* stream)
{
    return cptc::update3_small(d_FtV, d_Ainv, d_F, rows, R, d_G, d_norms, d_lambda, d_other,
                               d_FtF, nzero, d_grams, d_fit, next_pinv, cptc::as_stream(stream));
}

extern "C" int cptc_gram_normalize_absorb(double* d_F, size_t rows, int R, double* d_G,
                                          double* d_norms, double* d_lambda, void* stream)
{
    return cptc::gram_normalize_absorb_tail(d_F, rows, R, d_G, d_norms, d_lambda, nullptr,
                                            cptc::as_stream(stream));
}

extern "C" int cptc_gram_normalize_absorb_next(double* d_F, size_t rows, int R, double* d_G,
                                               double* d_norms, double* d_lambda,
                                               const double* d_other, double* d_FtF, void* stream)
{
    return cptc::gram_normalize_absorb_next_tail(d_F, rows, R, d_G, d_norms, d_lambda, d_other,
                                                 d_FtF, nullptr, cptc::as_stream(stream));
}

extern "C" int cptc_zero(double* d_p, size_t n, void* stream)
{
    if (n == 0) return CPTC_OK;
    CPTC_REQUIRE(d_p, CPTC_ERR_ARG, "cptc_zero: null pointer");
    hipLaunchKernelGGL(zero_kernel, dim3(cptc::grid_for(n, 256, 2048)), dim3(256), 0,
                       cptc::as_stream(stream), d_p, n);
    CPTC_LAUNCHED();
    return CPTC_OK;
}

extern "C" int cptc_hadamard(const double* d_A, const double* d_B, double* d_C, size_t n,
                             void* stream)
{
    CPTC_REQUIRE(d_A && d_B && d_C, CPTC_ERR_ARG, "cptc_hadamard: null pointer");
    if (n == 0) return CPTC_OK;
    hipLaunchKernelGGL(hadamard_kernel, dim3(cptc::grid_for(n, 256, 4096)), dim3(256), 0,
                       cptc::as_stream(stream), d_A, d_B, d_C, n);
    CPTC_LAUNCHED();
    return CPTC_OK;
}

namespace {
// The pinv kernels on caller-provided workspace: work (R x R, the matrix in
// global memory; read only when R > 128), V (R x R Jacobi eigenvectors) and
// flag (the path: 0 fast, 1 Jacobi).
int pinv_launch_ws(const double* d_FtF, double* d_Ainv, int R, int* flag, double* work,
                   double* V, hipStream_t s)
{
    const size_t RR = size_t(R) * R;
    const bool use_lds = RR * sizeof(double) <= 128 * 1024;
    const size_t lds = use_lds ? RR * sizeof(double) : 0;
    static cptc::DeviceOnce attr;
    CPTC_HIP(attr.lds_limit({reinterpret_cast<const void*>(chol_inverse_kernel),
                             reinterpret_cast<const void*>(jacobi_pinv_kernel)},
                            128 * 1024));
    // R <= 64: the sweep kernel runs its own Jacobi fallback (one launch)
    if (R <= 16)
        hipLaunchKernelGGL(sweep_inverse_kernel<16>, dim3(1), dim3(SWEEP_T), 0, s, d_FtF, R, d_Ainv,
                           flag, V);
    else if (R <= 32)
        hipLaunchKernelGGL(sweep_inverse_kernel<32>, dim3(1), dim3(SWEEP_T), 0, s, d_FtF, R, d_Ainv,
                           flag, V);
    else if (R <= 64)
        hipLaunchKernelGGL(sweep_inverse_kernel<64>, dim3(1), dim3(SWEEP_T), 0, s, d_FtF, R, d_Ainv,
                           flag, V);
    else
    {
        hipLaunchKernelGGL(chol_inverse_kernel, dim3(1), dim3(PINV_THREADS), lds, s, d_FtF, R,
                           work, d_Ainv, flag, int(use_lds));
        CPTC_LAUNCHED();
        hipLaunchKernelGGL(jacobi_pinv_kernel, dim3(1), dim3(PINV_THREADS), lds, s, d_FtF, R, work,
                           V, d_Ainv, flag, int(use_lds));
    }
    CPTC_LAUNCHED();
    return CPTC_OK;
}

int pinv_launch(const double* d_FtF, double* d_Ainv, int R, int* d_path, hipStream_t s)
{
    const size_t RR = size_t(R) * R;
    // scratch: [work RR (global A when R > 128)] [V RR] [flag]
    void* buf = nullptr;
    CPTC_TRY(cptc::scratch_get(cptc::SCR_PINV, (2 * RR + 2) * sizeof(double), &buf));
    double* work = static_cast<double*>(buf);
    double* V = work + RR;
    int* flag = d_path ? d_path : reinterpret_cast<int*>(V + RR);
    return pinv_launch_ws(d_FtF, d_Ainv, R, flag, work, V, s);
}

int apply_launch(const double* d_FtV, const double* d_Ainv, double* d_F, size_t dim, int R,
                 const double* d_div, hipStream_t s)
{
    if (dim == 0) return CPTC_OK;
    if (R <= APPLY_SMALL_R)
    {
        const unsigned grid = cptc::grid_for(dim * size_t(R), 256, 4096);
        hipLaunchKernelGGL(apply_small_kernel, dim3(grid), dim3(256), 0, s, d_FtV, d_Ainv, d_F,
                           dim, R, d_div);
    }
    else
    {
        CPTC_REQUIRE((dim + 15) / 16 < (size_t(1) << 31), CPTC_ERR_ARG, "apply: %zu rows", dim);
        const dim3 grid{unsigned((dim + 15) / 16), unsigned((R + 127) / 128)};
        hipLaunchKernelGGL(apply_mfma_kernel, grid, dim3(256), 0, s, d_FtV, d_Ainv, d_F, dim, R,
                           d_div);
    }
    CPTC_LAUNCHED();
    return CPTC_OK;
}
}  // namespace

extern "C" int cptc_pinv_sym(const double* d_FtF, double* d_Ainv, int R, int* d_path,
                             void* stream)
{
    CPTC_REQUIRE(R >= 1 && R <= 512 && d_FtF && d_Ainv, CPTC_ERR_ARG,
                 "cptc_pinv_sym: bad arguments (R %d, supported 1..512)", R);
    return pinv_launch(d_FtF, d_Ainv, R, d_path, cptc::as_stream(stream));
}

extern "C" int cptc_solve_pinv(const double* d_FtF, const double* d_FtV, double* d_F, size_t dim,
                               int R, const double* d_div, void* stream)
{
    CPTC_REQUIRE(R >= 1 && R <= 512 && d_FtF && d_FtV && d_F, CPTC_ERR_ARG,
                 "cptc_solve_pinv: bad arguments (R %d, supported 1..512)", R);
    hipStream_t s = cptc::as_stream(stream);
    void* buf = nullptr;
    CPTC_TRY(cptc::scratch_get(cptc::SCR_FLAGS, size_t(R) * R * sizeof(double) + 64, &buf));
    double* Ainv = static_cast<double*>(buf);
    CPTC_TRY(pinv_launch(d_FtF, Ainv, R, nullptr, s));
    return apply_launch(d_FtV, Ainv, d_F, dim, R, d_div, s);
}

// ---------------------------------------------------------------------------
// Allocation-free solve.  The solve's workspace lives in `scratch`, a
// file-scope device array that every GPU the library runs on holds until the
// process ends: [Ainv: NOALLOC_MAX_R^2 doubles] [V: NOALLOC_MAX_R^2 doubles]
// [path flag].  Host code never passes `scratch` itself (in host code the
// name is a host-side stand-in, not a device address): the first call on a
// device takes the device address with hipGetSymbolAddress and keeps it per
// device.  Nothing needs clearing between calls (the fast kernel writes the
// flag before the Jacobi kernel reads it; Ainv and V are written before they
// are read).  Calls that overlap on one GPU share the array and race.
// ---------------------------------------------------------------------------
namespace {
constexpr int NOALLOC_MAX_R = 128;
constexpr size_t NOALLOC_RR = size_t(NOALLOC_MAX_R) * NOALLOC_MAX_R;
constexpr int NOALLOC_MAX_DEV = 64;
static_assert(NOALLOC_RR * sizeof(double) <= 128 * 1024, "R <= 128 keeps the matrix in LDS");

static __device__ __align__(256) double scratch[2 * NOALLOC_RR + 32];

std::mutex g_scratch_mu;
double* g_scratch_ptr[NOALLOC_MAX_DEV] = {};

int noalloc_scratch(double** out)
{
    int dev = 0;
    CPTC_HIP(hipGetDevice(&dev));
    CPTC_REQUIRE(dev >= 0 && dev < NOALLOC_MAX_DEV, CPTC_ERR_ARG,
                 "cptc_solve_pinv_noalloc: device %d beyond %d", dev, NOALLOC_MAX_DEV);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev])
    {
        void* p = nullptr;
        CPTC_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        CPTC_REQUIRE(p != nullptr, CPTC_ERR_HIP, "cptc_solve_pinv_noalloc: no scratch address");
        g_scratch_ptr[dev] = static_cast<double*>(p);
    }
    *out = g_scratch_ptr[dev];
    return CPTC_OK;
}
}  // namespace

extern "C" int cptc_solve_pinv_noalloc(const double* d_FtF, const double* d_FtV, double* d_F,
                                       size_t dim, int R, const double* d_div, void* stream)
{
    CPTC_REQUIRE(R >= 1 && d_FtF && d_FtV && d_F, CPTC_ERR_ARG,
                 "cptc_solve_pinv_noalloc: bad arguments");
    CPTC_REQUIRE(R <= NOALLOC_MAX_R, CPTC_ERR_ARG,
                 "cptc_solve_pinv_noalloc: R = %d exceeds the allocation-free maximum %d "
                 "(use cptc_solve_pinv)", R, NOALLOC_MAX_R);
    hipStream_t s = cptc::as_stream(stream);
    double* ws = nullptr;
    CPTC_TRY(noalloc_scratch(&ws));
    double* Ainv = ws;
    double* V = ws + NOALLOC_RR;
    int* flag = reinterpret_cast<int*>(ws + 2 * NOALLOC_RR);
    // R <= 128: the kernels keep the matrix in LDS and never read `work`
    CPTC_TRY(pinv_launch_ws(d_FtF, Ainv, R, flag, V, V, s));
    return apply_launch(d_FtV, Ainv, d_F, dim, R, d_div, s);
}

extern "C" int cptc_apply_pinv(const double* d_FtV, const double* d_Ainv, double* d_F,
                               size_t dim, int R, const double* d_div, void* stream)
{
    CPTC_REQUIRE(R >= 1 && R <= 512 && d_FtV && d_Ainv && d_F, CPTC_ERR_ARG,
                 "cptc_apply_pinv: bad arguments (R %d, supported 1..512)", R);
    return apply_launch(d_FtV, d_Ainv, d_F, dim, R, d_div, cptc::as_stream(stream));
}

namespace {
int col_reduce(const double* F, const double* M, size_t rows, int R, hipStream_t s, double** part,
               int* P_out)
{
    // up to 256 workgroups of >= 64 rows (113 of 256 rows left the column
    // sums of a 28818-row factor latency-bound at 46 us)
    const int P = partials_for(rows, 64);
    const size_t rpw = (rows + P - 1) / P;
    void* buf = nullptr;
    CPTC_TRY(cptc::scratch_get(cptc::SCR_REDUCE, size_t(P) * R * sizeof(double), &buf));
    double* pd = static_cast<double*>(buf);
    hipLaunchKernelGGL(col_partial_kernel, dim3(P), dim3(256), 0, s, F, M, rows, R, rpw, pd);
    CPTC_LAUNCHED();
    *part = pd;
    *P_out = P;
    return CPTC_OK;
}
}  // namespace

extern "C" int cptc_colnorms(const double* d_F, size_t rows, int R, double* d_norms, void* stream)
{
    CPTC_REQUIRE(R >= 1 && d_F && d_norms, CPTC_ERR_ARG, "cptc_colnorms: bad arguments");
    hipStream_t s = cptc::as_stream(stream);
    double* part = nullptr;
    int P = 0;
    CPTC_TRY(col_reduce(d_F, nullptr, rows, R, s, &part, &P));
    hipLaunchKernelGGL(norms_finalize_kernel, dim3(1), dim3(256), 0, s, part, P, R, d_norms);
    CPTC_LAUNCHED();
    return CPTC_OK;
}

extern "C" int cptc_normalize_absorb(double* d_F, size_t rows, int R, const double* d_norms,
                                     double* d_lambda, void* stream)
{
    CPTC_REQUIRE(R >= 1 && d_F && d_norms && d_lambda, CPTC_ERR_ARG,
                 "cptc_normalize_absorb: bad arguments");
    const size_t n = rows * size_t(R);
    hipLaunchKernelGGL(normalize_absorb_kernel, dim3(cptc::grid_for(n, 256, 4096)), dim3(256), 0,
                       cptc::as_stream(stream), d_F, rows, R, d_norms, d_lambda);
    CPTC_LAUNCHED();
    return CPTC_OK;
}

extern "C" int cptc_fit_gram(const double* d_F, const double* d_M, size_t rows,
                             const double* d_lambda, const double* d_grams, int ngram, int R,
                             double* d_out2, void* stream)
{
    CPTC_REQUIRE(R >= 1 && d_F && d_M && d_lambda && d_grams && d_out2 && ngram >= 1,
                 CPTC_ERR_ARG, "cptc_fit_gram: bad arguments");
    hipStream_t s = cptc::as_stream(stream);
    double* part = nullptr;
    int P = 0;
    CPTC_REQUIRE(R <= FIT_T, CPTC_ERR_ARG, "cptc_fit_gram: R %d > %d", R, FIT_T);
    CPTC_TRY(col_reduce(d_F, d_M, rows, R, s, &part, &P));
    hipLaunchKernelGGL(fit_finalize_kernel, dim3(1), dim3(FIT_T), 0, s, part, P, R, d_lambda,
                       d_grams, ngram, d_out2);
    CPTC_LAUNCHED();
    return CPTC_OK;
}

namespace {

__global__ void clamp_kernel(double* __restrict__ x, size_t n, double lo, double hi)
{
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
        x[i] = x[i] < lo ? lo : (x[i] > hi ? hi : x[i]);
}

}  // namespace

extern "C" int cptc_clamp(double* d_x, size_t n, double lo, double hi, void* stream)
{
    if (n == 0) return CPTC_OK;
    CPTC_REQUIRE(d_x && lo <= hi, CPTC_ERR_ARG, "cptc_clamp: null pointer or lo > hi");
    hipLaunchKernelGGL(clamp_kernel, dim3(cptc::grid_for(n, 256, 4096)), dim3(256), 0,
                       cptc::as_stream(stream), d_x, n, lo, hi);
    CPTC_LAUNCHED();
    return CPTC_OK;
}
