// Kernels of the generic N-order CP-ALS path for CDNA4 (wave64): the FP64
// segment MTTKRP, dense-unit packing and outer weights, the Gram Hadamard,
// the ridge Cholesky solve, column normalisation and the exact residual.
// The dense-unit MFMA contraction shares dense_tiles.hip with order 3.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "../host/hip_util.hpp"

namespace {

constexpr int WAVE = 64;
constexpr int MAXM = CPTC_MAX_MODES;

struct Factors
{
    const double* p[MAXM];
};

template <int VEC>
struct Row;
template <>
struct Row<2>
{
    double x[2];
    __device__ void load(const double* __restrict__ q)
    {
        const double2 v = *reinterpret_cast<const double2*>(q);
        x[0] = v.x;
        x[1] = v.y;
    }
};
template <>
struct Row<1>
{
    double x[1];
    __device__ void load(const double* __restrict__ q) { x[0] = *q; }
};

// ------------------------------------------------------ segment MTTKRP --
//
// One workgroup (4 waves) per row segment.  A lane owns VEC consecutive
// ranks; LPE = RT / VEC lanes cover one element, so a wave carries
// EPW = 64 / LPE element slots (R = 32 -> 4, 16 -> 8, 8 -> 16).  Each slot
// walks a contiguous chunk of the segment.
//
// The segment's other coordinates come in NO = N - 1 levels (the view's row
// order, G[q] = factor of level q).  The slot evaluates the sum as a tree
// over equal coordinate prefixes (the CSF form of the MTTKRP):
//   acc = sum_{o0} G0[o0] * sum_{o1} G1[o1] * ... * sum_{o_last} v * G_last[o_last]
// t[k] holds the open partial sum under the current prefix o0..ok; when
// o_k changes, levels deeper than k-1 are closed (t[k] * G_k[cur_k] is
// added one level up).  Each factor row is therefore gathered once per run
// of its prefix; in a view without runs this is one gather per level per
// element, the plain product.  Skipped (dense) elements touch nothing.
template <int N, int RT, int VEC, int UNROLL>
__global__ __launch_bounds__(256) void seg_nd_kernel(
    Factors F, const uint32_t* __restrict__ sc, uint64_t nnz,
    const double* __restrict__ vals, const uint8_t* __restrict__ skip,
    const uint32_t* __restrict__ seg_row, const uint32_t* __restrict__ seg_start,
    const uint32_t* __restrict__ seg_cnt, const uint8_t* __restrict__ single,
    double* __restrict__ FtV, int R)
{
    constexpr int NO = N - 1;                // levels
    constexpr int NL = (NO > 1) ? NO - 1 : 1; // run levels (0 .. NO-2)
    constexpr int LPE = RT / VEC;
    constexpr int EPW = WAVE / LPE;
    constexpr int WAVES = 4;
    constexpr int SLOTS = EPW * WAVES;

    const uint32_t seg = blockIdx.x;
    const uint32_t row = seg_row[seg];
    const uint32_t start = seg_start[seg];
    const uint32_t cnt = seg_cnt[seg];

    const int tid = threadIdx.x;
    const int lane = tid & (WAVE - 1);
    const int wave = tid / WAVE;
    const int slot = lane / LPE;
    const int r0 = (lane % LPE) * VEC;
    const bool rank_ok = r0 < R;
    const int rr = rank_ok ? r0 : 0;

    const uint32_t g = uint32_t(wave * EPW + slot);
    const uint32_t chunk = (cnt + SLOTS - 1) / SLOTS;
    uint32_t lo = start + g * chunk;
    const uint32_t hi = (g * chunk + chunk < cnt) ? lo + chunk : start + cnt;
    if (lo > hi) lo = hi;

    double acc[VEC];
    double t[NL][VEC];
    uint32_t cur[NL];
#pragma unroll
    for (int k = 0; k < VEC; ++k) acc[k] = 0.0;
#pragma unroll
    for (int l = 0; l < NL; ++l)
    {
        cur[l] = 0;
#pragma unroll
        for (int k = 0; k < VEC; ++k) t[l][k] = 0.0;
    }
    bool open = false;

    // close run levels from NO-2 down to `to` (all of them when to == 0)
    auto close_levels = [&](int to) {
#pragma unroll
        for (int l = NL - 1; l >= 0; --l)
        {
            if (l < to) break;
            Row<VEC> f;
            f.load(F.p[l] + size_t(cur[l]) * R + rr);
#pragma unroll
            for (int k = 0; k < VEC; ++k)
            {
                const double x = t[l][k] * f.x[k];
                if (l == 0)
                    acc[k] += x;
                else
                    t[l - 1][k] += x;
                t[l][k] = 0.0;
            }
        }
    };

    // one live element: coordinates o[0..NO-1], value-weighted last-level row p
    auto consume = [&](const uint32_t* o, const double* p) {
        if constexpr (NO == 1)
        {
#pragma unroll
            for (int k = 0; k < VEC; ++k) acc[k] += p[k];
        }
        else
        {
            int L = NL;
            if (!open)
            {
                L = 0;
                open = true;
            }
            else
            {
#pragma unroll
                for (int l = NL - 1; l >= 0; --l)
                    if (o[l] != cur[l]) L = l;
                if (L < NL) close_levels(L);
            }
#pragma unroll
            for (int l = 0; l < NL; ++l)
                if (l >= L) cur[l] = o[l];
#pragma unroll
            for (int k = 0; k < VEC; ++k) t[NL - 1][k] += p[k];
        }
    };

    uint32_t e = lo;
    for (; e + UNROLL <= hi; e += UNROLL)
    {
        uint32_t c[UNROLL][NO];
        double v[UNROLL];
        bool live[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u)
        {
            v[u] = __builtin_nontemporal_load(vals + e + u);
            live[u] = skip ? (__builtin_nontemporal_load(skip + e + u) == 0) : true;
#pragma unroll
            for (int q = 0; q < NO; ++q) c[u][q] = __builtin_nontemporal_load(sc + q * nnz + e + u);
        }
        double p[UNROLL][VEC];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u)
        {
            Row<VEC> f;
            if (live[u])
                f.load(F.p[NO - 1] + size_t(c[u][NO - 1]) * R + rr);
#pragma unroll
            for (int k = 0; k < VEC; ++k) p[u][k] = live[u] ? v[u] * f.x[k] : 0.0;
        }
#pragma unroll
        for (int u = 0; u < UNROLL; ++u)
            if (live[u]) consume(c[u], p[u]);
    }
    for (; e < hi; ++e)
    {
        if (skip && __builtin_nontemporal_load(skip + e) != 0) continue;
        uint32_t c[NO];
#pragma unroll
        for (int q = 0; q < NO; ++q) c[q] = __builtin_nontemporal_load(sc + q * nnz + e);
        const double v = __builtin_nontemporal_load(vals + e);
        Row<VEC> f;
        f.load(F.p[NO - 1] + size_t(c[NO - 1]) * R + rr);
        double p[VEC];
#pragma unroll
        for (int k = 0; k < VEC; ++k) p[k] = v * f.x[k];
        consume(c, p);
    }
    if constexpr (NO > 1)
        if (open) close_levels(0);
    if (!rank_ok)
#pragma unroll
        for (int k = 0; k < VEC; ++k) acc[k] = 0.0;

#pragma unroll
    for (int off = LPE; off < WAVE; off <<= 1)
#pragma unroll
        for (int k = 0; k < VEC; ++k) acc[k] += __shfl_xor(acc[k], off, WAVE);

    __shared__ double red[WAVES][RT];
    if (slot == 0)
#pragma unroll
        for (int k = 0; k < VEC; ++k) red[wave][r0 + k] = acc[k];
    __syncthreads();
    const bool store = single && single[seg] != 0;
    for (int x = tid; x < R; x += WAVE * WAVES)
    {
        double tot = 0.0;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) tot += red[w][x];
        double* out = FtV + size_t(row) * R + x;
        if (store)
            *out = tot;
        else if (tot != 0.0)
            atomicAdd(out, tot);
    }
}

template <int N, int RT, int VEC>
void launch_seg(const Factors& F, int mode, const uint32_t* sc, uint64_t nnz, const double* vals,
                const uint8_t* skip, const uint32_t* row, const uint32_t* st, const uint32_t* cn,
                const uint8_t* single, uint64_t nseg, double* FtV, int R, hipStream_t s)
{
    (void)mode;
    constexpr int UNROLL = (N <= 4) ? 4 : 2;
    hipLaunchKernelGGL((seg_nd_kernel<N, RT, VEC, UNROLL>), dim3(unsigned(nseg)), dim3(256), 0, s,
                       F, sc, nnz, vals, skip, row, st, cn, single, FtV, R);
}

template <int N, int VEC>
void launch_seg_r(const Factors& F, int mode, const uint32_t* sc, uint64_t nnz,
                  const double* vals, const uint8_t* skip, const uint32_t* row, const uint32_t* st,
                  const uint32_t* cn, const uint8_t* single, uint64_t nseg, double* FtV, int R,
                  hipStream_t s)
{
    if (R <= 8)
        launch_seg<N, 8, VEC>(F, mode, sc, nnz, vals, skip, row, st, cn, single, nseg, FtV, R, s);
    else if (R <= 16)
        launch_seg<N, 16, VEC>(F, mode, sc, nnz, vals, skip, row, st, cn, single, nseg, FtV, R, s);
    else
        launch_seg<N, 32, VEC>(F, mode, sc, nnz, vals, skip, row, st, cn, single, nseg, FtV, R, s);
}

template <int VEC>
void launch_seg_n(int N, const Factors& F, int mode, const uint32_t* sc, uint64_t nnz,
                  const double* vals, const uint8_t* skip, const uint32_t* row,
                  const uint32_t* st, const uint32_t* cn, const uint8_t* single, uint64_t nseg,
                  double* FtV, int R, hipStream_t s)
{
    switch (N)
    {
    case 2: launch_seg_r<2, VEC>(F, mode, sc, nnz, vals, skip, row, st, cn, single, nseg, FtV, R, s); break;
    case 3: launch_seg_r<3, VEC>(F, mode, sc, nnz, vals, skip, row, st, cn, single, nseg, FtV, R, s); break;
    case 4: launch_seg_r<4, VEC>(F, mode, sc, nnz, vals, skip, row, st, cn, single, nseg, FtV, R, s); break;
    case 5: launch_seg_r<5, VEC>(F, mode, sc, nnz, vals, skip, row, st, cn, single, nseg, FtV, R, s); break;
    case 6: launch_seg_r<6, VEC>(F, mode, sc, nnz, vals, skip, row, st, cn, single, nseg, FtV, R, s); break;
    case 7: launch_seg_r<7, VEC>(F, mode, sc, nnz, vals, skip, row, st, cn, single, nseg, FtV, R, s); break;
    default: launch_seg_r<8, VEC>(F, mode, sc, nnz, vals, skip, row, st, cn, single, nseg, FtV, R, s); break;
    }
}

// ------------------------------------------------------------ dense units --

// One workgroup per unit: FP64 accumulation in LDS (duplicates summed), one
// rounding to FP32 per cell.
__global__ __launch_bounds__(256) void units_pack_kernel(const uint32_t* __restrict__ unit6,
                                                         const uint32_t* __restrict__ lid,
                                                         const double* __restrict__ val,
                                                         float* __restrict__ tiles)
{
    __shared__ double T[4096];
    const size_t u = blockIdx.x;
    for (int c = threadIdx.x; c < 4096; c += 256) T[c] = 0.0;
    __syncthreads();
    const uint32_t n = unit6[6 * u + 3], st = unit6[6 * u + 4];
    for (uint32_t e = threadIdx.x; e < n; e += 256) atomicAdd(&T[lid[st + e] & 4095u], val[st + e]);
    __syncthreads();
    float4* out = reinterpret_cast<float4*>(tiles + u * 4096);
    for (int c = threadIdx.x; c < 1024; c += 256)
        out[c] = make_float4(float(T[4 * c]), float(T[4 * c + 1]), float(T[4 * c + 2]),
                             float(T[4 * c + 3]));
}

// The same cells in FP64 (the per-unit sums' operand): one workgroup per
// unit, FP64 accumulation in LDS (duplicates summed), written as doubles.
__global__ __launch_bounds__(256) void units_pack_f64_kernel(const uint32_t* __restrict__ unit6,
                                                             const uint32_t* __restrict__ lid,
                                                             const double* __restrict__ val,
                                                             double* __restrict__ img)
{
    __shared__ double T[4096];
    const size_t u = blockIdx.x;
    for (int c = threadIdx.x; c < 4096; c += 256) T[c] = 0.0;
    __syncthreads();
    const uint32_t n = unit6[6 * u + 3], st = unit6[6 * u + 4];
    for (uint32_t e = threadIdx.x; e < n; e += 256) atomicAdd(&T[lid[st + e] & 4095u], val[st + e]);
    __syncthreads();
    double2* out = reinterpret_cast<double2*>(img + u * 4096);
    for (int c = threadIdx.x; c < 2048; c += 256) out[c] = make_double2(T[2 * c], T[2 * c + 1]);
}

__global__ void units_weights_kernel(const uint32_t* __restrict__ unit6, uint64_t nunits,
                                     const uint32_t* __restrict__ oc, int nouter, Factors Fo,
                                     int R, double* __restrict__ W)
{
    const uint64_t total = nunits * uint64_t(R);
    const uint64_t stride = uint64_t(gridDim.x) * blockDim.x;
    for (uint64_t x = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; x < total; x += stride)
    {
        const uint64_t u = x / R;
        const int r = int(x % R);
        const uint32_t off = unit6[6 * u + 5];
        double w = 1.0;
#pragma unroll
        for (int k = 0; k < MAXM; ++k)
            if (k < nouter) w *= Fo.p[k][size_t(oc[off + k]) * R + r];
        W[x] = w;
    }
}

// ------------------------------------------------------------- small R x R --

__global__ void gram_hadamard_kernel(const double* __restrict__ G, int ngram, int skip, int RR,
                                     double* __restrict__ out)
{
    for (int x = blockIdx.x * blockDim.x + threadIdx.x; x < RR; x += gridDim.x * blockDim.x)
    {
        double v = 1.0;
        for (int g = 0; g < ngram; ++g)
            if (g != skip) v *= G[size_t(g) * RR + x];
        out[x] = v;
    }
}

// Ridge Cholesky + per-row substitution (generic.cu:746-819), in two
// kernels so that a driver can factor FtF while the MTTKRP that produces
// FtV is still running.
//
// chol_factor_kernel (four waves) factors FtF + eps I in registers: row i
// is split over 256 / RT threads, each holding RT^2 / 256 consecutive
// columns.  Step j broadcasts the pivot column through LDS, scales column j
// by the pivot's square root (the thread owning column j of each row) and
// every thread subtracts L[i][j] L[k][j] from its entries k > j.  Each entry
// therefore receives exactly the reference's sequence: (FtF + eps) minus
// the products for k = 0, 1, ... in ascending order, then the division by
// the pivot.  Entries above the diagonal take the same updates without a
// per-thread condition (they are never read).  L (R x R row-major, zeros
// above the diagonal) goes to global.
//
// chol_apply_kernel stages L in LDS and solves one right-hand-side row per
// lane with its y / x vector in registers (loops unrolled to RT >= R): the
// reference's k-ascending forward and backward substitutions, each pivot's
// division a multiplication by its reciprocal (chol_substitute).
constexpr int CHOL_RM = 32;
constexpr int CHOL_T = 64;     // chol_apply_kernel: one right-hand side per thread
constexpr int CHOL_FT = 256;   // chol_factor_kernel

template <int RT>
__global__ __launch_bounds__(CHOL_FT) void chol_factor_kernel(const double* __restrict__ FtF,
                                                              int R, double* __restrict__ Lout)
{
    // thread = row + RT * part; the thread holds columns part*C .. part*C+C-1
    constexpr int LPR = CHOL_FT / RT;
    constexpr int C = RT / LPR;
    static_assert(C >= 1 && C <= 16, "chol layout");
    __shared__ double col[RT];    // column j before scaling (pivot on the diagonal)
    __shared__ double lcol[RT];   // column j of L
    __shared__ double trs;
    const int tid = threadIdx.x;
    const int row = tid % RT;
    const int part = tid / RT;
    const int c0 = part * C;
    const bool mine = row < R;    // rows >= R hold eps I (see below)
    double a[C];
#pragma unroll
    for (int c = 0; c < C; ++c)
        a[c] = (mine && c0 + c < R) ? FtF[size_t(row) * R + c0 + c] : 0.0;
    // eps from the trace, summed in row order
#pragma unroll
    for (int c = 0; c < C; ++c)
        if (c0 + c == row) col[row] = a[c];
    __syncthreads();
    if (tid == 0)
    {
        double tr = 0.0;
        for (int i = 0; i < R; ++i) tr += col[i];
        trs = tr;
    }
    __syncthreads();
    const double tr = trs;
    const double eps = 1e-12 * ((tr > 0.0) ? tr / double(R) : 1.0) + 1e-300;
#pragma unroll
    for (int c = 0; c < C; ++c)
        if (c0 + c == row) a[c] += eps;
    // Steps j < R only; rows >= R hold zeros off the diagonal, so they
    // subtract exact zeros from the rows < R.
    for (int jp = 0; jp * C < R; ++jp)
    {
#pragma unroll
        for (int jc = 0; jc < C; ++jc)
        {
            const int j = jp * C + jc;
            if (j >= R) break;
            if (part == jp) col[row] = a[jc];
            __syncthreads();
            const double s = col[j];
            const double d = (s > 0.0) ? sqrt(s) : sqrt(eps);
            if (part == jp)
            {
                const double v = col[row];
                lcol[row] = (row == j) ? d : ((mine && row > j) ? v / d : v);   // L[row][j]
            }
            __syncthreads();
            const double lij = lcol[row];
#pragma unroll
            for (int c = 0; c < C; ++c)
            {
                if (part == jp && c == jc) a[c] = lij;
                else if (c0 + c > j) a[c] -= lij * lcol[c0 + c];
            }
        }
    }
    if (mine)
#pragma unroll
        for (int c = 0; c < C; ++c)
            if (c0 + c < R) Lout[size_t(row) * R + c0 + c] = (c0 + c <= row) ? a[c] : 0.0;
}

// L y' = y, then L^T x = y', with the Cholesky factor in LDS (RT x RT, padded
// with the identity, so padding entries stay exact zeros) and the reciprocals
// of its diagonal (dinv): row by row, each row's sum in ascending k as the
// reference's substitutions, the division by the pivot done as a
// multiplication by its reciprocal (one correctly rounded division per pivot
// per workgroup instead of one per pivot and right-hand side; the row's
// result differs from the division's by at most an ulp).  The next row's
// entries of L (and its reciprocal) load into a second register set while
// the current row's sum runs; the empty asm with a memory clobber keeps a
// later row's loads from being hoisted further, which would not fit the
// registers.
template <int RT>
__device__ __forceinline__ void chol_substitute(const double (*L)[RT + 1],
                                                const double* __restrict__ dinv,
                                                double (&y)[RT])
{
    double cur[RT], nxt[RT], cd = dinv[0], nd = 0.0;
#pragma unroll
    for (int i = 0; i < RT; ++i)
    {
        if (i + 1 < RT)
        {
#pragma unroll
            for (int k = 0; k <= i; ++k) nxt[k] = L[i + 1][k];
            nd = dinv[i + 1];
        }
        double s = y[i];
#pragma unroll
        for (int k = 0; k < i; ++k) s -= cur[k] * y[k];
        y[i] = s * cd;
        asm volatile("" ::: "memory");
#pragma unroll
        for (int k = 0; k <= i; ++k) cur[k] = nxt[k];
        cd = nd;
    }
    // L^T x = y': row i takes column i of L below the diagonal
    cd = dinv[RT - 1];
#pragma unroll
    for (int i = RT - 1; i >= 0; --i)
    {
        if (i > 0)
        {
#pragma unroll
            for (int k = i; k < RT; ++k) nxt[k] = L[k][i - 1];
            nd = dinv[i - 1];
        }
        double s = y[i];
#pragma unroll
        for (int k = i + 1; k < RT; ++k) s -= cur[k] * y[k];
        y[i] = s * cd;   // x[i]
        asm volatile("" ::: "memory");
#pragma unroll
        for (int k = i; k < RT; ++k) cur[k] = nxt[k];
        cd = nd;
    }
}

template <int RT>
__global__ __launch_bounds__(CHOL_T) void chol_apply_kernel(const double* __restrict__ Lg,
                                                            const double* __restrict__ FtV,
                                                            double* __restrict__ F, size_t dim,
                                                            int R)
{
    // L padded to RT with the identity: padding entries of y stay 0 and
    // only exact zeros are subtracted from the others, so the unrolled loops
    // below need no condition on R
    __shared__ double L[RT][RT + 1];
    __shared__ double dinv[RT];
    for (int x = threadIdx.x; x < RT * RT; x += CHOL_T)
    {
        const int i = x / RT, k = x % RT;
        const double v = (i < R && k < R) ? Lg[size_t(i) * R + k] : (i == k ? 1.0 : 0.0);
        L[i][k] = v;
        if (i == k) dinv[i] = 1.0 / v;
    }
    __syncthreads();
    const size_t row = size_t(blockIdx.x) * CHOL_T + threadIdx.x;
    if (row >= dim) return;
    const double* b = FtV + row * R;
    double y[RT];
#pragma unroll
    for (int i = 0; i < RT; ++i) y[i] = (i < R) ? b[i] : 0.0;
    chol_substitute<RT>(L, dinv, y);
    double* out = F + row * R;
#pragma unroll
    for (int i = 0; i < RT; ++i)
        if (i < R) out[i] = y[i];
}

// cptc_chol_ridge_factor + cptc_chol_ridge_apply in one launch, R <= RT <=
// 32: each 64-lane workgroup (one wave) factors FtF + eps I itself, lane i
// holding row i in registers and each step's pivot column passing through
// LDS inside the wave, so no workgroup barrier (chol_factor_kernel's 2 R
// barriers across four waves are most of its ~17 us at R = 32); every
// operation is chol_factor_kernel's, in its order, so L is the same bits.
// Then each lane solves one right-hand-side row as chol_apply_kernel.  The
// grids are small (one workgroup per 64 rows), so the kernel takes registers
// over occupancy (the row and the solve vector, 2 x 64 at RT = 32).
template <int RT>
__global__ __launch_bounds__(CHOL_T) __attribute__((amdgpu_waves_per_eu(1, 2))) void
chol_solve_wave_kernel(const double* __restrict__ FtF,
                                                                 const double* __restrict__ FtV,
                                                                 double* __restrict__ F,
                                                                 size_t dim, int R)
{
    static_assert(RT <= 32 && CHOL_T == 64, "one wave, one row per lane");
    __shared__ double L[RT][RT + 1];
    __shared__ double dinv[RT];
    __shared__ double lcol[2][RT];   // column j of L, alternating buffers by step
    const int lane = threadIdx.x;
    const bool act = lane < RT;
    const bool mine = lane < R;
    auto wave_sync = [] {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    // lane l's value of x (a wave-uniform result)
    auto lane_f64 = [](double x, int l) {
        const uint64_t u = __builtin_bit_cast(uint64_t, x);
        const uint32_t lo = uint32_t(__builtin_amdgcn_readlane(int(uint32_t(u)), l));
        const uint32_t hi = uint32_t(__builtin_amdgcn_readlane(int(uint32_t(u >> 32)), l));
        return __builtin_bit_cast(double, (uint64_t(hi) << 32) | lo);
    };
    double a[RT];
#pragma unroll
    for (int c = 0; c < RT; ++c) a[c] = (mine && c < R) ? FtF[size_t(lane) * R + c] : 0.0;
    // eps from the trace, summed in row order (the diagonal entry of row i is
    // lane i's a[i])
    double tr = 0.0;
#pragma unroll
    for (int i = 0; i < RT; ++i)
        if (i < R) tr += lane_f64(a[i], i);
    const double eps = 1e-12 * ((tr > 0.0) ? tr / double(R) : 1.0) + 1e-300;
#pragma unroll
    for (int c = 0; c < RT; ++c)
        if (c == lane) a[c] += eps;
    // (fully unrolled, so the row stays in registers: a partly unrolled
    // loop indexes it at run time and moves it to scratch memory).  The
    // pivot is lane j's a[j], read across lanes; column j of L goes through
    // LDS, in the buffer the step after next reuses (a wave's LDS operations
    // are in order, so the next step's writes to the other buffer need no
    // barrier behind this step's reads).
#pragma unroll
    for (int j = 0; j < RT; ++j)
    {
        if (j < R)   // steps j < R only (uniform; no early exit, so the loop unrolls)
        {
            const double sp = lane_f64(a[j], j);
            const double d = (sp > 0.0) ? sqrt(sp) : sqrt(eps);
            const double v = a[j];
            const double lij = (lane == j) ? d : ((mine && lane > j) ? v / d : v);
            double* lc = lcol[j & 1];
            if (act) lc[lane] = lij;
            wave_sync();
            a[j] = lij;
#pragma unroll
            for (int c = j + 1; c < RT; ++c) a[c] -= lij * lc[c];
        }
    }
    // L padded to RT with the identity (chol_apply_kernel's layout)
    if (act)
#pragma unroll
        for (int c = 0; c < RT; ++c)
        {
            const double v = (mine && c < R) ? ((c <= lane) ? a[c] : 0.0) : (c == lane ? 1.0 : 0.0);
            L[lane][c] = v;
            if (c == lane) dinv[lane] = 1.0 / v;
        }
    __syncthreads();
    const size_t row = size_t(blockIdx.x) * CHOL_T + size_t(lane);
    if (row >= dim) return;
    const double* b = FtV + row * R;
    double y[RT];
#pragma unroll
    for (int i = 0; i < RT; ++i) y[i] = (i < R) ? b[i] : 0.0;
    chol_substitute<RT>(L, dinv, y);
    double* out = F + row * R;
#pragma unroll
    for (int i = 0; i < RT; ++i)
        if (i < R) out[i] = y[i];
}

// Column sums of squares: P partials of R each (deterministic).
__global__ __launch_bounds__(256) void colsq_partial_kernel(const double* __restrict__ F,
                                                            size_t rows, int R,
                                                            double* __restrict__ part)
{
    // 256 threads = (256 / R) row lanes x R ranks (R <= 32 -> >= 8 row lanes)
    __shared__ double red[256];
    const int r = threadIdx.x % R;
    const int rl = threadIdx.x / R;
    const int nrl = 256 / R;
    double acc = 0.0;
    if (rl < nrl)
        for (size_t i = size_t(blockIdx.x) * nrl + rl; i < rows; i += size_t(gridDim.x) * nrl)
        {
            const double v = F[i * R + r];
            acc += v * v;
        }
    red[threadIdx.x] = acc;
    __syncthreads();
    if (threadIdx.x < R)
    {
        double t = 0.0;
        for (int q = 0; q < nrl; ++q) t += red[q * R + threadIdx.x];
        part[size_t(blockIdx.x) * R + threadIdx.x] = t;
    }
}

// Every block re-reduces the partials (P x R, small), divides its rows, and
// block 0 writes lambda.
__global__ __launch_bounds__(256) void normalize_nd_kernel(double* __restrict__ F, size_t rows,
                                                           int R, const double* __restrict__ part,
                                                           int P, double* __restrict__ lambda)
{
    __shared__ double nrm[32];
    if (threadIdx.x < R)
    {
        double s = 0.0;
        for (int p = 0; p < P; ++p) s += part[size_t(p) * R + threadIdx.x];
        double n = sqrt(s);
        if (!isfinite(n) || n < 1e-14) n = 1.0;
        nrm[threadIdx.x] = n;
        if (blockIdx.x == 0) lambda[threadIdx.x] = n;
    }
    __syncthreads();
    const size_t total = rows * size_t(R);
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    for (size_t x = size_t(blockIdx.x) * blockDim.x + threadIdx.x; x < total; x += stride)
        F[x] /= nrm[x % R];
}

// A small factor's update tail in one workgroup (rows x R <= SMALL_UPDATE_MAX,
// R <= 32): the normalisation of normalize_nd_kernel (lambda_r = the column's
// 2-norm, 1 when it is not finite or below 1e-14; F /= lambda), the Gram
// G_mode = F^T F of the normalised factor and, when next >= 0, the next
// mode's FtF = prod_{g != next} G_g in mode order (gram_hadamard_kernel) and
// its first nzero FtV entries zeroed: one launch instead of six.  Rows are
// staged in LDS 64 at a time; each Gram entry sums its rows in order.
constexpr int SMALL_UPDATE_MAX = 1 << 16;

__global__ __launch_bounds__(1024) void small_update_kernel(
    double* __restrict__ F, int rows, int R, double* __restrict__ lambda, double* __restrict__ grams,
    int ngram, int mode, int next, double* __restrict__ FtF, double* __restrict__ FtV, int nzero)
{
    __shared__ double red[1024];
    __shared__ double nrm[32];
    __shared__ double tile[64 * 32];
    const int tid = threadIdx.x;
    const int RR = R * R;
    const int r = tid % R, rl = tid / R, nrl = 1024 / R;
    double acc = 0.0;
    if (rl < nrl)
        for (int i = rl; i < rows; i += nrl)
        {
            const double v = F[size_t(i) * R + r];
            acc += v * v;
        }
    red[tid] = acc;
    __syncthreads();
    if (tid < R)
    {
        double sq = 0.0;
        for (int q = 0; q < nrl; ++q) sq += red[q * R + tid];
        double n = sqrt(sq);
        if (!isfinite(n) || n < 1e-14) n = 1.0;
        nrm[tid] = n;
        lambda[tid] = n;
    }
    __syncthreads();
    // Gram entry e = tid % RR, row group q = tid / RR of NQ: group q sums the
    // rows i = q mod NQ, then the groups' sums are added in group order
    const int NQ = 1024 / RR;
    const int e = tid % RR, q = tid / RR;
    const int a = e / R, b = e % R;
    double g = 0.0;
    for (int i0 = 0; i0 < rows; i0 += 64)
    {
        const int nr = min(64, rows - i0);
        for (int x = tid; x < nr * R; x += 1024)
        {
            const double v = F[size_t(i0) * R + x] / nrm[x % R];
            F[size_t(i0) * R + x] = v;
            tile[x] = v;
        }
        __syncthreads();
        if (q < NQ)
            for (int i = q; i < nr; i += NQ) g += tile[i * R + a] * tile[i * R + b];
        __syncthreads();
    }
    red[tid] = g;
    __syncthreads();
    if (tid < RR)
    {
        g = 0.0;
        for (int p = 0; p < NQ; ++p) g += red[p * RR + tid];
        grams[size_t(mode) * RR + tid] = g;
    }
    if (next >= 0)
    {
        if (tid < RR)
        {
            double v = 1.0;
            for (int gm = 0; gm < ngram; ++gm)
                if (gm != next) v *= (gm == mode) ? g : grams[size_t(gm) * RR + tid];
            FtF[tid] = v;
        }
        for (int x = tid; x < nzero; x += 1024) FtV[x] = 0.0;
    }
}

// --------------------------------------------------------- exact residual --

__global__ __launch_bounds__(256) void residual_nd_kernel(int nmodes,
                                                          const uint32_t* __restrict__ coords,
                                                          const double* __restrict__ vals,
                                                          uint64_t nnz, Factors F,
                                                          const double* __restrict__ lambda,
                                                          int R, double* __restrict__ part)
{
    __shared__ double red[2][256];
    double res = 0.0, sq = 0.0;
    const uint64_t stride = uint64_t(gridDim.x) * blockDim.x;
    for (uint64_t e = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; e < nnz; e += stride)
    {
        const double* rowp[MAXM];
#pragma unroll
        for (int m = 0; m < MAXM; ++m)
            rowp[m] = (m < nmodes) ? F.p[m] + size_t(coords[uint64_t(m) * nnz + e]) * R : nullptr;
        double xhat = 0.0;
        for (int r = 0; r < R; ++r)
        {
            double p = lambda ? lambda[r] : 1.0;
#pragma unroll
            for (int m = 0; m < MAXM; ++m)
                if (m < nmodes) p *= rowp[m][r];
            xhat += p;
        }
        const double v = vals[e];
        const double d = v - xhat;
        res += d * d;
        sq += v * v;
    }
    red[0][threadIdx.x] = res;
    red[1][threadIdx.x] = sq;
    __syncthreads();
    for (int h = 128; h > 0; h >>= 1)
    {
        if (int(threadIdx.x) < h)
        {
            red[0][threadIdx.x] += red[0][threadIdx.x + h];
            red[1][threadIdx.x] += red[1][threadIdx.x + h];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0)
    {
        part[2 * size_t(blockIdx.x)] = red[0][0];
        part[2 * size_t(blockIdx.x) + 1] = red[1][0];
    }
}

__global__ void finalize_add2_kernel(const double* __restrict__ part, int P,
                                     double* __restrict__ out2)
{
    if (threadIdx.x < 2)
    {
        double t = 0.0;
        for (int p = 0; p < P; ++p) t += part[2 * size_t(p) + threadIdx.x];
        out2[threadIdx.x] += t;
    }
}

bool factors_ok(int n, const double* const* h_F)
{
    if (!h_F) return false;
    for (int m = 0; m < n; ++m)
        if (!h_F[m]) return false;
    return true;
}

}  // namespace

extern "C" uint64_t cptc_gen_hash(uint64_t x)
{
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

extern "C" int cptc_mttkrp_seg_nd(int nmodes, int mode, const uint32_t* d_scoords,
                                  const int* level_modes, const double* d_vals,
                                  const uint8_t* d_skip, uint64_t nnz, const uint32_t* d_seg_row,
                                  const uint32_t* d_seg_start, const uint32_t* d_seg_cnt,
                                  const uint8_t* d_single, uint64_t nseg,
                                  const double* const* h_F, double* d_FtV, int R, void* stream)
{
    CPTC_REQUIRE(nmodes >= 2 && nmodes <= MAXM && mode >= 0 && mode < nmodes, CPTC_ERR_ARG,
                 "cptc_mttkrp_seg_nd: nmodes %d mode %d", nmodes, mode);
    CPTC_REQUIRE(R >= 1 && R <= 32, CPTC_ERR_ARG, "cptc_mttkrp_seg_nd: R %d (1..32)", R);
    if (nseg == 0) return CPTC_OK;
    CPTC_REQUIRE(nseg < (uint64_t(1) << 31) && nnz <= 0x7FFFFFFFull, CPTC_ERR_ARG,
                 "cptc_mttkrp_seg_nd: %llu segments / %llu nnz", (unsigned long long)nseg,
                 (unsigned long long)nnz);
    CPTC_REQUIRE(d_scoords && d_vals && d_seg_row && d_seg_start && d_seg_cnt && d_FtV &&
                     factors_ok(nmodes, h_F),
                 CPTC_ERR_ARG, "cptc_mttkrp_seg_nd: null pointer");
    // factors in level order (the d_scoords rows)
    Factors F{};
    bool aligned = (R % 2 == 0);
    unsigned seen = 1u << mode;
    for (int q = 0; q < nmodes - 1; ++q)
    {
        const int m = level_modes ? level_modes[q] : (q < mode ? q : q + 1);
        CPTC_REQUIRE(m >= 0 && m < nmodes && !(seen & (1u << m)), CPTC_ERR_ARG,
                     "cptc_mttkrp_seg_nd: level_modes is not a permutation of the other modes");
        seen |= 1u << m;
        F.p[q] = h_F[m];
        if (reinterpret_cast<uintptr_t>(h_F[m]) & 15) aligned = false;
    }
    hipStream_t s = cptc::as_stream(stream);
    if (aligned)
        launch_seg_n<2>(nmodes, F, mode, d_scoords, nnz, d_vals, d_skip, d_seg_row, d_seg_start,
                        d_seg_cnt, d_single, nseg, d_FtV, R, s);
    else
        launch_seg_n<1>(nmodes, F, mode, d_scoords, nnz, d_vals, d_skip, d_seg_row, d_seg_start,
                        d_seg_cnt, d_single, nseg, d_FtV, R, s);
    CPTC_LAUNCHED();
    return CPTC_OK;
}

extern "C" int cptc_units_pack_nd(const uint32_t* d_unit6, uint64_t nunits, const uint32_t* d_lid,
                                  const double* d_val, float* d_tiles, void* stream)
{
    if (nunits == 0) return CPTC_OK;
    CPTC_REQUIRE(d_unit6 && d_lid && d_val && d_tiles, CPTC_ERR_ARG,
                 "cptc_units_pack_nd: null pointer");
    CPTC_REQUIRE(nunits < (uint64_t(1) << 31), CPTC_ERR_ARG, "cptc_units_pack_nd: too many units");
    hipLaunchKernelGGL(units_pack_kernel, dim3(unsigned(nunits)), dim3(256), 0,
                       cptc::as_stream(stream), d_unit6, d_lid, d_val, d_tiles);
    CPTC_LAUNCHED();
    return CPTC_OK;
}

extern "C" int cptc_units_pack_nd_f64(const uint32_t* d_unit6, uint64_t nunits,
                                      const uint32_t* d_lid, const double* d_val, double* d_img,
                                      void* stream)
{
    if (nunits == 0) return CPTC_OK;
    CPTC_REQUIRE(d_unit6 && d_lid && d_val && d_img, CPTC_ERR_ARG,
                 "cptc_units_pack_nd_f64: null pointer");
    CPTC_REQUIRE((reinterpret_cast<uintptr_t>(d_img) & 15) == 0, CPTC_ERR_ARG,
                 "cptc_units_pack_nd_f64: the image must be 16-byte aligned");
    CPTC_REQUIRE(nunits < (uint64_t(1) << 31), CPTC_ERR_ARG,
                 "cptc_units_pack_nd_f64: too many units");
    hipLaunchKernelGGL(units_pack_f64_kernel, dim3(unsigned(nunits)), dim3(256), 0,
                       cptc::as_stream(stream), d_unit6, d_lid, d_val, d_img);
    CPTC_LAUNCHED();
    return CPTC_OK;
}

extern "C" int cptc_units_weights_nd(const uint32_t* d_unit6, uint64_t nunits,
                                     const uint32_t* d_outer_coords, int nouter,
                                     const int* outer_modes, const double* const* h_F, int R,
                                     double* d_W, void* stream)
{
    CPTC_REQUIRE(R >= 1 && nouter >= 0 && nouter <= MAXM - 3, CPTC_ERR_ARG,
                 "cptc_units_weights_nd: R %d nouter %d", R, nouter);
    if (nunits == 0) return CPTC_OK;
    CPTC_REQUIRE(d_unit6 && d_W && (nouter == 0 || (d_outer_coords && outer_modes && h_F)),
                 CPTC_ERR_ARG, "cptc_units_weights_nd: null pointer");
    Factors Fo{};
    for (int k = 0; k < nouter; ++k)
    {
        CPTC_REQUIRE(outer_modes[k] >= 0 && outer_modes[k] < MAXM && h_F[outer_modes[k]],
                     CPTC_ERR_ARG, "cptc_units_weights_nd: outer mode %d", outer_modes[k]);
        Fo.p[k] = h_F[outer_modes[k]];
    }
    const uint64_t total = nunits * uint64_t(R);
    hipLaunchKernelGGL(units_weights_kernel, dim3(cptc::grid_for(total, 256, 65536)), dim3(256), 0,
                       cptc::as_stream(stream), d_unit6, nunits, d_outer_coords, nouter, Fo, R,
                       d_W);
    CPTC_LAUNCHED();
    return CPTC_OK;
}

extern "C" int cptc_gram_hadamard(const double* d_grams, int ngram, int skip, int R,
                                  double* d_out, void* stream)
{
    CPTC_REQUIRE(R >= 1 && ngram >= 0 && d_out && (ngram == 0 || d_grams), CPTC_ERR_ARG,
                 "cptc_gram_hadamard: bad arguments");
    const int RR = R * R;
    hipLaunchKernelGGL(gram_hadamard_kernel, dim3(cptc::grid_for(size_t(RR), 256, 256)),
                       dim3(256), 0, cptc::as_stream(stream), d_grams, ngram, skip, RR, d_out);
    CPTC_LAUNCHED();
    return CPTC_OK;
}

extern "C" int cptc_chol_ridge_factor(const double* d_FtF, double* d_L, int R, void* stream)
{
    CPTC_REQUIRE(R >= 1 && R <= CHOL_RM, CPTC_ERR_ARG, "cptc_chol_ridge_factor: R %d (1..32)", R);
    CPTC_REQUIRE(d_FtF && d_L, CPTC_ERR_ARG, "cptc_chol_ridge_factor: null pointer");
    hipStream_t s = cptc::as_stream(stream);
    if (R <= 16)
        hipLaunchKernelGGL(chol_factor_kernel<16>, dim3(1), dim3(CHOL_FT), 0, s, d_FtF, R, d_L);
    else
        hipLaunchKernelGGL(chol_factor_kernel<CHOL_RM>, dim3(1), dim3(CHOL_FT), 0, s, d_FtF, R,
                           d_L);
    CPTC_LAUNCHED();
    return CPTC_OK;
}

extern "C" int cptc_chol_ridge_apply(const double* d_L, const double* d_FtV, double* d_F,
                                     size_t dim, int R, void* stream)
{
    CPTC_REQUIRE(R >= 1 && R <= CHOL_RM, CPTC_ERR_ARG, "cptc_chol_ridge_apply: R %d (1..32)", R);
    if (dim == 0) return CPTC_OK;
    CPTC_REQUIRE(d_L && d_FtV && d_F, CPTC_ERR_ARG, "cptc_chol_ridge_apply: null pointer");
    CPTC_REQUIRE(dim / CHOL_T < (size_t(1) << 31), CPTC_ERR_ARG,
                 "cptc_chol_ridge_apply: %zu rows", dim);
    const dim3 grid(unsigned((dim + CHOL_T - 1) / CHOL_T));
    hipStream_t s = cptc::as_stream(stream);
    if (R <= 8)
        hipLaunchKernelGGL(chol_apply_kernel<8>, grid, dim3(CHOL_T), 0, s, d_L, d_FtV, d_F, dim, R);
    else if (R <= 16)
        hipLaunchKernelGGL(chol_apply_kernel<16>, grid, dim3(CHOL_T), 0, s, d_L, d_FtV, d_F, dim,
                           R);
    else
        hipLaunchKernelGGL(chol_apply_kernel<CHOL_RM>, grid, dim3(CHOL_T), 0, s, d_L, d_FtV, d_F,
                           dim, R);
    CPTC_LAUNCHED();
    return CPTC_OK;
}

extern "C" int cptc_chol_ridge_solve(const double* d_FtF, const double* d_FtV, double* d_F,
                                     size_t dim, int R, void* stream)
{
    CPTC_REQUIRE(R >= 1 && R <= CHOL_RM, CPTC_ERR_ARG, "cptc_chol_ridge_solve: R %d (1..32)", R);
    if (dim == 0) return CPTC_OK;
    CPTC_REQUIRE(d_FtF && d_FtV && d_F, CPTC_ERR_ARG, "cptc_chol_ridge_solve: null pointer");
    CPTC_REQUIRE(dim / CHOL_T < (size_t(1) << 31), CPTC_ERR_ARG,
                 "cptc_chol_ridge_solve: %zu rows", dim);
    // one launch: every workgroup factors (one wave, ~1-2 us) and solves its
    // 64 rows; the same bits as cptc_chol_ridge_factor + cptc_chol_ridge_apply
    const dim3 grid(unsigned((dim + CHOL_T - 1) / CHOL_T));
    hipStream_t s = cptc::as_stream(stream);
    if (R <= 8)
        hipLaunchKernelGGL(chol_solve_wave_kernel<8>, grid, dim3(CHOL_T), 0, s, d_FtF, d_FtV, d_F,
                           dim, R);
    else if (R <= 16)
        hipLaunchKernelGGL(chol_solve_wave_kernel<16>, grid, dim3(CHOL_T), 0, s, d_FtF, d_FtV,
                           d_F, dim, R);
    else
        hipLaunchKernelGGL(chol_solve_wave_kernel<CHOL_RM>, grid, dim3(CHOL_T), 0, s, d_FtF,
                           d_FtV, d_F, dim, R);
    CPTC_LAUNCHED();
    return CPTC_OK;
}

extern "C" int cptc_gen_normalize(double* d_F, size_t rows, int R, double* d_lambda, void* stream)
{
    CPTC_REQUIRE(R >= 1 && R <= 32 && d_F && d_lambda, CPTC_ERR_ARG,
                 "cptc_gen_normalize: R %d (1..32) or null pointer", R);
    const int nrl = 256 / R;
    const int P = int(cptc::grid_for(rows, unsigned(nrl) * 8, 256));
    void* buf = nullptr;
    CPTC_TRY(cptc::scratch_get(cptc::SCR_REDUCE, size_t(P) * R * sizeof(double), &buf));
    double* part = static_cast<double*>(buf);
    hipStream_t s = cptc::as_stream(stream);
    hipLaunchKernelGGL(colsq_partial_kernel, dim3(P), dim3(256), 0, s, d_F, rows, R, part);
    CPTC_LAUNCHED();
    hipLaunchKernelGGL(normalize_nd_kernel, dim3(cptc::grid_for(rows * size_t(R), 256, 1024)),
                       dim3(256), 0, s, d_F, rows, R, part, P, d_lambda);
    CPTC_LAUNCHED();
    return CPTC_OK;
}

extern "C" int cptc_gen_normalize_gram(double* d_F, size_t rows, int R, double* d_lambda,
                                       double* d_grams, int ngram, int mode, int next,
                                       double* d_FtF, double* d_FtV, size_t nzero, void* stream)
{
    CPTC_REQUIRE(R >= 1 && R <= 32 && rows >= 1 && rows * size_t(R) <= size_t(SMALL_UPDATE_MAX),
                 CPTC_ERR_ARG, "cptc_gen_normalize_gram: rows %zu x R %d (R <= 32, <= %d values)",
                 rows, R, SMALL_UPDATE_MAX);
    CPTC_REQUIRE(ngram >= 1 && mode >= 0 && mode < ngram && next >= -1 && next < ngram &&
                     nzero <= (size_t(1) << 24),
                 CPTC_ERR_ARG, "cptc_gen_normalize_gram: ngram %d mode %d next %d nzero %zu",
                 ngram, mode, next, nzero);
    CPTC_REQUIRE(d_F && d_lambda && d_grams && (next < 0 || d_FtF) && (nzero == 0 || d_FtV),
                 CPTC_ERR_ARG, "cptc_gen_normalize_gram: null pointer");
    hipLaunchKernelGGL(small_update_kernel, dim3(1), dim3(1024), 0, cptc::as_stream(stream), d_F,
                       int(rows), R, d_lambda, d_grams, ngram, mode, next, d_FtF, d_FtV,
                       next >= 0 ? int(nzero) : 0);
    CPTC_LAUNCHED();
    return CPTC_OK;
}

extern "C" int cptc_residual_nd(int nmodes, const uint32_t* d_coords, const double* d_vals,
                                uint64_t nnz, const double* const* h_F, const double* d_lambda,
                                int R, double* d_out2, void* stream)
{
    CPTC_REQUIRE(nmodes >= 1 && nmodes <= MAXM && R >= 1 && d_out2, CPTC_ERR_ARG,
                 "cptc_residual_nd: nmodes %d R %d", nmodes, R);
    if (nnz == 0) return CPTC_OK;
    CPTC_REQUIRE(d_coords && d_vals && factors_ok(nmodes, h_F), CPTC_ERR_ARG,
                 "cptc_residual_nd: null pointer");
    Factors F{};
    for (int m = 0; m < nmodes; ++m) F.p[m] = h_F[m];
    const int P = int(cptc::grid_for(nnz, 256 * 8, 2048));
    void* buf = nullptr;
    CPTC_TRY(cptc::scratch_get(cptc::SCR_REDUCE, size_t(P) * 2 * sizeof(double), &buf));
    double* part = static_cast<double*>(buf);
    hipStream_t s = cptc::as_stream(stream);
    hipLaunchKernelGGL(residual_nd_kernel, dim3(P), dim3(256), 0, s, nmodes, d_coords, d_vals, nnz,
                       F, d_lambda, R, part);
    CPTC_LAUNCHED();
    hipLaunchKernelGGL(finalize_add2_kernel, dim3(1), dim3(64), 0, s, part, P, d_out2);
    CPTC_LAUNCHED();
    return CPTC_OK;
}
