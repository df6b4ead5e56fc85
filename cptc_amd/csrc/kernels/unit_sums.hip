// Outer-mode MTTKRP of the generic driver when every element lies in a
// dense unit: per-unit FP64 inner sums (formed once after the inner modes'
// updates) and their scatter into an outer mode's rows.  An outer mode's
// MTTKRP over unit elements factors as s_u[r] * prod over the other outer
// modes o of F_o[i_o(u)][r] with s_u[r] = sum v Fa[la][r] Fb[lb][r] Fc[lc][r]
// over the unit's pool: the same FP64 sum as the segment kernel over all
// elements (generic.cu:271-343, the reference's outer-mode path), in another
// order.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "../host/hip_util.hpp"

namespace {

// Per-unit inner sums, R <= 32: s[u][r] = sum over the unit's elements of
// v Fa[16 bi + la][r] Fb[16 bj + lb][r] Fc[16 bk + lc][r] (FP64; the unit's
// contraction over its three inner modes, lid = la 256 + lb 16 + lc).
//
// A workgroup takes one chunk of units that share their inner block triple
// (bi, bj, bk) (cptc_gen_unit_sums_plan), so the three 16-row factor blocks
// are staged in LDS once per chunk (rows past a factor's end and ranks past R
// as zeros), and each wave takes every 4th unit of the chunk.  A lane owns
// one element (64 per batch, coalesced loads, the next batch's loaded during
// this one) and loops over the RT ranks with its element's three row
// addresses fixed: per two ranks three 16-byte LDS reads (immediate offsets)
// and six FP64 operations, no cross-lane traffic in the element loop.  A
// staged row is RT + 2 doubles (2 RT + 4 dwords), so the 16 rows of a block
// start on 16 distinct 4-bank groups of the 64 banks and a wave's 16-byte
// reads (at most 16 distinct rows, equal rows broadcast) do not conflict.
// Per unit the lanes' RT partial sums are added across the wave through a
// per-wave LDS buffer, 8 ranks at a time (each rank's 64 partials summed by
// 8 lanes, then 3 xor shuffles).
constexpr int USUM_R = 32;
constexpr int USUM_WAVES = 4;
template <int RT>
__global__ __launch_bounds__(64 * USUM_WAVES) void unit_sums_kernel(
    const uint32_t* __restrict__ unit6, const uint32_t* __restrict__ order,
    const uint32_t* __restrict__ chunk_off, const uint32_t* __restrict__ lid,
    const double* __restrict__ val, const double* __restrict__ Fa, const double* __restrict__ Fb,
    const double* __restrict__ Fc, int da, int db, int dc, int R, double* __restrict__ sums)
{
    constexpr int ROWD = RT + 2;           // doubles per staged row
    constexpr int BLKD = 16 * ROWD;        // doubles per staged block
    constexpr int REDS = 9;                // doubles per lane in the reduction buffer
    __shared__ __attribute__((aligned(16))) double blk[3 * BLKD];
    __shared__ double red[USUM_WAVES][64 * REDS];
    const uint32_t i0 = chunk_off[blockIdx.x], i1 = chunk_off[blockIdx.x + 1];
    {
        const uint32_t* h = unit6 + size_t(order[i0]) * 6;
        const int r0[3] = {int(h[0]) * 16, int(h[1]) * 16, int(h[2]) * 16};
        const int dim[3] = {da, db, dc};
        const double* F[3] = {Fa, Fb, Fc};
        constexpr int PER = 16 * (RT / 2);   // double2 items per block
        for (int x = threadIdx.x; x < 3 * PER; x += 64 * USUM_WAVES)
        {
            const int f = x / PER, rem = x % PER;
            const int row = rem / (RT / 2), c = (rem % (RT / 2)) * 2;
            const int g = r0[f] + row;
            double2 v = make_double2(0.0, 0.0);
            if (g < dim[f])
            {
                const double* src = F[f] + size_t(g) * R;
                if (c < R) v.x = src[c];
                if (c + 1 < R) v.y = src[c + 1];
            }
            *reinterpret_cast<double2*>(blk + f * BLKD + row * ROWD + c) = v;
        }
    }
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    double* rb = red[w];
    for (uint32_t i = i0 + uint32_t(w); i < i1; i += USUM_WAVES)
    {
        const uint32_t u = order[i];
        const uint32_t cnt = unit6[size_t(u) * 6 + 3];
        const uint32_t st = unit6[size_t(u) * 6 + 4];
        double acc[RT];
#pragma unroll
        for (int q = 0; q < RT; ++q) acc[q] = 0.0;
        uint32_t ln = 0;
        double vn = 0.0;
        if (uint32_t(lane) < cnt)
        {
            ln = lid[st + uint32_t(lane)];
            vn = val[st + uint32_t(lane)];
        }
        for (uint32_t b0 = 0; b0 < cnt; b0 += 64)
        {
            const uint32_t l = ln;
            const double v = vn;   // 0 past the unit's end: those lanes add zeros
            const uint32_t e = b0 + 64 + uint32_t(lane);
            ln = 0;
            vn = 0.0;
            if (e < cnt)
            {
                ln = lid[st + e];
                vn = val[st + e];
            }
            const double* pa = blk + (l >> 8) * ROWD;
            const double* pb = blk + BLKD + ((l >> 4) & 15u) * ROWD;
            const double* pc = blk + 2 * BLKD + (l & 15u) * ROWD;
#pragma unroll
            for (int r = 0; r < RT; r += 2)
            {
                const double2 fa = *reinterpret_cast<const double2*>(pa + r);
                const double2 fb = *reinterpret_cast<const double2*>(pb + r);
                const double2 fc = *reinterpret_cast<const double2*>(pc + r);
                acc[r] = __builtin_fma(v * fa.x * fb.x, fc.x, acc[r]);
                acc[r + 1] = __builtin_fma(v * fa.y * fb.y, fc.y, acc[r + 1]);
            }
        }
        const int j = lane & 7, sl = lane >> 3;
#pragma unroll
        for (int q = 0; q < RT; q += 8)
        {
#pragma unroll
            for (int k = 0; k < 8; ++k) rb[lane * REDS + k] = acc[q + k];
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            double t = 0.0;
#pragma unroll
            for (int k = 0; k < 8; ++k) t += rb[(sl * 8 + k) * REDS + j];
            t += __shfl_xor(t, 8);
            t += __shfl_xor(t, 16);
            t += __shfl_xor(t, 32);
            if (lane < 8 && q + lane < R) sums[size_t(u) * R + size_t(q + lane)] = t;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
    }
}

// The same sums on the FP64 matrix cores (v_mfma_f64_16x16x4f64) from the
// units' dense FP64 images (cptc_units_pack_nd_f64, cell la 256 + lb 16 +
// lc): s_u[r] = sum_la Fa[la][r] sum_lb Fb[lb][r] X_la[lb][r] with X_la =
// T_la Fc_blk, T_la the unit's 16 x 16 (lb x lc) slab at la.  unit_sums_kernel
// reads three factor rows from LDS per element and rank pair and is bound by
// the LDS; here each element meets its Fc row inside the matrix product, and
// the Fb and Fa weights are applied once per (la, lb) and per la.
//
// Chunks and staging as unit_sums_kernel; each wave takes every 4th unit.
// Per la and 16-rank tile c: four MFMA steps over lc, where lane l = 16 q +
// j holds A = T_la[lb = j][lc = 4 q + s] (the lane's four cells are one
// 32-byte load; the 64 lanes read the 2 KB slab contiguously) and B =
// Fc[4 q + s][16 c + j]; the result's element v of lane l is X_la[lb = q +
// 4 v][16 c + j] (this instruction's output layout).  The lane then adds
// Fa[la][16 c + j] * sum_v Fb[q + 4 v][16 c + j] X[v] to its sum, and the
// four lane groups q are added at the end.  The B operands and Fb weights
// are fixed per chunk and held in registers.  Rows past a factor's end and
// ranks past R are staged as zeros (image cells there are zero).
typedef double usum_d4 __attribute__((ext_vector_type(4)));
template <int NT>   // 16-rank tiles
__global__ __launch_bounds__(64 * USUM_WAVES) void unit_sums_mfma_kernel(
    const uint32_t* __restrict__ unit6, const uint32_t* __restrict__ order,
    const uint32_t* __restrict__ chunk_off, const double* __restrict__ img,
    const double* __restrict__ Fa, const double* __restrict__ Fb, const double* __restrict__ Fc,
    int da, int db, int dc, int R, double* __restrict__ sums)
{
    constexpr int RT = 16 * NT;
    __shared__ double blk[3][16][RT];
    const uint32_t i0 = chunk_off[blockIdx.x], i1 = chunk_off[blockIdx.x + 1];
    {
        const uint32_t* h = unit6 + size_t(order[i0]) * 6;
        const int r0[3] = {int(h[0]) * 16, int(h[1]) * 16, int(h[2]) * 16};
        const int dim[3] = {da, db, dc};
        const double* F[3] = {Fa, Fb, Fc};
        for (int x = threadIdx.x; x < 3 * 16 * RT; x += 64 * USUM_WAVES)
        {
            const int f = x / (16 * RT), rem = x % (16 * RT);
            const int row = rem / RT, c = rem % RT;
            const int g = r0[f] + row;
            blk[f][row][c] = (g < dim[f] && c < R) ? F[f][size_t(g) * R + c] : 0.0;
        }
    }
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int j = lane & 15, q = lane >> 4;
    double bfr[NT][4], fbw[NT][4];
#pragma unroll
    for (int c = 0; c < NT; ++c)
#pragma unroll
        for (int k = 0; k < 4; ++k)
        {
            bfr[c][k] = blk[2][4 * q + k][16 * c + j];
            fbw[c][k] = blk[1][q + 4 * k][16 * c + j];
        }
    // the wave's units are i0 + w, i0 + w + 4, ...; each in four steps of
    // four la slabs (8 KB), the next step's slabs loaded during this one's
    // MFMAs (two register sets in turn, kept in that order by scheduling
    // barriers), across unit boundaries
    const uint32_t n_unit = (i1 - i0 > uint32_t(w)) ? (i1 - i0 - uint32_t(w) + USUM_WAVES - 1) / USUM_WAVES : 0u;
    const uint32_t n_step = 4 * n_unit;
    struct Slabs
    {
        double2 a[4][2];
    };
    auto load = [&](uint32_t k, Slabs& x) {
        const uint32_t kk = k < n_step ? k : n_step - 1;   // past the end: a reload, never used
        const uint32_t u = order[i0 + uint32_t(w) + USUM_WAVES * (kk >> 2)];
        const double* __restrict__ T = img + size_t(u) * 4096 + (kk & 3u) * 1024u + 16 * j + 4 * q;
#pragma unroll
        for (int b = 0; b < 4; ++b)
        {
            x.a[b][0] = *reinterpret_cast<const double2*>(T + b * 256);
            x.a[b][1] = *reinterpret_cast<const double2*>(T + b * 256 + 2);
        }
    };
    double acc[NT];
#pragma unroll
    for (int c = 0; c < NT; ++c) acc[c] = 0.0;
    auto compute = [&](uint32_t k, const Slabs& x) {
        const int la0 = int(k & 3u) * 4;
        usum_d4 xs[4][NT];
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int c = 0; c < NT; ++c)
            {
                usum_d4 y = {0.0, 0.0, 0.0, 0.0};
                y = __builtin_amdgcn_mfma_f64_16x16x4f64(x.a[b][0].x, bfr[c][0], y, 0, 0, 0);
                y = __builtin_amdgcn_mfma_f64_16x16x4f64(x.a[b][0].y, bfr[c][1], y, 0, 0, 0);
                y = __builtin_amdgcn_mfma_f64_16x16x4f64(x.a[b][1].x, bfr[c][2], y, 0, 0, 0);
                y = __builtin_amdgcn_mfma_f64_16x16x4f64(x.a[b][1].y, bfr[c][3], y, 0, 0, 0);
                xs[b][c] = y;
            }
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int c = 0; c < NT; ++c)
            {
                double t = xs[b][c][0] * fbw[c][0];
                t = __builtin_fma(xs[b][c][1], fbw[c][1], t);
                t = __builtin_fma(xs[b][c][2], fbw[c][2], t);
                t = __builtin_fma(xs[b][c][3], fbw[c][3], t);
                acc[c] = __builtin_fma(blk[0][la0 + b][16 * c + j], t, acc[c]);
            }
        if ((k & 3u) == 3u)   // the unit's last step: its sums
        {
            const uint32_t u = order[i0 + uint32_t(w) + USUM_WAVES * (k >> 2)];
#pragma unroll
            for (int c = 0; c < NT; ++c)
            {
                double v = acc[c];
                v += __shfl_xor(v, 16);
                v += __shfl_xor(v, 32);
                const int r = 16 * c + j;
                if (q == 0 && r < R) sums[size_t(u) * R + r] = v;
                acc[c] = 0.0;
            }
        }
    };
    if (n_step > 0)
    {
        Slabs P, Q;
        load(0, P);
        for (uint32_t k = 0; k < n_step; k += 2)   // n_step is a multiple of 4
        {
            load(k + 1, Q);
            __builtin_amdgcn_sched_barrier(0);
            compute(k, P);
            __builtin_amdgcn_sched_barrier(0);
            load(k + 2, P);
            __builtin_amdgcn_sched_barrier(0);
            compute(k + 1, Q);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

// FtV[i_m(u)][r] += s[u][r] * prod over the other outer modes o of
// F_o[i_o(u)][r] (outer mode m = outer[pos]); a workgroup takes 256 units,
// sums them per (row, rank) in LDS when dim_m x R <= 4096 and flushes once;
// otherwise one atomic add per (unit, rank).
constexpr int USC_LDS = 4096;
__global__ __launch_bounds__(256) void unit_scatter_kernel(
    const uint32_t* __restrict__ outer_coords, size_t nunits, int nouter, int pos,
    const double* const* __restrict__ Fo, const double* __restrict__ sums, int R, size_t dim_m,
    double* __restrict__ FtV)
{
    __shared__ double acc[USC_LDS];
    const bool lds = dim_m * size_t(R) <= size_t(USC_LDS);
    const int n_l = lds ? int(dim_m) * R : 0;
    for (int x = threadIdx.x; x < n_l; x += 256) acc[x] = 0.0;
    __syncthreads();
    const size_t u0 = size_t(blockIdx.x) * 256;
    for (int x = threadIdx.x; x < 256 * R; x += 256)
    {
        const size_t u = u0 + size_t(x / R);
        const int r = x % R;
        if (u >= nunits) break;
        const uint32_t* oc = outer_coords + u * size_t(nouter);
        double v = sums[u * size_t(R) + r];
        for (int o = 0; o < nouter; ++o)
            if (o != pos) v *= Fo[o][size_t(oc[o]) * R + r];
        const size_t row = oc[pos];
        if (lds)
            atomicAdd(&acc[row * R + r], v);
        else
            atomicAdd(FtV + row * size_t(R) + r, v);
    }
    if (!lds) return;
    __syncthreads();
    for (int x = threadIdx.x; x < n_l; x += 256)
        if (acc[x] != 0.0) atomicAdd(FtV + x, acc[x]);
}

}  // namespace

extern "C" int cptc_gen_unit_sums_plan(const uint32_t* h_unit6, size_t nunits, int max_chunk,
                                       uint32_t* h_order, uint32_t* h_chunk_off, size_t* nchunks)
{
    CPTC_REQUIRE(h_unit6 && h_order && h_chunk_off && nchunks && max_chunk >= 1, CPTC_ERR_ARG,
                 "cptc_gen_unit_sums_plan: bad arguments");
    CPTC_REQUIRE(nunits < (size_t(1) << 32), CPTC_ERR_ARG, "cptc_gen_unit_sums_plan: %zu units",
                 nunits);
    auto key = [&](uint32_t u) {
        const uint32_t* h = h_unit6 + size_t(u) * 6;
        return (uint64_t(h[0]) << 42) | (uint64_t(h[1]) << 21) | uint64_t(h[2]);
    };
    for (size_t u = 0; u < nunits; ++u) h_order[u] = uint32_t(u);
    std::stable_sort(h_order, h_order + nunits,
                     [&](uint32_t a, uint32_t b) { return key(a) < key(b); });
    size_t n = 0;
    for (size_t i = 0; i < nunits;)
    {
        h_chunk_off[n++] = uint32_t(i);
        const uint64_t k = key(h_order[i]);
        size_t j = i + 1;
        while (j < nunits && j - i < size_t(max_chunk) && key(h_order[j]) == k) ++j;
        i = j;
    }
    h_chunk_off[n] = uint32_t(nunits);
    *nchunks = n;
    return CPTC_OK;
}

extern "C" int cptc_gen_unit_sums(const uint32_t* d_unit6, size_t nunits, const uint32_t* d_lid,
                                  const double* d_val, const uint32_t* d_order,
                                  const uint32_t* d_chunk_off, size_t nchunks, const double* d_Fa,
                                  const double* d_Fb, const double* d_Fc, int da, int db, int dc,
                                  int R, double* d_sums, void* stream)
{
    CPTC_REQUIRE(R >= 1 && R <= USUM_R && da >= 1 && db >= 1 && dc >= 1, CPTC_ERR_ARG,
                 "cptc_gen_unit_sums: R %d (1..%d) or dims", R, USUM_R);
    if (nunits == 0) return CPTC_OK;
    CPTC_REQUIRE(d_unit6 && d_lid && d_val && d_order && d_chunk_off && d_Fa && d_Fb && d_Fc &&
                     d_sums && nchunks >= 1,
                 CPTC_ERR_ARG, "cptc_gen_unit_sums: null pointer or no chunks");
    CPTC_REQUIRE(nchunks <= nunits && nchunks < (size_t(1) << 31), CPTC_ERR_ARG,
                 "cptc_gen_unit_sums: %zu chunks for %zu units", nchunks, nunits);
    hipStream_t s = cptc::as_stream(stream);
    const dim3 grid{unsigned(nchunks)}, block{64 * USUM_WAVES};
    if (R <= 8)
        hipLaunchKernelGGL(unit_sums_kernel<8>, grid, block, 0, s, d_unit6, d_order, d_chunk_off,
                           d_lid, d_val, d_Fa, d_Fb, d_Fc, da, db, dc, R, d_sums);
    else if (R <= 16)
        hipLaunchKernelGGL(unit_sums_kernel<16>, grid, block, 0, s, d_unit6, d_order, d_chunk_off,
                           d_lid, d_val, d_Fa, d_Fb, d_Fc, da, db, dc, R, d_sums);
    else
        hipLaunchKernelGGL(unit_sums_kernel<32>, grid, block, 0, s, d_unit6, d_order, d_chunk_off,
                           d_lid, d_val, d_Fa, d_Fb, d_Fc, da, db, dc, R, d_sums);
    CPTC_LAUNCHED();
    return CPTC_OK;
}

extern "C" int cptc_gen_unit_sums_img(const uint32_t* d_unit6, size_t nunits, const double* d_img,
                                      const uint32_t* d_order, const uint32_t* d_chunk_off,
                                      size_t nchunks, const double* d_Fa, const double* d_Fb,
                                      const double* d_Fc, int da, int db, int dc, int R,
                                      double* d_sums, void* stream)
{
    CPTC_REQUIRE(R >= 1 && R <= USUM_R && da >= 1 && db >= 1 && dc >= 1, CPTC_ERR_ARG,
                 "cptc_gen_unit_sums_img: R %d (1..%d) or dims", R, USUM_R);
    if (nunits == 0) return CPTC_OK;
    CPTC_REQUIRE(d_unit6 && d_img && d_order && d_chunk_off && d_Fa && d_Fb && d_Fc && d_sums &&
                     nchunks >= 1,
                 CPTC_ERR_ARG, "cptc_gen_unit_sums_img: null pointer or no chunks");
    CPTC_REQUIRE((reinterpret_cast<uintptr_t>(d_img) & 15) == 0, CPTC_ERR_ARG,
                 "cptc_gen_unit_sums_img: the image must be 16-byte aligned");
    CPTC_REQUIRE(nchunks <= nunits && nchunks < (size_t(1) << 31), CPTC_ERR_ARG,
                 "cptc_gen_unit_sums_img: %zu chunks for %zu units", nchunks, nunits);
    hipStream_t s = cptc::as_stream(stream);
    const dim3 grid{unsigned(nchunks)}, block{64 * USUM_WAVES};
    if (R <= 16)
        hipLaunchKernelGGL(unit_sums_mfma_kernel<1>, grid, block, 0, s, d_unit6, d_order,
                           d_chunk_off, d_img, d_Fa, d_Fb, d_Fc, da, db, dc, R, d_sums);
    else
        hipLaunchKernelGGL(unit_sums_mfma_kernel<2>, grid, block, 0, s, d_unit6, d_order,
                           d_chunk_off, d_img, d_Fa, d_Fb, d_Fc, da, db, dc, R, d_sums);
    CPTC_LAUNCHED();
    return CPTC_OK;
}

extern "C" int cptc_gen_unit_scatter(const uint32_t* d_outer_coords, size_t nunits, int nouter,
                                     int pos, const double* const* d_Fo, const double* d_sums,
                                     int R, size_t dim_m, double* d_FtV, void* stream)
{
    CPTC_REQUIRE(R >= 1 && R <= 64 && nouter >= 1 && pos >= 0 && pos < nouter, CPTC_ERR_ARG,
                 "cptc_gen_unit_scatter: bad arguments");
    if (nunits == 0) return CPTC_OK;
    CPTC_REQUIRE(d_outer_coords && d_Fo && d_sums && d_FtV, CPTC_ERR_ARG,
                 "cptc_gen_unit_scatter: null pointer");
    hipLaunchKernelGGL(unit_scatter_kernel, dim3(unsigned((nunits + 255) / 256)), dim3(256), 0,
                       cptc::as_stream(stream), d_outer_coords, nunits, nouter, pos, d_Fo, d_sums,
                       R, dim_m, d_FtV);
    CPTC_LAUNCHED();
    return CPTC_OK;
}
