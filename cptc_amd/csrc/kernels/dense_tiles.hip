// Dense 16^3 tiles on CDNA4 FP32 MFMA with FP64 output accumulation — the
// gfx950 counterpart of dense_tile_mttkrp_wmma (dense.cu:89-1077) for
// order-3 tiles and of g_dense_tile_mttkrp_kernel (generic.cu:429-561) for
// the generic path's dense units, whose contribution is also scaled by the
// unit's FP64 outer-mode weights.  gfx950 has no xf32, so the inner products
// run in FP32, which is more accurate than the reference's TF32.
//
// For target mode 0, one tile and one 16-rank block rb:
//   out[i, r] = sum_{j,k} T[i, j, k] * (B[b1 + j, rb + r] * C[b2 + k, rb + r])
//   FtV[b0 + i, rb + r] += out[i, r]                 (FP64, one atomic)
// i.e. a 16 x 256 x 16 product of the tile with the Khatri-Rao block of the
// other two factors.  The reference contracts one factor per k-slice on the
// tensor cores and weights each slice by the third factor in FP64
// (dense.cu:406-549); the same sum in one MFMA chain per rank block needs
// no per-slice epilogue.  Mode 1 contracts (i, k) against A and C, mode 2
// (i, j) against A and B.
//
// One wave64 owns one tile (or a group of tiles with the same target block).
// v_mfma_f32_16x16x4f32 lane layout (CDNA3/4):
//   A[m][kk]: lane = m + 16*kk;  B[kk][n]: lane = n + 16*kk;
//   D[m][n]:  lane = n + 16*(m/4), element m%4.
// The lane's 64 tile cells for all 64 K-steps are held in registers (the
// tile is read from HBM once per launch).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cfloat>
#include <cstdlib>
#include <vector>

#include "../host/hip_util.hpp"
#include "tiles_b3_body.hpp"
#include "tiles_body.hpp"

namespace {

constexpr int WAVE = 64;
constexpr int WAVES_PER_WG = 4;

// The kernel body (cptc_k::dense_tiles_body) is in tiles_body.hpp.
template <int MODE, int HDR, bool HAS_W, bool GROUPED>
__global__ __launch_bounds__(WAVE* WAVES_PER_WG) __attribute__((amdgpu_waves_per_eu(2, 2))) void dense_tiles_kernel(
    const int32_t* __restrict__ hdr, const float* __restrict__ tile_f32, size_t ntiles,
    const uint32_t* __restrict__ order, const uint32_t* __restrict__ goff, size_t ngroups,
    const double* __restrict__ A, const double* __restrict__ B, const double* __restrict__ C,
    const double* __restrict__ W, double* __restrict__ FtV, int R, int Rp, int dimI, int dimJ,
    int dimK, int S)
{
    extern __shared__ double gacc_lds[];
    cptc_k::dense_tiles_body<MODE, HDR, HAS_W, GROUPED>(blockIdx.x, gacc_lds, hdr, tile_f32,
                                                        ntiles, order, goff, ngroups, A, B, C, W,
                                                        FtV, R, Rp, dimI, dimJ, dimK, S);
}

// Split-bf16 variant (cptc_k::dense_tiles_b3_body in tiles_b3_body.hpp);
// COMPACT reads the compacted tile image (cmask / csegoff / cseg).
template <int MODE, int HDR, bool HAS_W, bool GROUPED, bool COMPACT>
#ifndef CPTC_B3_WAVES
#define CPTC_B3_WAVES 2   // resident waves per SIMD of the split-bf16 kernel
#endif
#ifndef CPTC_B3_SMIN
#define CPTC_B3_SMIN 1    // least waves per tile (rank split) of its grouped form
#endif
__global__ __launch_bounds__(WAVE* WAVES_PER_WG) __attribute__((amdgpu_waves_per_eu(CPTC_B3_WAVES, CPTC_B3_WAVES))) void dense_tiles_b3_kernel(
    const int32_t* __restrict__ hdr, const float* __restrict__ tile_f32,
    const uint32_t* __restrict__ cmask, const uint32_t* __restrict__ csegoff,
    const cptc_k::u32x4* __restrict__ cseg, size_t ntiles, const uint32_t* __restrict__ order,
    const uint32_t* __restrict__ goff, size_t ngroups, const cptc_k::u32x4* __restrict__ fs_hi,
    const cptc_k::u32x4* __restrict__ fs_lo, const float4* __restrict__ fw,
    const double* __restrict__ W, double* __restrict__ FtV, int R, int Rq, int odim, int S)
{
    extern __shared__ double gacc_lds[];
    cptc_k::dense_tiles_b3_body<MODE, HDR, HAS_W, GROUPED, COMPACT>(
        blockIdx.x, gacc_lds, hdr, tile_f32, cmask, csegoff, cseg, ntiles, order, goff, ngroups,
        fs_hi, fs_lo, fw, W, FtV, R, Rq, odim, S);
}

// Compacted split image of one target slot, the split-bf16 kernel's A
// operand: tile cell (a, w, c) (target, weight and contracted coordinate of
// the slot) is image cell (a, c, w) for slot 0, (c, a, w) for slot 1 and
// (c, w, a) for slot 2 (the image is [i][j][k], k fastest).  Segment
// s = a * 64 + w * 4 + e holds the cells c = 4e .. 4e + 3 as 4 bf16 hi
// halves then their 4 bf16 lo halves (16 bytes; the kernel's split of each
// value, so the products are the same bits); it is occupied when any of its
// 4 FP32 cells has a nonzero bit.  cmask[64 t + x], x < 32: occupancy bits
// of segments 32x .. 32x + 31; cmask[64 t + 32 + x]: occupied segments
// before word x; the occupied segments in order at seg[segoff[t] ..].
template <int SLOT>
__device__ __forceinline__ int slot_cell(int a, int w, int c)
{
    if constexpr (SLOT == 0) return (a * 16 + c) * 16 + w;
    if constexpr (SLOT == 1) return (c * 16 + a) * 16 + w;
    return (c * 16 + w) * 16 + a;
}

// pass 1: the occupancy words and running counts; counts[t] = occupied segments
template <int SLOT>
__global__ __launch_bounds__(256) void compact_split_mask_kernel(const float* __restrict__ tiles,
                                                                 uint32_t* __restrict__ cmask,
                                                                 uint32_t* __restrict__ counts)
{
    __shared__ uint32_t wmask[32];
    const size_t t = blockIdx.x;
    if (threadIdx.x < 32) wmask[threadIdx.x] = 0u;
    __syncthreads();
    const uint32_t* __restrict__ src = reinterpret_cast<const uint32_t*>(tiles + t * 4096);
    for (int sg = threadIdx.x; sg < 1024; sg += 256)
    {
        const int a = sg >> 6, w = (sg >> 2) & 15, e = sg & 3;
        uint32_t any = 0u;
#pragma unroll
        for (int q = 0; q < 4; ++q) any |= src[slot_cell<SLOT>(a, w, 4 * e + q)];
        if (any != 0u) atomicOr(&wmask[sg >> 5], 1u << (sg & 31));
    }
    __syncthreads();
    if (threadIdx.x == 0)
    {
        uint32_t run = 0;
        for (int x = 0; x < 32; ++x)
        {
            cmask[t * 64 + x] = wmask[x];
            cmask[t * 64 + 32 + x] = run;
            run += uint32_t(__builtin_popcount(wmask[x]));
        }
        counts[t] = run;
    }
}

// pass 2: the occupied segments of tile t, split, in segment order at segoff[t]
template <int SLOT>
__global__ __launch_bounds__(256) void compact_split_fill_kernel(const float* __restrict__ tiles,
                                                                 const uint32_t* __restrict__ cmask,
                                                                 const uint32_t* __restrict__ segoff,
                                                                 uint4* __restrict__ seg)
{
    const size_t t = blockIdx.x;
    const float* __restrict__ src = tiles + t * 4096;
    const uint32_t* __restrict__ mp = cmask + t * 64;
    for (int sg = threadIdx.x; sg < 1024; sg += 256)
    {
        const int a = sg >> 6, w = (sg >> 2) & 15, e = sg & 3;
        const int x = sg >> 5, b = sg & 31;
        const uint32_t m = mp[x];
        if (!((m >> b) & 1u)) continue;
        uint32_t hv[2], lv[2];
#pragma unroll
        for (int d = 0; d < 2; ++d)
        {
            const float x0 = src[slot_cell<SLOT>(a, w, 4 * e + 2 * d)];
            const float x1 = src[slot_cell<SLOT>(a, w, 4 * e + 2 * d + 1)];
            cptc_k::split_bf16x2(x0, x1, hv[d], lv[d],
                                 __builtin_amdgcn_fmed3f(x0, -cptc_k::BF16_MAX, cptc_k::BF16_MAX),
                                 __builtin_amdgcn_fmed3f(x1, -cptc_k::BF16_MAX, cptc_k::BF16_MAX));
        }
        seg[size_t(segoff[t]) + mp[32 + x] + uint32_t(__builtin_popcount(m & ((1u << b) - 1u)))] =
            make_uint4(hv[0], hv[1], lv[0], lv[1]);
    }
}

// A factor entry, or 0 past the factor's rows or ranks: the load is made
// from a clamped address on every path and zeroed by an AND with a mask an
// empty asm has made opaque (a `cond ? load : 0` lets the compiler put each
// load under a branch with a memory wait of its own).
__device__ __forceinline__ float operand_entry(const double* __restrict__ F, int row, int dim,
                                               int r, int R)
{
    const double v = F[size_t(max(0, min(row, dim - 1))) * R + min(r, R - 1)];
    long long m = (row < dim && r < R) ? -1LL : 0LL;
    asm volatile("" : "+v"(m));
    return float(__longlong_as_double(__double_as_longlong(v) & m));
}

// Operand images of the split-bf16 kernel for one target slot: the
// contracted factor Fc split into bf16 hi / lo, 8 rows of one rank per 16
// bytes ([row / 8][Rq]), and the weight factor in FP32, 16 rows of one rank
// per 64 bytes ([row / 16][Rq]); rows past the factor and ranks >= R are 0.
__global__ __launch_bounds__(256) void tile_operands_kernel(
    const double* __restrict__ Fc, int cdim, const double* __restrict__ Fw, int wdim, int R,
    int Rq, size_t nc, size_t nw, cptc_k::u32x4* __restrict__ fs_hi,
    cptc_k::u32x4* __restrict__ fs_lo, float4* __restrict__ fw)
{
    const size_t idx = size_t(blockIdx.x) * 256 + threadIdx.x;
    if (idx < nc)
    {
        const int b = int(idx / size_t(Rq)), r = int(idx % size_t(Rq));
        float x[8];
#pragma unroll
        for (int q = 0; q < 8; ++q)
        {
            x[q] = operand_entry(Fc, 8 * b + q, cdim, r, R);
        }
        cptc_k::u32x4 hv, lv;
#pragma unroll
        for (int s = 0; s < 4; ++s)
        {
            uint32_t hh, ll;
            cptc_k::split_bf16x2(x[2 * s], x[2 * s + 1], hh, ll);
            hv[s] = hh;
            lv[s] = ll;
        }
        fs_hi[idx] = hv;
        fs_lo[idx] = lv;
    }
    else if (idx < nc + nw)
    {
        const size_t k = idx - nc;
        const int b = int(k / size_t(Rq)), r = int(k % size_t(Rq));
        float x[16];
#pragma unroll
        for (int u = 0; u < 16; ++u)
        {
            x[u] = operand_entry(Fw, 16 * b + u, wdim, r, R);
        }
#pragma unroll
        for (int s = 0; s < 4; ++s)
            fw[k * 4 + s] = make_float4(x[4 * s], x[4 * s + 1], x[4 * s + 2], x[4 * s + 3]);
    }
}

// Tile materialisation: cell value of the last pool entry per lid (pool
// order), clamped to +-FLT_MAX (dense.cu:150-190), 0 elsewhere.
__global__ __launch_bounds__(256) void pack_tiles_kernel(const int32_t* __restrict__ lid,
                                                         const double* __restrict__ val,
                                                         const uint64_t* __restrict__ off,
                                                         float* __restrict__ out)
{
    __shared__ int win[4096];
    const size_t t = blockIdx.x;
    for (int c = threadIdx.x; c < 4096; c += 256) win[c] = -1;
    __syncthreads();
    const uint64_t lo = off[t], hi = off[t + 1];
    for (uint64_t e = lo + threadIdx.x; e < hi; e += 256) atomicMax(&win[lid[e] & 4095], int(e - lo));
    __syncthreads();
    for (int c = threadIdx.x; c < 4096; c += 256)
    {
        float f = 0.0f;
        if (win[c] >= 0)
        {
            double x = val[lo + uint64_t(win[c])];
            x = x > double(FLT_MAX) ? double(FLT_MAX) : (x < -double(FLT_MAX) ? -double(FLT_MAX) : x);
            f = float(x);
        }
        out[t * 4096 + c] = f;
    }
}

}  // namespace

extern "C" int cptc_dense_tiles_pack3(const int32_t* d_pool_lid, const double* d_pool_val,
                                      const uint64_t* d_pool_off, size_t ntiles, float* d_tile_f32,
                                      void* stream)
{
    if (ntiles == 0) return CPTC_OK;
    CPTC_REQUIRE(d_pool_lid && d_pool_val && d_pool_off && d_tile_f32, CPTC_ERR_ARG,
                 "cptc_dense_tiles_pack3: null pointer");
    CPTC_REQUIRE(ntiles < (size_t(1) << 31), CPTC_ERR_ARG, "cptc_dense_tiles_pack3: too many tiles");
    hipLaunchKernelGGL(pack_tiles_kernel, dim3(unsigned(ntiles)), dim3(256), 0,
                       cptc::as_stream(stream), d_pool_lid, d_pool_val, d_pool_off, d_tile_f32);
    CPTC_LAUNCHED();
    return CPTC_OK;
}

namespace {

constexpr int GROUP_LDS_MAX_R = 128;   // 4 waves x 16 rows x 128 ranks x 8 B = 64 KB

// Rank-block split: S waves per tile / group (wave s takes the group's
// 16-rank blocks s, s + S, ...; every (row, rank) is still summed by one
// wave in the same order).  Used when the tiles or groups alone give fewer
// waves than the chip has SIMDs; CPTC_TILE_SPLIT=<n> fixes it (tuning).
int rank_split(size_t items, int R, hipStream_t s)
{
    const int nrb = (R + 15) / 16;
    static const int fixed = [] {
        const char* e = std::getenv("CPTC_TILE_SPLIT");
        return e ? std::atoi(e) : 0;
    }();
    if (fixed > 0) return std::min(fixed, nrb);
    int dev = 0;
    if (hipStreamGetDevice(s, &dev) != hipSuccess || dev < 0) dev = 0;
    const size_t want = size_t(4) * size_t(cptc::cu_count(dev));   // SIMDs
    if (items >= want) return 1;
    return int(std::min<size_t>((want + items - 1) / items, size_t(nrb)));
}

template <int MODE, int HDR, bool HAS_W>
int launch_tiles(const int32_t* hdr, const float* tiles, size_t ntiles, const uint32_t* order,
                 const uint32_t* goff, size_t ngroups, const double* A, const double* B,
                 const double* C, const double* W, double* FtV, int R, int dI, int dJ, int dK,
                 hipStream_t s)
{
    const dim3 block{WAVE * WAVES_PER_WG};
    const bool grouped = order && goff && ngroups > 0 && R <= GROUP_LDS_MAX_R;
    const size_t items = grouped ? ngroups : ntiles;
    const int S = rank_split(items, R, s);
    const size_t wgs = (items * size_t(S) + WAVES_PER_WG - 1) / WAVES_PER_WG;
    CPTC_REQUIRE(wgs < (size_t(1) << 31), CPTC_ERR_ARG, "dense tiles: too many tiles");
    if (grouped)
    {
        const int Rp = (R + 15) / 16 * 16;
        const size_t lds = size_t(WAVES_PER_WG) * 16 * Rp * sizeof(double);
        hipLaunchKernelGGL((dense_tiles_kernel<MODE, HDR, HAS_W, true>),
                           dim3(static_cast<unsigned>(wgs)), block, lds, s, hdr, tiles, ntiles,
                           order, goff, ngroups, A, B, C, W, FtV, R, Rp, dI, dJ, dK, S);
    }
    else
    {
        hipLaunchKernelGGL((dense_tiles_kernel<MODE, HDR, HAS_W, false>),
                           dim3(static_cast<unsigned>(wgs)), block, 0, s, hdr, tiles, ntiles,
                           nullptr, nullptr, size_t(0), A, B, C, W, FtV, R, R, dI, dJ, dK, S);
    }
    CPTC_LAUNCHED();
    return CPTC_OK;
}

// Workspace of the split-bf16 kernel: operand images for contracted and
// weight factors of up to `maxdim` rows.
size_t b3_bytes(uint64_t maxdim, int R)
{
    const size_t Rq = size_t(R + 31) / 32 * 32;
    const size_t d16 = size_t((maxdim + 15) / 16) * 16;
    return Rq * d16 * 4 /* hi + lo bf16 */ + Rq * d16 * 4 /* FP32 */ + 256;
}

// compacted split image of the launch's target slot (all null: the dense
// tile_f32 image)
struct CompactImg
{
    const uint32_t* mask = nullptr;
    const uint32_t* segoff = nullptr;
    const cptc_k::u32x4* seg = nullptr;
};

template <int MODE, int HDR, bool HAS_W>
int launch_tiles_b3(const int32_t* hdr, const float* tiles, CompactImg ci, size_t ntiles,
                    const uint32_t* order, const uint32_t* goff, size_t ngroups, const double* Fc,
                    int cdim, const double* Fw, int wdim, const double* W, double* FtV, int R,
                    int odim, void* ws, size_t ws_bytes, hipStream_t s)
{
    const bool compact = ci.mask != nullptr;
    const int Rq = (R + 31) / 32 * 32;
    const size_t nc = size_t((cdim + 15) / 16) * 2 * size_t(Rq);   // 8-row blocks x Rq
    const size_t nw = size_t((wdim + 15) / 16) * size_t(Rq);        // 16-row blocks x Rq
    const size_t need = nc * 32 + nw * 64;
    CPTC_REQUIRE(ws && ws_bytes >= need && (reinterpret_cast<uintptr_t>(ws) & 255) == 0,
                 CPTC_ERR_ARG, "dense tiles (bf16 split): workspace %zu bytes, need %zu (256-aligned)",
                 ws_bytes, need);
    auto* fs_hi = static_cast<cptc_k::u32x4*>(ws);
    auto* fs_lo = fs_hi + nc;
    auto* fw = reinterpret_cast<float4*>(fs_lo + nc);
    const size_t nthreads = nc + nw;
    hipLaunchKernelGGL(tile_operands_kernel, dim3(unsigned((nthreads + 255) / 256)), dim3(256), 0,
                       s, Fc, cdim, Fw, wdim, R, Rq, nc, nw, fs_hi, fs_lo, fw);
    CPTC_LAUNCHED();
    const dim3 block{WAVE * WAVES_PER_WG};
    const bool grouped = order && goff && ngroups > 0 && Rq <= GROUP_LDS_MAX_R;
    const size_t items = grouped ? ngroups : ntiles;
    int S = rank_split(items, Rq / 2, s);   // 32-rank blocks
    if (grouped) S = std::min(std::max(S, CPTC_B3_SMIN), Rq / 32);
    const size_t wgs = (items * size_t(S) + WAVES_PER_WG - 1) / WAVES_PER_WG;
    CPTC_REQUIRE(wgs < (size_t(1) << 31), CPTC_ERR_ARG, "dense tiles: too many tiles");
    if (grouped)
    {
        // per wave 16 rows x its rank blocks (<= 64 KB per workgroup)
        const size_t lds = size_t(WAVES_PER_WG) * 16 * size_t((Rq / 32 + S - 1) / S * 32) *
                           sizeof(double);
        if (compact)
            hipLaunchKernelGGL((dense_tiles_b3_kernel<MODE, HDR, HAS_W, true, true>),
                               dim3(static_cast<unsigned>(wgs)), block, lds, s, hdr, tiles,
                               ci.mask, ci.segoff, ci.seg, ntiles, order, goff, ngroups, fs_hi,
                               fs_lo, fw, W, FtV, R, Rq, odim, S);
        else
            hipLaunchKernelGGL((dense_tiles_b3_kernel<MODE, HDR, HAS_W, true, false>),
                               dim3(static_cast<unsigned>(wgs)), block, lds, s, hdr, tiles,
                               ci.mask, ci.segoff, ci.seg, ntiles, order, goff, ngroups, fs_hi,
                               fs_lo, fw, W, FtV, R, Rq, odim, S);
    }
    else
    {
        if (compact)
            hipLaunchKernelGGL((dense_tiles_b3_kernel<MODE, HDR, HAS_W, false, true>),
                               dim3(static_cast<unsigned>(wgs)), block, 0, s, hdr, tiles, ci.mask,
                               ci.segoff, ci.seg, ntiles, nullptr, nullptr, size_t(0), fs_hi,
                               fs_lo, fw, W, FtV, R, Rq, odim, S);
        else
            hipLaunchKernelGGL((dense_tiles_b3_kernel<MODE, HDR, HAS_W, false, false>),
                               dim3(static_cast<unsigned>(wgs)), block, 0, s, hdr, tiles, ci.mask,
                               ci.segoff, ci.seg, ntiles, nullptr, nullptr, size_t(0), fs_hi,
                               fs_lo, fw, W, FtV, R, Rq, odim, S);
    }
    CPTC_LAUNCHED();
    return CPTC_OK;
}

// slot 0: contract slot 1, weight slot 2; slot 1: contract 0, weight 2;
// slot 2: contract 0, weight 1
template <int HDR, bool HAS_W>
int launch_slot_b3(int slot, const int32_t* hdr, const float* tiles, CompactImg ci, size_t ntiles,
                   const uint32_t* order, const uint32_t* goff, size_t ngroups, const double* F0,
                   const double* F1, const double* F2, const double* W, double* FtV, int R,
                   int d0, int d1, int d2, void* ws, size_t ws_bytes, hipStream_t s)
{
    if (slot == 0)
        return launch_tiles_b3<0, HDR, HAS_W>(hdr, tiles, ci, ntiles, order, goff, ngroups, F1, d1,
                                              F2, d2, W, FtV, R, d0, ws, ws_bytes, s);
    if (slot == 1)
        return launch_tiles_b3<1, HDR, HAS_W>(hdr, tiles, ci, ntiles, order, goff, ngroups, F0, d0,
                                              F2, d2, W, FtV, R, d1, ws, ws_bytes, s);
    return launch_tiles_b3<2, HDR, HAS_W>(hdr, tiles, ci, ntiles, order, goff, ngroups, F0, d0, F1,
                                          d1, W, FtV, R, d2, ws, ws_bytes, s);
}

template <int HDR, bool HAS_W>
int launch_slot(int slot, const int32_t* hdr, const float* tiles, size_t ntiles,
                const uint32_t* order, const uint32_t* goff, size_t ngroups, const double* A,
                const double* B, const double* C, const double* W, double* FtV, int R, int dI,
                int dJ, int dK, hipStream_t s)
{
    if (slot == 0)
        return launch_tiles<0, HDR, HAS_W>(hdr, tiles, ntiles, order, goff, ngroups, A, B, C, W,
                                           FtV, R, dI, dJ, dK, s);
    if (slot == 1)
        return launch_tiles<1, HDR, HAS_W>(hdr, tiles, ntiles, order, goff, ngroups, A, B, C, W,
                                           FtV, R, dI, dJ, dK, s);
    return launch_tiles<2, HDR, HAS_W>(hdr, tiles, ntiles, order, goff, ngroups, A, B, C, W, FtV,
                                       R, dI, dJ, dK, s);
}

}  // namespace

extern "C" int cptc_mttkrp_dense_tiles3(int mode, const int32_t* d_tiles, const float* d_tile_f32,
                                        size_t ntiles, const uint32_t* d_order,
                                        const uint32_t* d_group_off, size_t ngroups,
                                        const double* d_A, const double* d_B, const double* d_C,
                                        double* d_FtV, int R, int dimI, int dimJ, int dimK,
                                        void* stream)
{
    CPTC_REQUIRE(mode >= 0 && mode < 3 && R >= 1, CPTC_ERR_ARG,
                 "cptc_mttkrp_dense_tiles3: mode %d R %d", mode, R);
    if (ntiles == 0) return CPTC_OK;
    CPTC_REQUIRE(d_tiles && d_tile_f32 && d_A && d_B && d_C && d_FtV, CPTC_ERR_ARG,
                 "cptc_mttkrp_dense_tiles3: null pointer");
    return launch_slot<4, false>(mode, d_tiles, d_tile_f32, ntiles, d_order, d_group_off, ngroups,
                                 d_A, d_B, d_C, nullptr, d_FtV, R, dimI, dimJ, dimK,
                                 cptc::as_stream(stream));
}

extern "C" size_t cptc_tile_operands_bytes(uint64_t max_dim, int R)
{
    return R >= 1 ? b3_bytes(max_dim, R) : 0;
}

extern "C" int cptc_mttkrp_dense_tiles3_ws(int mode, const int32_t* d_tiles,
                                           const float* d_tile_f32, size_t ntiles,
                                           const uint32_t* d_order, const uint32_t* d_group_off,
                                           size_t ngroups, const double* d_A, const double* d_B,
                                           const double* d_C, double* d_FtV, int R, int dimI,
                                           int dimJ, int dimK, void* d_ws, size_t ws_bytes,
                                           void* stream)
{
    CPTC_REQUIRE(mode >= 0 && mode < 3 && R >= 1, CPTC_ERR_ARG,
                 "cptc_mttkrp_dense_tiles3_ws: mode %d R %d", mode, R);
    if (ntiles == 0) return CPTC_OK;
    CPTC_REQUIRE(d_tiles && d_tile_f32 && d_A && d_B && d_C && d_FtV, CPTC_ERR_ARG,
                 "cptc_mttkrp_dense_tiles3_ws: null pointer");
    return launch_slot_b3<4, false>(mode, d_tiles, d_tile_f32, CompactImg{}, ntiles, d_order,
                                    d_group_off, ngroups, d_A, d_B, d_C, nullptr, d_FtV, R, dimI,
                                    dimJ, dimK, d_ws, ws_bytes, cptc::as_stream(stream));
}

extern "C" int cptc_dense_tiles_compact3_mask(const float* d_tile_f32, size_t ntiles, int slot,
                                              uint32_t* d_cmask, uint32_t* d_segoff,
                                              uint64_t* total_segments, void* stream)
{
    CPTC_REQUIRE(total_segments, CPTC_ERR_ARG, "cptc_dense_tiles_compact3_mask: null total");
    *total_segments = 0;
    CPTC_REQUIRE(slot >= 0 && slot < 3, CPTC_ERR_ARG, "cptc_dense_tiles_compact3_mask: slot %d",
                 slot);
    if (ntiles == 0) return CPTC_OK;
    CPTC_REQUIRE(d_tile_f32 && d_cmask && d_segoff && ntiles < (size_t(1) << 31), CPTC_ERR_ARG,
                 "cptc_dense_tiles_compact3_mask: bad arguments");
    hipStream_t s = cptc::as_stream(stream);
    uint32_t* counts = nullptr;
    CPTC_HIP(hipMallocAsync(reinterpret_cast<void**>(&counts), ntiles * sizeof(uint32_t), s));
    if (slot == 0)
        hipLaunchKernelGGL(compact_split_mask_kernel<0>, dim3(unsigned(ntiles)), dim3(256), 0, s,
                           d_tile_f32, d_cmask, counts);
    else if (slot == 1)
        hipLaunchKernelGGL(compact_split_mask_kernel<1>, dim3(unsigned(ntiles)), dim3(256), 0, s,
                           d_tile_f32, d_cmask, counts);
    else
        hipLaunchKernelGGL(compact_split_mask_kernel<2>, dim3(unsigned(ntiles)), dim3(256), 0, s,
                           d_tile_f32, d_cmask, counts);
    hipError_t le = hipGetLastError();
    std::vector<uint32_t> h(ntiles);
    hipError_t ce = hipMemcpyAsync(h.data(), counts, ntiles * sizeof(uint32_t),
                                   hipMemcpyDeviceToHost, s);
    hipError_t se = hipStreamSynchronize(s);
    (void)hipFreeAsync(counts, s);
    CPTC_REQUIRE(le == hipSuccess && ce == hipSuccess && se == hipSuccess, CPTC_ERR_HIP,
                 "cptc_dense_tiles_compact3_mask: %s",
                 hipGetErrorString(le != hipSuccess ? le : ce != hipSuccess ? ce : se));
    std::vector<uint32_t> off(ntiles + 1);
    uint64_t run = 0;
    for (size_t t = 0; t < ntiles; ++t)
    {
        off[t] = uint32_t(run);
        run += h[t];
    }
    CPTC_REQUIRE(run < (uint64_t(1) << 32), CPTC_ERR_UNSUPPORTED,
                 "cptc_dense_tiles_compact3_mask: %llu segments exceed 32-bit offsets",
                 (unsigned long long)run);
    off[ntiles] = uint32_t(run);
    CPTC_HIP(hipMemcpyAsync(d_segoff, off.data(), off.size() * sizeof(uint32_t),
                            hipMemcpyHostToDevice, s));
    CPTC_HIP(hipStreamSynchronize(s));
    *total_segments = run;
    return CPTC_OK;
}

extern "C" int cptc_dense_tiles_compact3_fill(const float* d_tile_f32, size_t ntiles, int slot,
                                              const uint32_t* d_cmask, const uint32_t* d_segoff,
                                              void* d_seg, void* stream)
{
    CPTC_REQUIRE(slot >= 0 && slot < 3, CPTC_ERR_ARG, "cptc_dense_tiles_compact3_fill: slot %d",
                 slot);
    if (ntiles == 0) return CPTC_OK;
    CPTC_REQUIRE(d_tile_f32 && d_cmask && d_segoff && d_seg && ntiles < (size_t(1) << 31),
                 CPTC_ERR_ARG, "cptc_dense_tiles_compact3_fill: bad arguments");
    CPTC_REQUIRE((reinterpret_cast<uintptr_t>(d_seg) & 15) == 0, CPTC_ERR_ARG,
                 "cptc_dense_tiles_compact3_fill: segments must be 16-byte aligned");
    hipStream_t s = cptc::as_stream(stream);
    uint4* seg = static_cast<uint4*>(d_seg);
    if (slot == 0)
        hipLaunchKernelGGL(compact_split_fill_kernel<0>, dim3(unsigned(ntiles)), dim3(256), 0, s,
                           d_tile_f32, d_cmask, d_segoff, seg);
    else if (slot == 1)
        hipLaunchKernelGGL(compact_split_fill_kernel<1>, dim3(unsigned(ntiles)), dim3(256), 0, s,
                           d_tile_f32, d_cmask, d_segoff, seg);
    else
        hipLaunchKernelGGL(compact_split_fill_kernel<2>, dim3(unsigned(ntiles)), dim3(256), 0, s,
                           d_tile_f32, d_cmask, d_segoff, seg);
    CPTC_LAUNCHED();
    return CPTC_OK;
}

extern "C" int cptc_mttkrp_dense_tiles3_cws(int mode, const int32_t* d_tiles,
                                            const uint32_t* d_cmask, const uint32_t* d_segoff,
                                            const void* d_seg, uint64_t nseg, size_t ntiles,
                                            const uint32_t* d_order, const uint32_t* d_group_off,
                                            size_t ngroups, const double* d_A, const double* d_B,
                                            const double* d_C, double* d_FtV, int R, int dimI,
                                            int dimJ, int dimK, void* d_ws, size_t ws_bytes,
                                            void* stream)
{
    CPTC_REQUIRE(mode >= 0 && mode < 3 && R >= 1, CPTC_ERR_ARG,
                 "cptc_mttkrp_dense_tiles3_cws: mode %d R %d", mode, R);
    if (ntiles == 0) return CPTC_OK;
    CPTC_REQUIRE(d_tiles && d_cmask && d_segoff && d_seg && d_A && d_B && d_C && d_FtV,
                 CPTC_ERR_ARG, "cptc_mttkrp_dense_tiles3_cws: null pointer");
    CPTC_REQUIRE((reinterpret_cast<uintptr_t>(d_seg) & 15) == 0, CPTC_ERR_ARG,
                 "cptc_mttkrp_dense_tiles3_cws: segments must be 16-byte aligned");
    // the kernel's 32-bit buffer offsets (an unoccupied segment reads at 2^32 - 16)
    CPTC_REQUIRE(nseg * 16u < 0xFFFFFFF0ull, CPTC_ERR_UNSUPPORTED,
                 "cptc_mttkrp_dense_tiles3_cws: %llu segments exceed 32-bit byte offsets",
                 (unsigned long long)nseg);
    CompactImg ci;
    ci.mask = d_cmask;
    ci.segoff = d_segoff;
    ci.seg = static_cast<const cptc_k::u32x4*>(d_seg);
    return launch_slot_b3<4, false>(mode, d_tiles, nullptr, ci, ntiles, d_order, d_group_off,
                                    ngroups, d_A, d_B, d_C, nullptr, d_FtV, R, dimI, dimJ, dimK,
                                    d_ws, ws_bytes, cptc::as_stream(stream));
}

extern "C" int cptc_mttkrp_units_nd_ws(int slot, const uint32_t* d_unit6, uint64_t nunits,
                                       const float* d_tiles, const double* d_W,
                                       const uint32_t* d_order, const uint32_t* d_group_off,
                                       size_t ngroups, const double* d_F0, const double* d_F1,
                                       const double* d_F2, int dim0, int dim1, int dim2,
                                       double* d_FtV, int R, void* d_ws, size_t ws_bytes,
                                       void* stream)
{
    CPTC_REQUIRE(slot >= 0 && slot < 3 && R >= 1, CPTC_ERR_ARG,
                 "cptc_mttkrp_units_nd_ws: slot %d R %d", slot, R);
    if (nunits == 0) return CPTC_OK;
    CPTC_REQUIRE(d_unit6 && d_tiles && d_W && d_F0 && d_F1 && d_F2 && d_FtV, CPTC_ERR_ARG,
                 "cptc_mttkrp_units_nd_ws: null pointer");
    return launch_slot_b3<6, true>(slot, reinterpret_cast<const int32_t*>(d_unit6), d_tiles,
                                   CompactImg{}, size_t(nunits), d_order, d_group_off, ngroups,
                                   d_F0, d_F1, d_F2, d_W, d_FtV, R, dim0, dim1, dim2, d_ws,
                                   ws_bytes, cptc::as_stream(stream));
}

extern "C" int cptc_mttkrp_units_nd_cws(int slot, const uint32_t* d_unit6, uint64_t nunits,
                                        const uint32_t* d_cmask, const uint32_t* d_segoff,
                                        const void* d_seg, uint64_t nseg, const double* d_W,
                                        const uint32_t* d_order, const uint32_t* d_group_off,
                                        size_t ngroups, const double* d_F0, const double* d_F1,
                                        const double* d_F2, int dim0, int dim1, int dim2,
                                        double* d_FtV, int R, void* d_ws, size_t ws_bytes,
                                        void* stream)
{
    CPTC_REQUIRE(slot >= 0 && slot < 3 && R >= 1, CPTC_ERR_ARG,
                 "cptc_mttkrp_units_nd_cws: slot %d R %d", slot, R);
    if (nunits == 0) return CPTC_OK;
    CPTC_REQUIRE(d_unit6 && d_cmask && d_segoff && d_seg && d_W && d_F0 && d_F1 && d_F2 && d_FtV,
                 CPTC_ERR_ARG, "cptc_mttkrp_units_nd_cws: null pointer");
    CPTC_REQUIRE((reinterpret_cast<uintptr_t>(d_seg) & 15) == 0, CPTC_ERR_ARG,
                 "cptc_mttkrp_units_nd_cws: segments must be 16-byte aligned");
    CPTC_REQUIRE(nseg * 16u < 0xFFFFFFF0ull, CPTC_ERR_UNSUPPORTED,
                 "cptc_mttkrp_units_nd_cws: %llu segments exceed 32-bit byte offsets",
                 (unsigned long long)nseg);
    CompactImg ci;
    ci.mask = d_cmask;
    ci.segoff = d_segoff;
    ci.seg = static_cast<const cptc_k::u32x4*>(d_seg);
    return launch_slot_b3<6, true>(slot, reinterpret_cast<const int32_t*>(d_unit6), nullptr, ci,
                                   size_t(nunits), d_order, d_group_off, ngroups, d_F0, d_F1, d_F2,
                                   d_W, d_FtV, R, dim0, dim1, dim2, d_ws, ws_bytes,
                                   cptc::as_stream(stream));
}

extern "C" int cptc_mttkrp_units_nd(int slot, const uint32_t* d_unit6, uint64_t nunits,
                                    const float* d_tiles, const double* d_W,
                                    const uint32_t* d_order, const uint32_t* d_group_off,
                                    size_t ngroups, const double* d_F0, const double* d_F1,
                                    const double* d_F2, int dim0, int dim1, int dim2,
                                    double* d_FtV, int R, void* stream)
{
    CPTC_REQUIRE(slot >= 0 && slot < 3 && R >= 1, CPTC_ERR_ARG,
                 "cptc_mttkrp_units_nd: slot %d R %d", slot, R);
    if (nunits == 0) return CPTC_OK;
    CPTC_REQUIRE(d_unit6 && d_tiles && d_W && d_F0 && d_F1 && d_F2 && d_FtV, CPTC_ERR_ARG,
                 "cptc_mttkrp_units_nd: null pointer");
    return launch_slot<6, true>(slot, reinterpret_cast<const int32_t*>(d_unit6), d_tiles,
                                size_t(nunits), d_order, d_group_off, ngroups, d_F0, d_F1, d_F2,
                                d_W, d_FtV, R, dim0, dim1, dim2, cptc::as_stream(stream));
}

// Host: tiles in (target block, other blocks) order, cut into runs of at
// most max_group tiles with one target block.
extern "C" int cptc_dense_groups(const int32_t* hdr, int hdr_words, size_t ntiles, int slot,
                                 int max_group, uint32_t* order_out, uint32_t* group_off_out,
                                 size_t* ngroups_out)
{
    CPTC_REQUIRE(hdr_words >= 3 && slot >= 0 && slot < 3 && max_group >= 1 &&
                     (ntiles == 0 || (hdr && order_out && group_off_out)) && ngroups_out,
                 CPTC_ERR_ARG, "cptc_dense_groups: bad arguments");
    CPTC_REQUIRE(ntiles < (size_t(1) << 32), CPTC_ERR_ARG, "cptc_dense_groups: too many tiles");
    const int p = (slot + 1) % 3, q = (slot + 2) % 3;
    std::vector<uint32_t> ord(ntiles);
    for (size_t t = 0; t < ntiles; ++t) ord[t] = uint32_t(t);
    auto key = [&](uint32_t t, int c) { return hdr[size_t(hdr_words) * t + c]; };
    std::stable_sort(ord.begin(), ord.end(), [&](uint32_t a, uint32_t b) {
        if (key(a, slot) != key(b, slot)) return key(a, slot) < key(b, slot);
        if (key(a, p) != key(b, p)) return key(a, p) < key(b, p);
        return key(a, q) < key(b, q);
    });
    size_t ng = 0;
    group_off_out[0] = 0;
    for (size_t i = 0; i < ntiles;)
    {
        size_t j = i + 1;
        while (j < ntiles && j - i < size_t(max_group) && key(ord[j], slot) == key(ord[i], slot))
            ++j;
        group_off_out[++ng] = uint32_t(j);
        i = j;
    }
    // longest groups first (ties in block order): the launch's last waves
    // are the short groups, so the SIMDs run out of work together
    std::vector<uint32_t> gi(ng);
    for (size_t g = 0; g < ng; ++g) gi[g] = uint32_t(g);
    std::stable_sort(gi.begin(), gi.end(), [&](uint32_t a, uint32_t b) {
        return group_off_out[a + 1] - group_off_out[a] > group_off_out[b + 1] - group_off_out[b];
    });
    std::vector<uint32_t> off2(ng + 1);
    size_t pos = 0;
    for (size_t g = 0; g < ng; ++g)
    {
        off2[g] = uint32_t(pos);
        for (uint32_t i = group_off_out[gi[g]]; i < group_off_out[gi[g] + 1]; ++i)
            order_out[pos++] = ord[i];
    }
    off2[ng] = uint32_t(pos);
    for (size_t g = 0; g <= ng; ++g) group_off_out[g] = off2[g];
    *ngroups_out = ng;
    return CPTC_OK;
}
