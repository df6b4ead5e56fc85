// Merged single-grid order-3 MTTKRP: the MFMA dense tiles and the FP64
// residual segments of one mode in ONE launch, the gfx950 counterpart of
// mttkrp_merged_kernel / compute_mttkrp_merged_async (dense.cu:1914-2058,
// 2258-2511; selected by ALS_FUSED, als.cu:28, 529-555).
//
// Roles.  Workgroup b of the grid is a tile workgroup when b % every == 0
// and b / every < D (D = tile workgroups of 4 waves, one tile group or tile
// per wave), otherwise the sparse workgroup of segment
// s = b - min(D, b / every + 1) (the number of tile workgroups at positions
// <= b), idle when s >= the segment count.  Grid = D + segments and
// every = max(1, grid / D), so the last tile position every * (D - 1) is
// inside the grid, every other position is one segment, and the two kinds
// of work interleave evenly over the dispatch order.  Both roles only add
// into FtV with FP64 atomics (the caller zeroes it), so the result is the
// two-launch one up to the order of those additions.
//
// The tile role is dense_tiles_body (tiles_body.hpp) and the segment role
// seg3_body (seg3_body.hpp), the bodies of the two separate kernels; the
// register allocation is the larger of the two (the tile role's), so the
// segment role runs at the tile kernel's occupancy.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "../host/hip_util.hpp"
#include "seg3_body.hpp"
#include "tiles_body.hpp"

namespace {

constexpr int WAVES = 4;
constexpr int SEG_UNROLL = 8;

template <int MODE, int RT, bool GROUPED>
__global__ __launch_bounds__(64 * WAVES) void mttkrp3_merged_kernel(
    const int32_t* __restrict__ hdr, const float* __restrict__ tile_f32, size_t ntiles,
    const uint32_t* __restrict__ order, const uint32_t* __restrict__ goff, size_t ngroups,
    uint32_t dense_wgs, const uint64_t* __restrict__ coords, const double* __restrict__ vals,
    const uint32_t* __restrict__ blk_row, const uint32_t* __restrict__ blk_start,
    const uint32_t* __restrict__ blk_cnt, uint32_t nseg, uint32_t every,
    const double* __restrict__ A, const double* __restrict__ B, const double* __restrict__ C,
    double* __restrict__ FtV, int R, int Rp, int dimI, int dimJ, int dimK)
{
    extern __shared__ double gacc_lds[];
    const uint32_t b = blockIdx.x;
    const uint32_t d = b / every;
    if (b - d * every == 0 && d < dense_wgs)
    {
        cptc_k::dense_tiles_body<MODE, 4, false, GROUPED>(d, gacc_lds, hdr, tile_f32, ntiles,
                                                          order, goff, ngroups, A, B, C, nullptr,
                                                          FtV, R, Rp, dimI, dimJ, dimK, 1);
        return;
    }
    const uint32_t before = d + 1 < dense_wgs ? d + 1 : dense_wgs;
    const uint32_t s = b - before;
    if (s >= nseg) return;
    const double* F1 = (MODE == 0) ? B : A;
    const double* F2 = (MODE == 2) ? B : C;
    cptc_k::seg3_body<RT, 2, WAVES, SEG_UNROLL>(s, 0, MODE, coords, vals, blk_row, blk_start,
                                                blk_cnt, F1, F2, FtV, R);
}

template <int MODE, int RT, bool GROUPED>
void launch(dim3 grid, size_t lds, hipStream_t st, const int32_t* hdr, const float* tiles,
            size_t ntiles, const uint32_t* order, const uint32_t* goff, size_t ngroups,
            uint32_t dwg, const uint64_t* coords, const double* vals, const uint32_t* br,
            const uint32_t* bs, const uint32_t* bc, uint32_t nseg, uint32_t every, const double* A,
            const double* B, const double* C, double* FtV, int R, int Rp, int dI, int dJ, int dK)
{
    hipLaunchKernelGGL((mttkrp3_merged_kernel<MODE, RT, GROUPED>), grid, dim3(64 * WAVES), lds, st,
                       hdr, tiles, ntiles, order, goff, ngroups, dwg, coords, vals, br, bs, bc,
                       nseg, every, A, B, C, FtV, R, Rp, dI, dJ, dK);
}

template <int MODE, int RT>
void launch_g(bool grouped, dim3 grid, size_t lds, hipStream_t st, const int32_t* hdr,
              const float* tiles, size_t ntiles, const uint32_t* order, const uint32_t* goff,
              size_t ngroups, uint32_t dwg, const uint64_t* coords, const double* vals,
              const uint32_t* br, const uint32_t* bs, const uint32_t* bc, uint32_t nseg,
              uint32_t every, const double* A, const double* B, const double* C, double* FtV,
              int R, int Rp, int dI, int dJ, int dK)
{
    if (grouped)
        launch<MODE, RT, true>(grid, lds, st, hdr, tiles, ntiles, order, goff, ngroups, dwg,
                               coords, vals, br, bs, bc, nseg, every, A, B, C, FtV, R, Rp, dI, dJ,
                               dK);
    else
        launch<MODE, RT, false>(grid, lds, st, hdr, tiles, ntiles, order, goff, ngroups, dwg,
                                coords, vals, br, bs, bc, nseg, every, A, B, C, FtV, R, Rp, dI,
                                dJ, dK);
}

template <int RT>
void launch_m(int mode, bool grouped, dim3 grid, size_t lds, hipStream_t st, const int32_t* hdr,
              const float* tiles, size_t ntiles, const uint32_t* order, const uint32_t* goff,
              size_t ngroups, uint32_t dwg, const uint64_t* coords, const double* vals,
              const uint32_t* br, const uint32_t* bs, const uint32_t* bc, uint32_t nseg,
              uint32_t every, const double* A, const double* B, const double* C, double* FtV,
              int R, int Rp, int dI, int dJ, int dK)
{
    if (mode == 0)
        launch_g<0, RT>(grouped, grid, lds, st, hdr, tiles, ntiles, order, goff, ngroups, dwg,
                        coords, vals, br, bs, bc, nseg, every, A, B, C, FtV, R, Rp, dI, dJ, dK);
    else if (mode == 1)
        launch_g<1, RT>(grouped, grid, lds, st, hdr, tiles, ntiles, order, goff, ngroups, dwg,
                        coords, vals, br, bs, bc, nseg, every, A, B, C, FtV, R, Rp, dI, dJ, dK);
    else
        launch_g<2, RT>(grouped, grid, lds, st, hdr, tiles, ntiles, order, goff, ngroups, dwg,
                        coords, vals, br, bs, bc, nseg, every, A, B, C, FtV, R, Rp, dI, dJ, dK);
}

}  // namespace

// dense_every > 0 fixes the interleave (every dense_every-th workgroup a
// tile workgroup, ALS_MERGED_STRIDE, dense.cu:2350-2381); flags bit 0 drops
// the tile role (ALS_MERGED_NO_DENSE), bit 1 the segment role
// (ALS_MERGED_NO_SPARSE) (dense.cu:2277-2283, 2326-2336).
extern "C" int cptc_mttkrp_merged3_ex(int mode, const int32_t* d_tiles, const float* d_tile_f32,
                                      size_t ntiles, const uint32_t* d_order,
                                      const uint32_t* d_group_off, size_t ngroups,
                                      const uint64_t* d_coords, const double* d_vals,
                                      const uint32_t* d_blk_row, const uint32_t* d_blk_start,
                                      const uint32_t* d_blk_cnt, size_t nblocks, const double* d_A,
                                      const double* d_B, const double* d_C, double* d_FtV, int R,
                                      int dimI, int dimJ, int dimK, int dense_every, int flags,
                                      void* stream)
{
    CPTC_REQUIRE(mode >= 0 && mode < 3 && R >= 1, CPTC_ERR_ARG,
                 "cptc_mttkrp_merged3: mode %d R %d", mode, R);
    CPTC_REQUIRE(R <= 128 && R % 2 == 0, CPTC_ERR_UNSUPPORTED,
                 "cptc_mttkrp_merged3: R %d (even R <= 128 only)", R);
    CPTC_REQUIRE((flags & ~3) == 0, CPTC_ERR_ARG, "cptc_mttkrp_merged3: flags %d", flags);
    if (flags & 1) ntiles = 0;
    if (flags & 2) nblocks = 0;
    if (ntiles == 0 && nblocks == 0) return CPTC_OK;
    CPTC_REQUIRE(d_A && d_B && d_C && d_FtV, CPTC_ERR_ARG, "cptc_mttkrp_merged3: null factor");
    CPTC_REQUIRE(ntiles == 0 || (d_tiles && d_tile_f32), CPTC_ERR_ARG,
                 "cptc_mttkrp_merged3: null tiles");
    CPTC_REQUIRE(nblocks == 0 || (d_coords && d_vals && d_blk_row && d_blk_start && d_blk_cnt),
                 CPTC_ERR_ARG, "cptc_mttkrp_merged3: null view");
    for (const double* p : {d_A, d_B, d_C})
        CPTC_REQUIRE((reinterpret_cast<uintptr_t>(p) & 15) == 0, CPTC_ERR_UNSUPPORTED,
                     "cptc_mttkrp_merged3: factors must be 16-byte aligned");
    const bool grouped = ntiles > 0 && d_order && d_group_off && ngroups > 0;
    const size_t items = ntiles == 0 ? 0 : (grouped ? ngroups : ntiles);
    const size_t dwg = (items + WAVES - 1) / WAVES;
    // the automatic interleave spreads the D tile workgroups evenly over the
    // grid of D + segments; a fixed stride k places tile workgroup d at
    // position d k, so the grid must reach k (D - 1) (every other position
    // before the end is a segment, later ones too: D + segments suffices)
    size_t grid = dwg + nblocks;
    uint32_t every;
    if (dwg == 0)
        every = uint32_t(std::min<size_t>(grid + 1, 0xFFFFFFFFu));
    else if (dense_every > 0 && nblocks > 0)
    {
        every = uint32_t(dense_every);
        grid = std::max(grid, size_t(every) * (dwg - 1) + 1);
    }
    else
        every = uint32_t(std::max<size_t>(1, grid / dwg));
    CPTC_REQUIRE(grid < (size_t(1) << 31), CPTC_ERR_ARG, "cptc_mttkrp_merged3: grid too large");
    const int Rp = (R + 15) / 16 * 16;
    const size_t lds = grouped ? size_t(WAVES) * 16 * Rp * sizeof(double) : 0;
    hipStream_t st = cptc::as_stream(stream);
    const dim3 g{unsigned(grid)};
    if (lds > 48 * 1024)
    {
        // the grouped tile role's accumulators (64 KB at R = 128)
        static cptc::DeviceOnce attr;
        CPTC_HIP(attr.lds_limit(
            {reinterpret_cast<const void*>(mttkrp3_merged_kernel<0, 128, true>),
             reinterpret_cast<const void*>(mttkrp3_merged_kernel<1, 128, true>),
             reinterpret_cast<const void*>(mttkrp3_merged_kernel<2, 128, true>)},
            64 * 1024));
    }
    const int dI = dimI, dJ = dimJ, dK = dimK;
#define CPTC_MERGED_ARGS                                                                       \
    mode, grouped, g, lds, st, d_tiles, d_tile_f32, ntiles, d_order, d_group_off, ngroups,     \
        uint32_t(dwg), d_coords, d_vals, d_blk_row, d_blk_start, d_blk_cnt, uint32_t(nblocks), \
        every, d_A, d_B, d_C, d_FtV, R, Rp, dI, dJ, dK
    if (R <= 8)
        launch_m<8>(CPTC_MERGED_ARGS);
    else if (R <= 16)
        launch_m<16>(CPTC_MERGED_ARGS);
    else if (R <= 32)
        launch_m<32>(CPTC_MERGED_ARGS);
    else if (R <= 64)
        launch_m<64>(CPTC_MERGED_ARGS);
    else
        launch_m<128>(CPTC_MERGED_ARGS);
#undef CPTC_MERGED_ARGS
    CPTC_LAUNCHED();
    return CPTC_OK;
}

extern "C" int cptc_mttkrp_merged3(int mode, const int32_t* d_tiles, const float* d_tile_f32,
                                   size_t ntiles, const uint32_t* d_order,
                                   const uint32_t* d_group_off, size_t ngroups,
                                   const uint64_t* d_coords, const double* d_vals,
                                   const uint32_t* d_blk_row, const uint32_t* d_blk_start,
                                   const uint32_t* d_blk_cnt, size_t nblocks, const double* d_A,
                                   const double* d_B, const double* d_C, double* d_FtV, int R,
                                   int dimI, int dimJ, int dimK, void* stream)
{
    return cptc_mttkrp_merged3_ex(mode, d_tiles, d_tile_f32, ntiles, d_order, d_group_off,
                                  ngroups, d_coords, d_vals, d_blk_row, d_blk_start, d_blk_cnt,
                                  nblocks, d_A, d_B, d_C, d_FtV, R, dimI, dimJ, dimK, 0, 0, stream);
}
