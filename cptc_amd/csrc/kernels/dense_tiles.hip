// Dense 16^3 tiles on CDNA4 FP32 MFMA with an FP64 epilogue — the gfx950
// counterpart of dense_tile_mttkrp_wmma (dense.cu:89-1077) for order-3 tiles
// and of g_dense_tile_mttkrp_kernel (generic.cu:429-561) for the generic
// path's dense units, whose contribution is also scaled by the unit's FP64
// outer-mode weights.  gfx950 has no xf32, so the inner products run in FP32,
// which is more accurate than the reference's TF32.
//
// For target mode 0 and one 16-rank block rb:
//   out_k[i, r] = sum_j T[i, j, k] * B[b1 + j, rb + r]        (FP32 MFMA)
//   acc[i, r]  += out_k[i, r] * C[b2 + k, rb + r]              (FP64)
//   FtV[b0 + i, rb + r] += acc[i, r]                          (one atomic)
// Mode 1 contracts i against A and weights by C[b2 + k]; mode 2 contracts i
// against A per j-slice and weights by B[b1 + j] (dense.cu:~560-1060).
//
// One wave64 owns one tile.  v_mfma_f32_16x16x4f32 lane layout (CDNA3/4):
//   A[m][kk]: lane = m + 16*kk;  B[kk][n]: lane = n + 16*kk;
//   D[m][n]:  lane = n + 16*(m/4), element m%4.
// The lane's 64 tile cells for all four K-steps and 16 slices are held in
// registers (the tile is read from HBM once per launch).
#include <hip/hip_runtime.h>

#include <cfloat>

#include "../host/hip_util.hpp"

namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int WAVE = 64;
constexpr int WAVES_PER_WG = 4;

__device__ inline float fold(const double* __restrict__ F, int row, int dim, int r, int R)
{
    return (row < dim && r < R) ? float(F[size_t(row) * R + r]) : 0.0f;
}

// MODE = target slot; HDR = int32 words per tile header (bi, bj, bk first):
// 4 for order-3 tiles, 6 for generic units.  HAS_W: the unit's FP64 outer
// weights W[t, r] scale its contribution (generic N-order units).
template <int MODE, int HDR, bool HAS_W>
__global__ __launch_bounds__(WAVE* WAVES_PER_WG) __attribute__((amdgpu_waves_per_eu(2, 2))) void dense_tiles_kernel(
    const int32_t* __restrict__ hdr, const float* __restrict__ tile_f32, size_t ntiles,
    const double* __restrict__ A, const double* __restrict__ B, const double* __restrict__ C,
    const double* __restrict__ W, double* __restrict__ FtV, int R, int dimI, int dimJ, int dimK)
{
    const size_t t = size_t(blockIdx.x) * WAVES_PER_WG + threadIdx.x / WAVE;
    if (t >= ntiles) return;
    const int lane = threadIdx.x & (WAVE - 1);
    const int lo = lane & 15;   // m (A operand row) / n (B, D column)
    const int hi = lane >> 4;   // kk (A, B) / m-group (D)
    const int b0 = hdr[HDR * t] * 16, b1 = hdr[HDR * t + 1] * 16, b2 = hdr[HDR * t + 2] * 16;
    const float* __restrict__ T = tile_f32 + t * 4096;

    // cells[s][x]: A operand of K-step s for slice x
    //   mode 0: T[lo][4s+hi][x]    mode 1: T[4s+hi][lo][x]    mode 2: T[4s+hi][x][lo]
    float cells[4][16];
#pragma unroll
    for (int s = 0; s < 4; ++s)
    {
        if (MODE == 0 || MODE == 1)
        {
            const int i = (MODE == 0) ? lo : 4 * s + hi;
            const int j = (MODE == 0) ? 4 * s + hi : lo;
            const float4* p = reinterpret_cast<const float4*>(T + (i * 16 + j) * 16);
#pragma unroll
            for (int q = 0; q < 4; ++q)
            {
                const float4 v = p[q];
                cells[s][4 * q + 0] = v.x;
                cells[s][4 * q + 1] = v.y;
                cells[s][4 * q + 2] = v.z;
                cells[s][4 * q + 3] = v.w;
            }
        }
        else
        {
#pragma unroll
            for (int x = 0; x < 16; ++x) cells[s][x] = T[((4 * s + hi) * 16 + x) * 16 + lo];
        }
    }

    // the contracted factor (B for mode 0, A otherwise) and its tile origin
    const double* __restrict__ Ff = (MODE == 0) ? B : A;
    const int fb = (MODE == 0) ? b1 : b0;
    const int fdim = (MODE == 0) ? dimJ : dimI;
    // the slice-weight factor (C for modes 0/1, B for mode 2)
    const double* __restrict__ Fw = (MODE == 2) ? B : C;
    const int wb = (MODE == 2) ? b1 : b2;
    const int wdim = (MODE == 2) ? dimJ : dimK;
    // output rows
    const int ob = (MODE == 0) ? b0 : (MODE == 1) ? b1 : b2;
    const int odim = (MODE == 0) ? dimI : (MODE == 1) ? dimJ : dimK;

    for (int rb = 0; rb < R; rb += 16)
    {
        const int r = rb + lo;
        float bf[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) bf[s] = fold(Ff, fb + 4 * s + hi, fdim, r, R);
        // four groups of four slices: inside a group the four 4-deep MFMA
        // chains are interleaved (s outer, slice inner); a scheduling
        // barrier between groups keeps only one group's accumulators live.
        // A slice beyond the mode holds no cells and gets weight 0.
        double tot[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
        for (int xg = 0; xg < 16; xg += 4)
        {
            double w[4];
#pragma unroll
            for (int xx = 0; xx < 4; ++xx)
                w[xx] = (r < R && wb + xg + xx < wdim) ? Fw[size_t(wb + xg + xx) * R + r] : 0.0;
            floatx4 d[4];
#pragma unroll
            for (int xx = 0; xx < 4; ++xx) d[xx] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int xx = 0; xx < 4; ++xx)
                    d[xx] = __builtin_amdgcn_mfma_f32_16x16x4f32(cells[s][xg + xx], bf[s], d[xx],
                                                                 0, 0, 0);
#pragma unroll
            for (int xx = 0; xx < 4; ++xx)
            {
                tot[0] += double(d[xx][0]) * w[xx];
                tot[1] += double(d[xx][1]) * w[xx];
                tot[2] += double(d[xx][2]) * w[xx];
                tot[3] += double(d[xx][3]) * w[xx];
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if (r < R)
        {
            if constexpr (HAS_W)
            {
                const double wr = W[t * size_t(R) + r];
#pragma unroll
                for (int v = 0; v < 4; ++v) tot[v] *= wr;
            }
#pragma unroll
            for (int v = 0; v < 4; ++v)
            {
                const int row = ob + 4 * hi + v;
                if (row < odim && tot[v] != 0.0) atomicAdd(FtV + size_t(row) * R + r, tot[v]);
            }
        }
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

extern "C" int cptc_mttkrp_dense_tiles3(int mode, const int32_t* d_tiles, const float* d_tile_f32,
                                        size_t ntiles, const double* d_A, const double* d_B,
                                        const double* d_C, double* d_FtV, int R, int dimI,
                                        int dimJ, int dimK, void* stream)
{
    CPTC_REQUIRE(mode >= 0 && mode < 3 && R >= 1, CPTC_ERR_ARG,
                 "cptc_mttkrp_dense_tiles3: mode %d R %d", mode, R);
    if (ntiles == 0) return CPTC_OK;
    CPTC_REQUIRE(d_tiles && d_tile_f32 && d_A && d_B && d_C && d_FtV, CPTC_ERR_ARG,
                 "cptc_mttkrp_dense_tiles3: null pointer");
    const size_t wgs = (ntiles + WAVES_PER_WG - 1) / WAVES_PER_WG;
    CPTC_REQUIRE(wgs < (size_t(1) << 31), CPTC_ERR_ARG, "cptc_mttkrp_dense_tiles3: too many tiles");
    hipStream_t s = cptc::as_stream(stream);
    const dim3 grid{static_cast<unsigned>(wgs)};
    const dim3 block{WAVE * WAVES_PER_WG};
    const double* noW = nullptr;
    if (mode == 0)
        hipLaunchKernelGGL((dense_tiles_kernel<0, 4, false>), grid, block, 0, s, d_tiles,
                           d_tile_f32, ntiles, d_A, d_B, d_C, noW, d_FtV, R, dimI, dimJ, dimK);
    else if (mode == 1)
        hipLaunchKernelGGL((dense_tiles_kernel<1, 4, false>), grid, block, 0, s, d_tiles,
                           d_tile_f32, ntiles, d_A, d_B, d_C, noW, d_FtV, R, dimI, dimJ, dimK);
    else
        hipLaunchKernelGGL((dense_tiles_kernel<2, 4, false>), grid, block, 0, s, d_tiles,
                           d_tile_f32, ntiles, d_A, d_B, d_C, noW, d_FtV, R, dimI, dimJ, dimK);
    CPTC_LAUNCHED();
    return CPTC_OK;
}

extern "C" int cptc_mttkrp_units_nd(int slot, const uint32_t* d_unit6, uint64_t nunits,
                                    const float* d_tiles, const double* d_W, const double* d_F0,
                                    const double* d_F1, const double* d_F2, int dim0, int dim1,
                                    int dim2, double* d_FtV, int R, void* stream)
{
    CPTC_REQUIRE(slot >= 0 && slot < 3 && R >= 1, CPTC_ERR_ARG,
                 "cptc_mttkrp_units_nd: slot %d R %d", slot, R);
    if (nunits == 0) return CPTC_OK;
    CPTC_REQUIRE(d_unit6 && d_tiles && d_W && d_F0 && d_F1 && d_F2 && d_FtV, CPTC_ERR_ARG,
                 "cptc_mttkrp_units_nd: null pointer");
    const size_t wgs = (nunits + WAVES_PER_WG - 1) / WAVES_PER_WG;
    CPTC_REQUIRE(wgs < (size_t(1) << 31), CPTC_ERR_ARG, "cptc_mttkrp_units_nd: too many units");
    hipStream_t s = cptc::as_stream(stream);
    const dim3 grid{static_cast<unsigned>(wgs)};
    const dim3 block{WAVE * WAVES_PER_WG};
    const int32_t* h = reinterpret_cast<const int32_t*>(d_unit6);
    if (slot == 0)
        hipLaunchKernelGGL((dense_tiles_kernel<0, 6, true>), grid, block, 0, s, h, d_tiles,
                           size_t(nunits), d_F0, d_F1, d_F2, d_W, d_FtV, R, dim0, dim1, dim2);
    else if (slot == 1)
        hipLaunchKernelGGL((dense_tiles_kernel<1, 6, true>), grid, block, 0, s, h, d_tiles,
                           size_t(nunits), d_F0, d_F1, d_F2, d_W, d_FtV, R, dim0, dim1, dim2);
    else
        hipLaunchKernelGGL((dense_tiles_kernel<2, 6, true>), grid, block, 0, s, h, d_tiles,
                           size_t(nunits), d_F0, d_F1, d_F2, d_W, d_FtV, R, dim0, dim1, dim2);
    CPTC_LAUNCHED();
    return CPTC_OK;
}
