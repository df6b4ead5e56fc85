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

namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int WAVE = 64;
constexpr int WAVES_PER_WG = 4;

// MODE = target slot; HDR = int32 words per tile header (bi, bj, bk first):
// 4 for order-3 tiles, 6 for generic units.  HAS_W: the unit's FP64 outer
// weights W[t, r] scale its contribution (generic N-order units).
// GROUPED: a wave takes a group of tiles that share the target row block
// (order[goff[g] .. goff[g+1]]) and sums their (row, rank) results in its own
// LDS block (16 x Rp doubles; each lane owns its entries, so no barrier),
// then flushes one atomic per (row, rank) per group instead of per tile.
//
// The contraction takes the Khatri-Rao block as the MFMA B operand:
//   out[i, r] = sum_{j,k} T[i, j, k] * (B[b1 + j, r] * C[b2 + k, r])   (mode 0)
// i.e. one 16 x 256 x 16 product per 16-rank block, accumulated in FP32
// over the tile's 256 (j, k) pairs and added to the FP64 output once per
// (row, rank, tile) or group.  K-step (x, s) covers slice x and contracted
// rows 4s..4s+3: the A operand is the lane's tile cells and the B operand is
// bf[s] * wf[x] formed in FP32.  Two interleaved accumulator
// chains; the next item's factor values (and, modes 0 and 1, the next
// tile's cells) load while the current item's MFMAs run.
template <int MODE, int HDR, bool HAS_W, bool GROUPED>
__global__ __launch_bounds__(WAVE* WAVES_PER_WG) __attribute__((amdgpu_waves_per_eu(2, 2))) void dense_tiles_kernel(
    const int32_t* __restrict__ hdr, const float* __restrict__ tile_f32, size_t ntiles,
    const uint32_t* __restrict__ order, const uint32_t* __restrict__ goff, size_t ngroups,
    const double* __restrict__ A, const double* __restrict__ B, const double* __restrict__ C,
    const double* __restrict__ W, double* __restrict__ FtV, int R, int Rp, int dimI, int dimJ,
    int dimK, int S)
{
    extern __shared__ double gacc_lds[];
    // the wave index is uniform across the wave: say so, so that the tile
    // loop, header loads and row pointers live in scalar registers.  S waves
    // share one tile / group: wave slice s takes rank blocks s, s + S, ...
    // (consecutive waves of a workgroup, so the tile cells they all read
    // come from L1 / L2 after the first).
    const size_t wall = size_t(blockIdx.x) * WAVES_PER_WG +
                        size_t(__builtin_amdgcn_readfirstlane(int(threadIdx.x / WAVE)));
    const size_t wid = wall / size_t(S);
    const int rb0 = int(wall - wid * size_t(S)) * 16;
    const int rstep = S * 16;
    size_t it0, it1;
    if constexpr (GROUPED)
    {
        if (wid >= ngroups) return;
        it0 = goff[wid];
        it1 = goff[wid + 1];
    }
    else
    {
        if (wid >= ntiles) return;
        it0 = wid;
        it1 = wid + 1;
    }
    const int lane = threadIdx.x & (WAVE - 1);
    const int lo = lane & 15;
    const int hi = lane >> 4;
    double* gacc = gacc_lds + size_t(threadIdx.x / WAVE) * 16 * Rp;
    if constexpr (GROUPED)
        for (int rb = rb0; rb < R; rb += rstep)
#pragma unroll
            for (int v = 0; v < 4; ++v) gacc[(4 * hi + v) * Rp + rb + lo] = 0.0;

    const double* __restrict__ Ff = (MODE == 0) ? B : A;   // contracted factor
    const double* __restrict__ Fw = (MODE == 2) ? B : C;   // slice factor
    const int fdim = (MODE == 0) ? dimJ : dimI;
    const int wdim = (MODE == 2) ? dimJ : dimK;
    const int odim = (MODE == 0) ? dimI : (MODE == 1) ? dimJ : dimK;

    auto tile_of = [&](size_t it) -> size_t { return GROUPED ? size_t(order[it]) : it; };
    // lane offset of a contracted row (fb + 4q + hi) from the wave-uniform
    // row pointer Ff + (fb + 4q) R + rb
    const int boff = hi * R + lo;
    double bn[4], wn[16];
    // interior tiles load factor values by buffer loads: the row block's
    // byte offset in soffset (32-bit scalar arithmetic), the lane's offset
    // in voffset; needs every row offset of both factors below 2^31
    const bool buf = uint64_t(fdim) * uint64_t(R) * 8u < (uint64_t(1) << 31) &&
                     uint64_t(wdim) * uint64_t(R) * 8u < (uint64_t(1) << 31);
    const __amdgpu_buffer_rsrc_t rsf =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<double*>(Ff), short(0), 0x7FFFFFFF, 0x00020000);
    const __amdgpu_buffer_rsrc_t rsw =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<double*>(Fw), short(0), 0x7FFFFFF0, 0x00020000);
    const uint32_t vbo = uint32_t(boff) * 8u, vwo = uint32_t(lo) * 8u;
    const uint32_t rowb = uint32_t(R) * 8u;
    auto ld = [](const __amdgpu_buffer_rsrc_t& rs, uint32_t voff, uint32_t soff) {
        return __builtin_bit_cast(double, __builtin_amdgcn_raw_buffer_load_b64(rs, voff, soff, 0));
    };
    auto load_factors = [&](size_t t, int rb) {
        const int b0 = hdr[HDR * t] * 16, b1 = hdr[HDR * t + 1] * 16, b2 = hdr[HDR * t + 2] * 16;
        const int fb = (MODE == 0) ? b1 : b0;
        const int wb = (MODE == 2) ? b1 : b2;
        if (buf && fb + 16 <= fdim && wb + 16 <= wdim && rb + 16 <= R)
        {
            // interior tile, full rank block: unconditional loads
            const uint32_t so = (uint32_t(fb) * uint32_t(R) + uint32_t(rb)) * 8u;
            const uint32_t sw = (uint32_t(wb) * uint32_t(R) + uint32_t(rb)) * 8u;
#pragma unroll
            for (int q = 0; q < 4; ++q) bn[q] = ld(rsf, vbo, so + uint32_t(4 * q) * rowb);
#pragma unroll
            for (int x = 0; x < 16; ++x) wn[x] = ld(rsw, vwo, sw + uint32_t(x) * rowb);
        }
        else
        {
            const int r = rb + lo;
#pragma unroll
            for (int q = 0; q < 4; ++q)
                bn[q] = (r < R && fb + 4 * q + hi < fdim) ? Ff[size_t(fb + 4 * q + hi) * R + r]
                                                          : 0.0;
#pragma unroll
            for (int x = 0; x < 16; ++x)
                wn[x] = (r < R && wb + x < wdim) ? Fw[size_t(wb + x) * R + r] : 0.0;
        }
    };
    float cells[4][16], ncells[4][16];
    auto load_cells = [&](size_t t, float (&c)[4][16]) {
        const float* __restrict__ T = tile_f32 + t * 4096;
#pragma unroll
        for (int q = 0; q < 4; ++q)
        {
            if (MODE == 0 || MODE == 1)
            {
                const int i = (MODE == 0) ? lo : 4 * q + hi;
                const int j = (MODE == 0) ? 4 * q + hi : lo;
                const float4* pp = reinterpret_cast<const float4*>(T + (i * 16 + j) * 16);
#pragma unroll
                for (int u = 0; u < 4; ++u)
                {
                    const float4 v = pp[u];
                    c[q][4 * u + 0] = v.x;
                    c[q][4 * u + 1] = v.y;
                    c[q][4 * u + 2] = v.z;
                    c[q][4 * u + 3] = v.w;
                }
            }
            else
            {
#pragma unroll
                for (int x = 0; x < 16; ++x) c[q][x] = T[((4 * q + hi) * 16 + x) * 16 + lo];
            }
        }
    };

    size_t it = it0;
    int rb = rb0;
    size_t t = tile_of(it);
    load_cells(t, cells);
    load_factors(t, rb0);
    int ob = 0;
    while (true)
    {
        float bf[4], wf[16];
#pragma unroll
        for (int q = 0; q < 4; ++q) bf[q] = float(bn[q]);
#pragma unroll
        for (int x = 0; x < 16; ++x) wf[x] = float(wn[x]);
        ob = hdr[HDR * t + MODE] * 16;
        const int r = rb + lo;
        size_t itn = it;
        int rbn = rb + rstep;
        if (rbn >= R)
        {
            rbn = rb0;
            ++itn;
        }
        const bool more = itn < it1;
        const size_t tn = more ? tile_of(itn) : t;
        if (more) load_factors(tn, rbn);
        // next tile's cells in registers (modes 0 / 1: mode 2's strided cell
        // loads leave no room for a second set)
        constexpr bool PF = GROUPED && MODE != 2;
        const bool next_tile = PF && rb == rb0 && it + 1 < it1;
        if (next_tile) load_cells(tile_of(it + 1), ncells);

        floatx4 a0 = floatx4{0.0f, 0.0f, 0.0f, 0.0f}, a1 = a0;
#pragma unroll
        for (int x = 0; x < 16; x += 2)
        {
#pragma unroll
            for (int q = 0; q < 4; ++q)
            {
                a0 = __builtin_amdgcn_mfma_f32_16x16x4f32(cells[q][x], bf[q] * wf[x], a0, 0, 0,
                                                          0);
                a1 = __builtin_amdgcn_mfma_f32_16x16x4f32(cells[q][x + 1], bf[q] * wf[x + 1], a1,
                                                          0, 0, 0);
            }
        }
        if (r < R)
        {
            double tot[4];
#pragma unroll
            for (int v = 0; v < 4; ++v) tot[v] = double(a0[v]) + double(a1[v]);
            if constexpr (HAS_W)
            {
                const double wr = W[t * size_t(R) + r];
#pragma unroll
                for (int v = 0; v < 4; ++v) tot[v] *= wr;
            }
            if constexpr (GROUPED)
            {
#pragma unroll
                for (int v = 0; v < 4; ++v) gacc[(4 * hi + v) * Rp + r] += tot[v];
            }
            else
            {
#pragma unroll
                for (int v = 0; v < 4; ++v)
                {
                    const int row = ob + 4 * hi + v;
                    if (row < odim && tot[v] != 0.0) atomicAdd(FtV + size_t(row) * R + r, tot[v]);
                }
            }
        }
        if (!more) break;
        if (itn != it)
        {
            if constexpr (PF)
            {
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (int x = 0; x < 16; ++x) cells[q][x] = ncells[q][x];
            }
            else
            {
                load_cells(tn, cells);
            }
        }
        it = itn;
        rb = rbn;
        t = tn;
    }
    if constexpr (GROUPED)
    {
        for (int rb2 = rb0; rb2 < R; rb2 += rstep)
        {
            const int r = rb2 + lo;
            if (r >= R) continue;
#pragma unroll
            for (int v = 0; v < 4; ++v)
            {
                const int row = ob + 4 * hi + v;
                const double x = gacc[(4 * hi + v) * Rp + r];
                if (row < odim && x != 0.0) atomicAdd(FtV + size_t(row) * R + r, x);
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
    static int simds[64] = {};
    int dev = 0;
    if (hipStreamGetDevice(s, &dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    if (simds[dev] == 0)
    {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0)
            n = 256;
        simds[dev] = 4 * n;
    }
    const size_t want = size_t(simds[dev]);
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
    for (size_t t = 0; t < ntiles; ++t) order_out[t] = ord[t];
    *ngroups_out = ng;
    return CPTC_OK;
}
