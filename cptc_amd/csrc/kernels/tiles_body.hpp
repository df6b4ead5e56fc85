// Body of the dense 16^3 tile / unit MFMA kernel, shared by the tile kernel
// (kernels/dense_tiles.hip) and the merged single-grid MTTKRP
// (kernels/merged3.hip).  `wg` is the workgroup's index among the tile
// workgroups; gacc_lds is the dynamic LDS of the grouped variant (4 waves x
// 16 rows x Rp ranks of doubles).
//
// v_mfma_f32_16x16x4f32 lane layout (CDNA3/4):
//   A[m][kk]: lane = m + 16*kk;  B[kk][n]: lane = n + 16*kk;
//   D[m][n]:  lane = n + 16*(m/4), element m%4.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace cptc_k {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int TILE_WAVE = 64;
constexpr int TILE_WAVES_PER_WG = 4;

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
__device__ __forceinline__ void dense_tiles_body(
    size_t wg, double* gacc_lds, const int32_t* __restrict__ hdr,
    const float* __restrict__ tile_f32, size_t ntiles, const uint32_t* __restrict__ order,
    const uint32_t* __restrict__ goff, size_t ngroups, const double* __restrict__ A,
    const double* __restrict__ B, const double* __restrict__ C, const double* __restrict__ W,
    double* __restrict__ FtV, int R, int Rp, int dimI, int dimJ, int dimK, int S)
{
    // the wave index is uniform across the wave: say so, so that the tile
    // loop, header loads and row pointers live in scalar registers.  S waves
    // share one tile / group: wave slice s takes rank blocks s, s + S, ...
    // (consecutive waves of a workgroup, so the tile cells they all read
    // come from L1 / L2 after the first).
    const size_t wall = wg * TILE_WAVES_PER_WG +
                        size_t(__builtin_amdgcn_readfirstlane(int(threadIdx.x / TILE_WAVE)));
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
    const int lane = threadIdx.x & (TILE_WAVE - 1);
    const int lo = lane & 15;
    const int hi = lane >> 4;
    double* gacc = gacc_lds + size_t(threadIdx.x / TILE_WAVE) * 16 * Rp;
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
                // LDS atomic adds without return (ds_add_f64), not
                // read-add-write chains; one owner lane per entry
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    __hip_atomic_fetch_add(&gacc[(4 * hi + v) * Rp + r], tot[v], __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_WORKGROUP);
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


}  // namespace cptc_k
