// Dense 16^3 tile / unit MTTKRP on the bf16 matrix cores with a three-term
// split (gfx950 v_mfma_f32_32x32x16_bf16), the fast counterpart of
// dense_tiles_body (tiles_body.hpp): same sum, same grouping, same FP64
// output accumulation.
//
// Contraction.  For target slot t, contracted slot c and weight slot w
// (mode 0: t = i, c = j, w = k; mode 1: t = j, c = i, w = k; mode 2:
// t = k, c = i, w = j):
//   M[a, w, r] = sum_c T[a, c, w] * Fc[c, r]          (bf16 matrix cores)
//   out[a, r]  = sum_w M[a, w, r] * Fw[w, r]           (FP32 VALU)
// One 32 x 32 x 16 product per (w pair, 32-rank block): its 32 rows are
// (w half, a) = (m / 16, m % 16) and its K dimension the tile's 16
// contracted rows, so one instruction contracts two w slices (w = p and
// w = 8 + p for instruction p = 0..7) and the lane multiplies each of its 16
// results by its own rank's Fw value.
//
// Split.  x = hi + lo with hi = bf16(x) and lo = bf16(x - hi) (both round
// to nearest even), so |x - hi - lo| <= 2^-18 |x|; the product
// x * y ~ hi_x hi_y + hi_x lo_y + lo_x hi_y (the lo_x lo_y term, <= 2^-18 |xy|,
// is dropped), accumulated in FP32, smallest terms first.  The relative error
// per product is a few 2^-18 at most (~1e-5 worst case, ~1e-6 typical), below
// the reference's TF32 (2^-11) inputs.
//
// Operands.  The tile cells come from the FP32 tile image (hi taken from the
// value clamped to the bf16 range, so it never overflows) and are split once
// per tile; the contracted factor arrives pre-split and the weight factor in
// FP32 (cptc_tile_operands), in the lanes' order:
//   fs_hi / fs_lo [c / 8][Rq] = 8 bf16 (rows 8 (c / 8) .. + 7 of one rank)
//   fw [w / 16][Rq] = 16 floats (rows 16 (w / 16) .. + 15 of one rank)
// Rq = R rounded up to 32, rows padded to 16 with zeros.
//
// Lane layout of v_mfma_f32_32x32x16_bf16 (checked on gfx950):
//   A[m][k]: lane = m + 32 * (k / 8), element k % 8;
//   B[k][n]: lane = n + 32 * (k / 8), element k % 8;
//   D[m][n]: lane = n + 32 * ((m / 4) % 2), element 4 * (m / 8) + m % 4.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#ifndef CPTC_B3_PIPE
#define CPTC_B3_PIPE 4   // MFMA accumulators in flight per wave (2 or 4)
#endif

namespace cptc_k {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr float BF16_MAX = 3.38953139e38f;   // (2 - 2^-7) * 2^127

// hi / lo bf16 pair of two values, packed as (first, second) in one dword
// each.  hi is taken from c0 / c1 (the values, or the values clamped to the
// bf16 range), lo from the values minus hi.
__device__ __forceinline__ void split_bf16x2(float x0, float x1, uint32_t& hi, uint32_t& lo,
                                             float c0, float c1)
{
    const __bf16 h0 = static_cast<__bf16>(c0), h1 = static_cast<__bf16>(c1);
    const uint32_t b0 = __builtin_bit_cast(uint16_t, h0), b1 = __builtin_bit_cast(uint16_t, h1);
    const float f0 = __builtin_bit_cast(float, b0 << 16), f1 = __builtin_bit_cast(float, b1 << 16);
    const __bf16 l0 = static_cast<__bf16>(x0 - f0), l1 = static_cast<__bf16>(x1 - f1);
    hi = b0 | (b1 << 16);
    lo = uint32_t(__builtin_bit_cast(uint16_t, l0)) | (uint32_t(__builtin_bit_cast(uint16_t, l1)) << 16);
}

__device__ __forceinline__ void split_bf16x2(float x0, float x1, uint32_t& hi, uint32_t& lo)
{
    split_bf16x2(x0, x1, hi, lo, x0, x1);
}

// MODE = target slot; HDR = int32 words per tile header (block indices of
// slots 0, 1, 2 first); HAS_W: FP64 outer weights W[t, r] scale the tile's
// contribution (generic N-order units); GROUPED: a wave sums a group of
// tiles with one target block (order[goff[g] .. goff[g + 1]]) in its own LDS
// block (16 x Rq doubles, each lane owns its entries) and flushes one atomic
// per (row, rank) per group.  S waves share one tile / group, wave s taking
// the 32-rank blocks s, s + S, ...
//
// COMPACT: the A operand comes split from the target slot's compacted image
// instead of tile_f32 (compact_split_*_kernel in dense_tiles.hip): segment
// a * 64 + w * 4 + e = the bf16 hi then lo halves of cells (a, w,
// 4e .. 4e + 3) (target, weight, contracted), 16 bytes; cmask[64 t + x] =
// occupancy bits of the tile's segments 32x .. 32x + 31, cmask[64 t + 32 +
// x] = occupied segments before word x, the occupied segments in order at
// cseg[csegoff[t] ..].
template <int MODE, int HDR, bool HAS_W, bool GROUPED, bool COMPACT = false>
__device__ __forceinline__ void dense_tiles_b3_body(
    size_t wg, double* gacc_lds, const int32_t* __restrict__ hdr,
    const float* __restrict__ tile_f32, const uint32_t* __restrict__ cmask,
    const uint32_t* __restrict__ csegoff, const u32x4* __restrict__ cseg,
    size_t ntiles, const uint32_t* __restrict__ order,
    const uint32_t* __restrict__ goff, size_t ngroups, const u32x4* __restrict__ fs_hi,
    const u32x4* __restrict__ fs_lo, const float4* __restrict__ fw,
    const double* __restrict__ W, double* __restrict__ FtV, int R, int Rq, int odim, int S)
{
    constexpr int WAVES = 4;
    constexpr int CS = (MODE == 0) ? 1 : 0;   // contracted slot
    constexpr int WS = (MODE == 2) ? 1 : 2;   // weight slot
    const size_t wall = wg * WAVES + size_t(__builtin_amdgcn_readfirstlane(int(threadIdx.x / 64)));
    const size_t wid = wall / size_t(S);
    const int rb0 = int(wall - wid * size_t(S)) * 32;
    const int rstep = S * 32;
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
    const int lane = threadIdx.x & 63;
    const int n = lane & 31;   // rank within the block; B column, D column
    const int h = lane >> 5;   // K group (A, B); row quad parity (D)
    const int m = lane & 31;   // A row: (w half, target row)
    const int ww = m >> 4, am = m & 15;
    // the wave's LDS block: 16 rows x (its rank blocks x 32) doubles, rank
    // block rb at column (rb - rb0) / rstep * 32
    const int gstride = (Rq / 32 + S - 1) / S * 32;
    double* gacc = gacc_lds + size_t(threadIdx.x / 64) * 16 * size_t(gstride);
    auto gcol = [&](int rbx) { return (rbx - rb0) / rstep * 32 + n; };
    // the lane's 8 D rows: target row a(o) = 8 (o / 4) + 4 h + o % 4, o = 0..7
    auto arow = [&](int o) { return 8 * (o >> 2) + 4 * h + (o & 3); };
    if constexpr (GROUPED)
        for (int rb = rb0; rb < Rq; rb += rstep)
#pragma unroll
            for (int o = 0; o < 8; ++o) gacc[arow(o) * gstride + gcol(rb)] = 0.0;

    auto tile_of = [&](size_t it) -> size_t { return GROUPED ? size_t(order[it]) : it; };

    // the lane's 64 cells of the dense image: cells[q][p] = T at (target am,
    // contracted 8 h + q, weight 8 ww + p)
    float cells[8][8];
    // compacted image: buffer loads over the segments (byte offsets below
    // 2^32, checked by the launcher); an unoccupied segment's load takes an
    // offset past the buffer's end, which reads zeros
    const __amdgpu_buffer_rsrc_t rseg = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<u32x4*>(cseg), short(0), int(0xFFFFFFF0u), 0x00020000);
    constexpr uint32_t OOB = 0xFFFFFFF0u;
    // the header of the tile whose operand loads next: lane x holds word x
    // of its 64 (occupancy words 0..31, running counts 32..63), loaded with
    // one coalesced 256-byte load a tile ahead; the lanes fetch the words
    // they need from it by lane shuffles
    uint32_t hdr_w = 0, hdr_so = 0;
    auto load_hdr = [&](size_t tt) {
        if constexpr (COMPACT)
        {
            hdr_w = cmask[tt * 64 + size_t(lane)];
            hdr_so = csegoff[tt];
        }
    };
    bf16x8 ahi[8], alo[8];
    // The A operand of the compacted image in two steps, so that the loads
    // of the next tile are in flight while the current rank block computes:
    // issue_a loads the header's tile's 16 segments of the lane into araw
    // (raw 16-byte segments: hi halves then lo halves of 4 cells each),
    // assemble_a moves them into the operand registers.
    using raw4 = decltype(__builtin_amdgcn_raw_buffer_load_b128(rseg, 0u, 0, 0));
    raw4 araw[16];
    auto issue_a = [&]() {
        // the lane's 16 segments (w = 8 ww + p, cells 8h .. 8h + 7) are bits
        // 4 p + 2 h and 4 p + 2 h + 1 of mask word 2 am + ww
        // (shifted by 2 h once, so the per-p masks and bit positions are
        // constants rather than per-lane registers)
        const uint32_t mw = uint32_t(__shfl(int(hdr_w), 2 * am + ww));
        const uint32_t sh = 2u * uint32_t(h);
        const uint32_t mwh = mw >> sh;
        const uint32_t base = hdr_so + uint32_t(__shfl(int(hdr_w), 32 + 2 * am + ww)) +
                              uint32_t(__builtin_popcount(mw & ((1u << sh) - 1u)));
#pragma unroll
        for (int p = 0; p < 8; ++p)
        {
            const uint32_t i0 = base + uint32_t(__builtin_popcount(mwh & ((1u << (4 * p)) - 1u)));
            const uint32_t b0 = (mwh >> (4 * p)) & 1u, b1 = (mwh >> (4 * p + 1)) & 1u;
            const uint32_t o0 = b0 ? i0 * 16u : OOB;
            const uint32_t o1 = b1 ? (i0 + b0) * 16u : OOB;
            araw[2 * p] = __builtin_amdgcn_raw_buffer_load_b128(rseg, o0, 0, 0);
            araw[2 * p + 1] = __builtin_amdgcn_raw_buffer_load_b128(rseg, o1, 0, 0);
        }
    };
    auto assemble_a = [&]() {
#pragma unroll
        for (int p = 0; p < 8; ++p)
        {
            // (the load's vector indexed directly: a __builtin_bit_cast of it
            // to another 4 x 32-bit vector type compiled to a one-dword load)
            const raw4 v0 = araw[2 * p], v1 = araw[2 * p + 1];
            u32x4 hv, lv;
            hv[0] = uint32_t(v0[0]);
            hv[1] = uint32_t(v0[1]);
            hv[2] = uint32_t(v1[0]);
            hv[3] = uint32_t(v1[1]);
            lv[0] = uint32_t(v0[2]);
            lv[1] = uint32_t(v0[3]);
            lv[2] = uint32_t(v1[2]);
            lv[3] = uint32_t(v1[3]);
            ahi[p] = __builtin_bit_cast(bf16x8, hv);
            alo[p] = __builtin_bit_cast(bf16x8, lv);
        }
    };
    auto load_cells = [&](size_t t) {
        if constexpr (COMPACT)
        {
            issue_a();
            assemble_a();
            return;
        }
        const float* __restrict__ T = tile_f32 + t * 4096;
#pragma unroll
        for (int q = 0; q < 8; ++q)
        {
            const int c = 8 * h + q;
            if constexpr (MODE == 0 || MODE == 1)
            {
                // (i, j, k) = (am, c, w) or (c, am, w): the 8 w values are contiguous
                const int base = (MODE == 0) ? (am * 16 + c) * 16 : (c * 16 + am) * 16;
                const float4* pp = reinterpret_cast<const float4*>(T + base + 8 * ww);
                const float4 v0 = pp[0], v1 = pp[1];
                cells[q][0] = v0.x;
                cells[q][1] = v0.y;
                cells[q][2] = v0.z;
                cells[q][3] = v0.w;
                cells[q][4] = v1.x;
                cells[q][5] = v1.y;
                cells[q][6] = v1.z;
                cells[q][7] = v1.w;
            }
            else
            {
                // (i, j, k) = (c, w, am)
#pragma unroll
                for (int p = 0; p < 8; ++p) cells[q][p] = T[(c * 16 + 8 * ww + p) * 16 + am];
            }
        }
    };
    auto split_cells = [&]() {
        if constexpr (COMPACT) return;   // the image holds the split halves
#pragma unroll
        for (int p = 0; p < 8; ++p)
        {
            u32x4 hv, lv;
#pragma unroll
            for (int s = 0; s < 4; ++s)
            {
                // FP32 values beyond the bf16 range (the image clamps to
                // +-FLT_MAX) keep hi finite: hi = the range limit, lo = rest
                const float x0 = cells[2 * s][p], x1 = cells[2 * s + 1][p];
                uint32_t hh, ll;
                split_bf16x2(x0, x1, hh, ll, __builtin_amdgcn_fmed3f(x0, -BF16_MAX, BF16_MAX),
                             __builtin_amdgcn_fmed3f(x1, -BF16_MAX, BF16_MAX));
                hv[s] = hh;
                lv[s] = ll;
            }
            ahi[p] = __builtin_bit_cast(bf16x8, hv);
            alo[p] = __builtin_bit_cast(bf16x8, lv);
        }
    };

    u32x4 bh, bl;
    float4 cw4[4];
    // the item's FP64 outer weight (HAS_W), loaded by every lane at a
    // clamped rank (no path skips the load, so the waits can count it)
    double wop = 1.0;
    auto load_ops = [&](size_t t, int rb) {
        const int cb = hdr[HDR * t + CS];   // contracted block (16 rows)
        const int wb = hdr[HDR * t + WS];   // weight block
        const size_t bi = (size_t(2 * cb + h) * size_t(Rq)) + size_t(rb + n);
        bh = fs_hi[bi];
        bl = fs_lo[bi];
        const float4* pw = fw + (size_t(wb) * size_t(Rq) + size_t(rb + n)) * 4;
#pragma unroll
        for (int s = 0; s < 4; ++s) cw4[s] = pw[s];
        if constexpr (HAS_W) wop = W[t * size_t(R) + size_t(rb + n < R ? rb + n : R - 1)];
    };

    size_t it = it0;
    int rb = rb0;
    size_t t = tile_of(it);
    load_hdr(t);
    load_cells(t);
    split_cells();
    if (it + 1 < it1) load_hdr(tile_of(it + 1));
    load_ops(t, rb);
    int ob = 0;
    while (true)
    {
        float cw[16];
#pragma unroll
        for (int s = 0; s < 4; ++s)
        {
            cw[4 * s + 0] = cw4[s].x;
            cw[4 * s + 1] = cw4[s].y;
            cw[4 * s + 2] = cw4[s].z;
            cw[4 * s + 3] = cw4[s].w;
        }
        ob = hdr[HDR * t + MODE] * 16;
        const int r = rb + n;
        // (the operands below were loaded with the previous item's; the
        // next item's overwrite them before this item's epilogue)
        const double wr = (r < R) ? wop : 0.0;
        size_t itn = it;
        int rbn = rb + rstep;
        if (rbn >= Rq)
        {
            rbn = rb0;
            ++itn;
        }
        const bool more = itn < it1;
        const size_t tn = more ? tile_of(itn) : t;
        // modes 0 / 1 of the dense image: the next tile's cells load while
        // this rank block computes (the raw cell registers are free once the
        // current tile is split; mode 2's 64 scalar loads leave no room for
        // that); the compacted image's next A operand likewise (issue_a)
        const bool next_tile = more && itn != it;
        constexpr bool PF_CELLS = MODE != 2 && !COMPACT;
        if (PF_CELLS && next_tile) load_cells(tn);
        if constexpr (COMPACT)
        {
            // this rank block's B and weight operands are waited for here,
            // before the next tile's loads are issued: the wait for them
            // below would otherwise count those loads too (the two paths
            // into the products merge with different loads in flight, and
            // the merged wait is the stricter one)
            asm volatile("" ::"v"(bh), "v"(bl), "v"(wop));
#pragma unroll
            for (int s = 0; s < 4; ++s)
                asm volatile("" ::"v"(cw4[s].x), "v"(cw4[s].y), "v"(cw4[s].z), "v"(cw4[s].w));
        }
        // the next tile's A operand loads during this rank block (its
        // address arithmetic placed after the first products are issued, so
        // it runs while the matrix cores work); the header after it loads
        // once its words have been read
        auto prefetch_a = [&]() {
            if constexpr (COMPACT)
                if (next_tile)
                {
                    issue_a();
                    if (itn + 1 < it1) load_hdr(tile_of(itn + 1));
                }
        };

        // Software pipeline over the four w pairs: the products of pair
        // pp + 1 are issued before the FMAs of pair pp consume theirs, so
        // the matrix cores and the VALU overlap within the wave, and at most
        // 4 accumulators (64 registers) are live, not 8.
        float out[8];
#pragma unroll
        for (int o = 0; o < 8; ++o) out[o] = 0.0f;
        auto products = [&](int p, floatx16& a0, floatx16& a1) {
            const bf16x8 bhi = __builtin_bit_cast(bf16x8, bh), blo = __builtin_bit_cast(bf16x8, bl);
            const floatx16 z = {};
            a0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(alo[p], bhi, z, 0, 0, 0);
            a1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(alo[p + 1], bhi, z, 0, 0, 0);
            a0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ahi[p], blo, a0, 0, 0, 0);
            a1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ahi[p + 1], blo, a1, 0, 0, 0);
            a0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ahi[p], bhi, a0, 0, 0, 0);
            a1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ahi[p + 1], bhi, a1, 0, 0, 0);
        };
        auto weigh = [&](int p, const floatx16& a0, const floatx16& a1) {
#pragma unroll
            for (int o = 0; o < 8; ++o)
            {
                // element o: w = p (first w half); element 8 + o: w = 8 + p
                out[o] = __builtin_fmaf(a0[o], cw[p], out[o]);
                out[o] = __builtin_fmaf(a0[o + 8], cw[8 + p], out[o]);
                out[o] = __builtin_fmaf(a1[o], cw[p + 1], out[o]);
                out[o] = __builtin_fmaf(a1[o + 8], cw[9 + p], out[o]);
            }
        };
        // ordering fence (no instructions): the FMAs issued so far complete
        // their `out` values here, and the products after it read a B
        // operand "redefined" here, so neither moves across
        auto fence = [&]() {
#pragma unroll
            for (int o = 0; o < 8; ++o) asm volatile("" : "+v"(out[o]));
            asm volatile("" : "+v"(bh), "+v"(bl));
        };
#if CPTC_B3_PIPE == 2
        floatx16 x0, x1;
        products(0, x0, x1);
        prefetch_a();
        weigh(0, x0, x1);
        fence();
        products(2, x0, x1);
        weigh(2, x0, x1);
        fence();
        products(4, x0, x1);
        weigh(4, x0, x1);
        fence();
        products(6, x0, x1);
        weigh(6, x0, x1);
#else
        floatx16 x0, x1, y0, y1;
        products(0, x0, x1);
        products(2, y0, y1);
        prefetch_a();
        weigh(0, x0, x1);
        fence();
        products(4, x0, x1);
        weigh(2, y0, y1);
        fence();
        products(6, y0, y1);
        weigh(4, x0, x1);
        fence();
        weigh(6, y0, y1);
#endif
        // unconditional (the last item reloads its own operands), so the
        // loads land in the registers the next rank block reads instead of
        // being copied there, with a wait, at the end of the iteration
        load_ops(tn, more ? rbn : rb);
        // unconditional epilogue (ranks >= R hold zeros and are not flushed),
        // so the FMAs above are not sunk into a branch
#pragma unroll
        for (int o = 0; o < 8; ++o)
        {
            double tot = double(out[o]);
            if constexpr (HAS_W) tot *= wr;
            if constexpr (GROUPED)
            {
                // LDS atomic add without return (ds_add_f64): the eight
                // updates do not wait on each other as read-add-write chains
                // through one register pair do (each entry has one owner
                // lane, whose LDS operations stay in order, so the sum is
                // the plain one).  Config 3: 0.37-0.38 -> 0.356-0.367 ms per
                // launch; config 5 units 0.080-0.091 -> 0.079-0.089 ms.
                __hip_atomic_fetch_add(&gacc[arow(o) * gstride + gcol(rb)], tot, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_WORKGROUP);
            }
            else
            {
                const int row = ob + arow(o);
                if (r < R && row < odim && tot != 0.0) atomicAdd(FtV + size_t(row) * R + r, tot);
            }
        }
        if (!more) break;
        if (next_tile)
        {
            if constexpr (COMPACT)
                assemble_a();
            else
            {
                if (!PF_CELLS) load_cells(tn);
                split_cells();
                if (itn + 1 < it1) load_hdr(tile_of(itn + 1));
            }
        }
        it = itn;
        rb = rbn;
        t = tn;
    }
    if constexpr (GROUPED)
    {
        for (int rb2 = rb0; rb2 < Rq; rb2 += rstep)
        {
            const int r = rb2 + n;
            if (r >= R) continue;
#pragma unroll
            for (int o = 0; o < 8; ++o)
            {
                const int row = ob + arow(o);
                const double x = gacc[arow(o) * gstride + gcol(rb2)];
                if (row < odim && x != 0.0) atomicAdd(FtV + size_t(row) * R + r, x);
            }
        }
    }
}

}  // namespace cptc_k
