// Body of the order-3 FP64 row-segment MTTKRP (sparse.cu:614-711 semantics),
// shared by mttkrp3_seg_kernel (kernels/mttkrp_sparse.hip) and the merged
// single-grid MTTKRP (kernels/merged3.hip).  `seg` is the segment, `rblk`
// the RT-wide rank block.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace cptc_k {

constexpr int SEG_WAVE = 64;

template <int VEC>
struct Row;
template <>
struct Row<2>
{
    double x[2];
    __device__ void load(const double* __restrict__ p)
    {
        const double2 v = *reinterpret_cast<const double2*>(p);
        x[0] = v.x;
        x[1] = v.y;
    }
};
template <>
struct Row<1>
{
    double x[1];
    __device__ void load(const double* __restrict__ p) { x[0] = *p; }
};

// One workgroup per row segment; each wave takes a contiguous quarter of it.
// A wave streams its range in windows of 64 elements: lane L loads element
// base + L (one coalesced load for the coordinates, one for the values), and
// the next window is requested before the current one is consumed, so the
// HBM latency of the view stream overlaps the factor gathers.  Inside a
// window the EPW element slots of the wave each take LPE consecutive
// elements (their coordinates and values are broadcast from the loading
// lanes) and walk them in view order (o1 ascending, then o0): t += v * F1[o0]
// over a run of equal o1, acc += t * F2[o1] once per run — the second factor
// row is gathered once per run (acc_r = sum_runs F2[o1, r] * sum_e v_e
// F1[o0_e, r], the reference's sum reassociated).  UNROLL gathers of a slot
// are in flight together.  View data uses non-temporal loads so it does not
// evict factor rows from L2.
template <int RT, int VEC, int WAVES, int UNROLL>
__device__ __forceinline__ void seg3_body(
    uint32_t seg, uint32_t rblk, int mode, const uint64_t* __restrict__ coords,
    const double* __restrict__ vals, const uint32_t* __restrict__ blk_row,
    const uint32_t* __restrict__ blk_start, const uint32_t* __restrict__ blk_cnt,
    const double* __restrict__ F1, const double* __restrict__ F2, double* __restrict__ FtV, int R)
{
    constexpr int LPE = RT / VEC;          // lanes per element = elements per slot per window
    constexpr int U = (UNROLL < LPE) ? UNROLL : LPE;
    static_assert(SEG_WAVE % LPE == 0, "rank tile must divide the wave");

    const uint32_t row = blk_row[seg];
    const uint32_t start = blk_start[seg];
    const uint32_t cnt = blk_cnt[seg];

    const int tid = threadIdx.x;
    const int lane = tid & (SEG_WAVE - 1);
    const int wave = tid / SEG_WAVE;
    const int slot = lane / LPE;
    const int r0 = int(rblk) * RT + (lane % LPE) * VEC;   // first rank of this lane
    const bool rank_ok = r0 < R;
    const int rr = rank_ok ? r0 : 0;                            // in-bounds row offset

    // per-mode field shifts of the packed (i<<30 | j<<15 | k) coordinate
    const int sh0 = (mode == 0) ? 15 : 30;   // o0 = j (mode 0) or i
    const int sh1 = (mode == 2) ? 15 : 0;    // o1 = k (modes 0,1) or j

    // this wave's contiguous range of the segment
    const uint32_t wchunk = (cnt + WAVES - 1) / WAVES;
    const uint32_t lo = start + min(cnt, uint32_t(wave) * wchunk);
    const uint32_t hi = start + min(cnt, uint32_t(wave + 1) * wchunk);

    double acc[VEC], t[VEC];
#pragma unroll
    for (int q = 0; q < VEC; ++q) acc[q] = t[q] = 0.0;
    uint32_t cur = 0xFFFFFFFFu;   // o1 of the open run (none yet)

    auto close_run = [&](uint32_t o1) {
        Row<VEC> f2;
        f2.load(F2 + size_t(o1) * R + rr);
#pragma unroll
        for (int q = 0; q < VEC; ++q)
        {
            acc[q] += t[q] * f2.x[q];
            t[q] = 0.0;
        }
    };

    uint64_t pc = 0;
    double v = 0.0;
    if (lo + uint32_t(lane) < hi)
    {
        pc = __builtin_nontemporal_load(coords + lo + lane);
        v = __builtin_nontemporal_load(vals + lo + lane);
    }
    for (uint32_t base = lo; base < hi; base += SEG_WAVE)
    {
        // request the next window before consuming this one
        uint64_t pcn = 0;
        double vn = 0.0;
        if (base + SEG_WAVE + uint32_t(lane) < hi)
        {
            pcn = __builtin_nontemporal_load(coords + base + SEG_WAVE + lane);
            vn = __builtin_nontemporal_load(vals + base + SEG_WAVE + lane);
        }
        // this slot's elements: window positions [slot*LPE, slot*LPE + n)
        const int j0 = slot * LPE;
        const int left = int(hi - base) - j0;
        const int n = left < 0 ? 0 : (left > LPE ? LPE : left);
        for (int i = 0; i < n; i += U)
        {
            uint32_t o0[U], o1[U];
            double ev[U];
            Row<VEC> f1[U];
#pragma unroll
            for (int u = 0; u < U; ++u)
            {
                const int j = j0 + i + u;
                const uint64_t pj = __shfl(pc, j, SEG_WAVE);
                ev[u] = __shfl(v, j, SEG_WAVE);
                o0[u] = uint32_t(pj >> sh0) & 0x7FFFu;
                o1[u] = uint32_t(pj >> sh1) & 0x7FFFu;
            }
            // the F2 row a run boundary at position u closes: the previous o1
            // (known now), requested together with the F1 rows
            Row<VEC> f2[U];
            bool closes[U];
#pragma unroll
            for (int u = 0; u < U; ++u)
            {
                const uint32_t prev = (u == 0) ? cur : o1[u - 1];
                closes[u] = (i + u < n) && o1[u] != prev && prev != 0xFFFFFFFFu;
                if (i + u < n) f1[u].load(F1 + size_t(o0[u]) * R + rr);
                if (closes[u]) f2[u].load(F2 + size_t(prev) * R + rr);
            }
#pragma unroll
            for (int u = 0; u < U; ++u)
            {
                if (i + u >= n) break;
                if (closes[u])
                {
#pragma unroll
                    for (int q = 0; q < VEC; ++q)
                    {
                        acc[q] += t[q] * f2[u].x[q];
                        t[q] = 0.0;
                    }
                }
                cur = o1[u];
#pragma unroll
                for (int q = 0; q < VEC; ++q) t[q] += ev[u] * f1[u].x[q];
            }
        }
        pc = pcn;
        v = vn;
    }
    if (cur != 0xFFFFFFFFu) close_run(cur);
    if (!rank_ok)
    {
#pragma unroll
        for (int q = 0; q < VEC; ++q) acc[q] = 0.0;
    }

    // reduce the EPW element slots of the wave (lanes l, l^LPE, l^2LPE, ...)
#pragma unroll
    for (int off = LPE; off < SEG_WAVE; off <<= 1)
#pragma unroll
        for (int q = 0; q < VEC; ++q) acc[q] += __shfl_xor(acc[q], off, SEG_WAVE);

    if constexpr (WAVES == 1)
    {
        if (slot == 0 && rank_ok)
        {
            double* out = FtV + size_t(row) * R + r0;
#pragma unroll
            for (int q = 0; q < VEC; ++q)
                if ((VEC == 1 || r0 + q < R) && acc[q] != 0.0) atomicAdd(out + q, acc[q]);
        }
    }
    else
    {
        __shared__ double red[WAVES][RT];
        if (slot == 0)
#pragma unroll
            for (int q = 0; q < VEC; ++q) red[wave][(lane % LPE) * VEC + q] = acc[q];
        __syncthreads();
        for (int x = tid; x < RT; x += SEG_WAVE * WAVES)
        {
            const int r = int(rblk) * RT + x;
            if (r >= R) continue;
            double tot = 0.0;
#pragma unroll
            for (int w = 0; w < WAVES; ++w) tot += red[w][x];
            if (tot != 0.0) atomicAdd(FtV + size_t(row) * R + r, tot);
        }
    }
}


}  // namespace cptc_k
