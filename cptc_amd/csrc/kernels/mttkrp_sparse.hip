// Order-3 FP64 sparse MTTKRP over row-sorted segments, for CDNA4 wave64.
//
// Semantics (sparse.cu:614-711 and 271-333): for every segment b of one
// mode's row-sorted view, acc_r = sum_e (v_e * F1[o0_e, r]) * F2[o1_e, r] and
// FtV[blk_row[b], r] += acc_r (one atomic per (row, rank, segment), skipped
// when acc_r == 0).  Any R >= 1.
//
// Mapping.  A lane owns VEC consecutive ranks (VEC = 2: one 16-byte load per
// factor row per lane, so a wave reads a 1 KB R=128 row as 64 x 16 B fully
// coalesced).  LPE = RT / VEC lanes cover one element's rank tile RT; a wave
// carries EPW = 64 / LPE element slots ("rank-dependent element packing":
// R=128 -> 1, 64 -> 2, 32 -> 4, 16 -> 8, 8 -> 16 slots per wave).  Partial
// sums meet in registers (xor-shuffles across the EPW slots of a wave) and
// then in LDS across waves.  R > RT runs RT-wide rank blocks on grid.y.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "../host/hip_util.hpp"
#include "seg3_body.hpp"

#ifndef CPTC_SPARSE3_UNROLL
#define CPTC_SPARSE3_UNROLL 8   // gathers in flight per element slot
#endif
#ifndef CPTC_SPARSE3_LANES_UNROLL
#define CPTC_SPARSE3_LANES_UNROLL 2   // elements per batch and slot, R <= 64
#endif

namespace {

constexpr int WAVE = 64;

// The kernel body (cptc_k::seg3_body) is in seg3_body.hpp.
template <int RT, int VEC, int WAVES, int UNROLL>
__global__ __launch_bounds__(WAVE* WAVES) void mttkrp3_seg_kernel(
    int mode, const uint64_t* __restrict__ coords, const double* __restrict__ vals,
    const uint32_t* __restrict__ blk_row, const uint32_t* __restrict__ blk_start,
    const uint32_t* __restrict__ blk_cnt, const double* __restrict__ F1,
    const double* __restrict__ F2, double* __restrict__ FtV, int R)
{
    cptc_k::seg3_body<RT, VEC, WAVES, UNROLL>(blockIdx.x, blockIdx.y, mode, coords, vals, blk_row,
                                              blk_start, blk_cnt, F1, F2, FtV, R);
}

// R in (64, 128] with 16-byte rows: one element per wave (LPE = 64), so the
// window position, the element's coordinates and value, the run state and
// the factor-row addresses are the same for every lane.  This variant keeps
// them wave-uniform and spends as few issue slots per element as it can,
// because the kernel shares its CUs with the MFMA tile kernel and every
// slot it frees goes to that kernel:
//   * the mode is a template parameter (constant field shifts);
//   * per 64-element window each lane decodes its own element once into the
//     byte offsets of its F1 and F2 rows; per element two v_readlane move
//     them to scalar registers, and the row loads are buffer loads with that
//     offset in soffset and the lane's fixed rank offset in voffset (no
//     per-element address arithmetic);
//   * the window's values are broadcast from a per-wave LDS slot (LDS pipe)
//     instead of by v_readlane;
//   * full windows run without per-element bound checks.
// Same sum and order as mttkrp3_seg_kernel.  The waves-per-EU bound keeps
// the register allocation free to hold UNROLL gathers in flight; UNROLL = 8
// ran fastest beside the MFMA tile kernel (config 3: 12.2 ms per iteration
// against 13.0 at UNROLL = 16 and 12.6 for the general kernel, before the
// issue-slot changes above took it to 11.7).
#ifndef CPTC_SPARSE3_WAVE_UNROLL
#define CPTC_SPARSE3_WAVE_UNROLL 8   // gathers in flight per wave
#endif
template <int MODE, int WAVES, int UNROLL>
__global__ __launch_bounds__(WAVE* WAVES) __attribute__((amdgpu_waves_per_eu(1, 3))) void mttkrp3_seg_wave_kernel(
    const uint64_t* __restrict__ coords, const double* __restrict__ vals,
    const uint32_t* __restrict__ blk_row, const uint32_t* __restrict__ blk_start,
    const uint32_t* __restrict__ blk_cnt, const double* __restrict__ F1,
    const double* __restrict__ F2, double* __restrict__ FtV, int R)
{
    constexpr int RT = 128;
    constexpr int U = UNROLL;
    // run state "no open run"; row offsets are < 2^31, so never equal to it
    constexpr uint32_t NONE = 0xFFFFFFFFu;
    const uint32_t seg = blockIdx.x;
    const uint32_t row = blk_row[seg];
    const uint32_t start = blk_start[seg];
    const uint32_t cnt = blk_cnt[seg];

    const int tid = threadIdx.x;
    const int lane = tid & (WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / WAVE);
    const int r0 = int(blockIdx.y) * RT + lane * 2;
    const bool rank_ok = r0 < R;
    const int rr = rank_ok ? r0 : 0;
    constexpr int sh0 = (MODE == 0) ? 15 : 30;
    constexpr int sh1 = (MODE == 2) ? 15 : 0;
    // factor rows by buffer loads: the row offset o*R*8 in soffset (scalar),
    // the lane's rank offset in voffset (fixed), no per-element vector
    // address arithmetic
    const __amdgpu_buffer_rsrc_t rs1 =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<double*>(F1), short(0), 0x7FFFFFFF, 0x00020000);
    const __amdgpu_buffer_rsrc_t rs2 =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<double*>(F2), short(0), 0x7FFFFFF0, 0x00020000);
    const uint32_t voff = uint32_t(rr) * 8u;
    const uint32_t rowb = uint32_t(R) * 8u;
    auto row_load = [&](const __amdgpu_buffer_rsrc_t& rs, uint32_t off) {
        const auto w = __builtin_amdgcn_raw_buffer_load_b128(rs, voff, off, 0);
        return make_double2(
            __longlong_as_double((long long)((uint64_t(uint32_t(w[1])) << 32) | uint32_t(w[0]))),
            __longlong_as_double((long long)((uint64_t(uint32_t(w[3])) << 32) | uint32_t(w[2]))));
    };

    const uint32_t wchunk = (cnt + WAVES - 1) / WAVES;
    const uint32_t lo = start + min(cnt, uint32_t(wave) * wchunk);
    const uint32_t hi = start + min(cnt, uint32_t(wave + 1) * wchunk);

    double acc0 = 0.0, acc1 = 0.0, t0 = 0.0, t1 = 0.0;
    uint32_t cur = NONE;

    uint64_t pc = 0;
    double v = 0.0;
    if (lo + uint32_t(lane) < hi)
    {
        pc = __builtin_nontemporal_load(coords + lo + lane);
        v = __builtin_nontemporal_load(vals + lo + lane);
    }
    // each window's values are broadcast from a per-wave LDS slot (LDS
    // pipe) instead of by v_readlane (VALU); a wave's LDS operations are
    // processed in order, so its own writes are visible to its later reads
    __shared__ double vbuf[WAVES][WAVE];
    double* const vw = vbuf[wave];
    // one batch of U elements starting at window position i; FULL: all U
    // elements exist (full 64-element window, no per-element guards)
    auto batch = [&](auto full, int i, int n, uint32_t off1_l, uint32_t off2_l) {
        constexpr bool FULL = decltype(full)::value;
        uint32_t o0[U], o1[U];
        double ev[U];
#pragma unroll
        for (int u = 0; u < U; ++u)
        {
            const int j = i + u;   // < 64: i <= 56 when U = 8
            o0[u] = uint32_t(__builtin_amdgcn_readlane(int(off1_l), j));
            o1[u] = uint32_t(__builtin_amdgcn_readlane(int(off2_l), j));
            ev[u] = vw[j];
        }
        double2 f1[U], f2[U];
        bool closes[U];
#pragma unroll
        for (int u = 0; u < U; ++u)
        {
            const bool live = FULL || i + u < n;
            const uint32_t prev = (u == 0) ? cur : o1[u - 1];
            // within a batch prev is an element's offset, never NONE
            closes[u] = live && o1[u] != prev && (u > 0 || prev != NONE);
            if (live) f1[u] = row_load(rs1, o0[u]);
            if (closes[u]) f2[u] = row_load(rs2, prev);
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
        {
            if (FULL || i + u < n)
            {
                if (closes[u])
                {
                    acc0 += t0 * f2[u].x;
                    acc1 += t1 * f2[u].y;
                    t0 = t1 = 0.0;
                }
                cur = o1[u];
                t0 += ev[u] * f1[u].x;
                t1 += ev[u] * f1[u].y;
            }
        }
    };
    for (uint32_t base = lo; base < hi; base += WAVE)
    {
        uint64_t pcn = 0;
        double vn = 0.0;
        if (base + WAVE + uint32_t(lane) < hi)
        {
            pcn = __builtin_nontemporal_load(coords + base + WAVE + lane);
            vn = __builtin_nontemporal_load(vals + base + WAVE + lane);
        }
        const int n = int(min(uint32_t(WAVE), hi - base));
        // each lane decodes its element once: byte offsets of its F1 and F2
        // rows (o * R * 8 < 2^31), broadcast per element by v_readlane
        const uint32_t off1_l = (uint32_t(pc >> sh0) & 0x7FFFu) * rowb;
        const uint32_t off2_l = (uint32_t(pc >> sh1) & 0x7FFFu) * rowb;
        asm volatile("" ::: "memory");   // the previous window's reads come first
        vw[lane] = v;
        asm volatile("" ::: "memory");
        if (n == WAVE)
        {
#pragma nounroll
            for (int i = 0; i < WAVE; i += U) batch(std::true_type{}, i, n, off1_l, off2_l);
        }
        else
        {
#pragma nounroll
            for (int i = 0; i < n; i += U) batch(std::false_type{}, i, n, off1_l, off2_l);
        }
        pc = pcn;
        v = vn;
    }
    if (cur != NONE)
    {
        const double2 f2 = row_load(rs2, cur);
        acc0 += t0 * f2.x;
        acc1 += t1 * f2.y;
    }
    if (!rank_ok) acc0 = acc1 = 0.0;

    __shared__ double red[WAVES][RT];
    red[wave][lane * 2] = acc0;
    red[wave][lane * 2 + 1] = acc1;
    __syncthreads();
    for (int x = tid; x < RT; x += WAVE * WAVES)
    {
        const int r = int(blockIdx.y) * RT + x;
        if (r >= R) continue;
        double tot = 0.0;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) tot += red[w][x];
        if (tot != 0.0) atomicAdd(FtV + size_t(row) * R + r, tot);
    }
}

// R <= 64 with 16-byte rows: EPW = 128 / RT element slots per wave (RT = 8,
// 16, 32, 64 -> 16, 8, 4, 2 slots of LPE = RT / 2 lanes), with the sum and
// run logic of mttkrp3_seg_kernel; the per-element work is cut, because at
// these R a lane's two ranks per element leave that kernel bound by
// instruction issue and by the latency of its window stream (config 2 at
// R = 32: 21 VALU, 12 SALU and 4 LDS instructions per element and slot):
//   * the mode is a template parameter (constant field shifts);
//   * a wave loads its whole range of the segment (up to CH elements) at
//     once, each lane decodes its elements into the byte offsets of their
//     F1 and F2 rows and writes {off1, off2, value} as 16-byte records to a
//     per-wave LDS array; no stream load is then left to wait behind the
//     row gathers (the hardware waits for loads in issue order);
//   * slot s takes a contiguous share of the range (runs of equal o1 are
//     cut only at share boundaries, not every 64 elements) and reads each
//     of its elements with one broadcast ds_read_b128;
//   * rows are buffer loads at voffset = the lane's rank offset + the row's
//     byte offset (o * R * 8 < 2^31);
//   * when every share holds the same multiple of U elements the batches
//     run without per-element guards; otherwise each element is guarded
//     (records past the range hold row 0 and value 0, so every load stays
//     in bounds).
constexpr int LANES_CH = 256;             // elements per wave and pass (a 1024-element segment / 4 waves)
constexpr int LANES_REC = LANES_CH + 32;  // records per wave: reads run past the range by < EPW + U

template <int MODE, int RT, int WAVES, int U>
__global__ __launch_bounds__(WAVE* WAVES) void mttkrp3_seg_lanes_kernel(
    const uint64_t* __restrict__ coords, const double* __restrict__ vals,
    const uint32_t* __restrict__ blk_row, const uint32_t* __restrict__ blk_start,
    const uint32_t* __restrict__ blk_cnt, const double* __restrict__ F1,
    const double* __restrict__ F2, double* __restrict__ FtV, int R)
{
    constexpr int LPE = RT / 2;           // lanes per element
    constexpr int EPW = WAVE / LPE;       // element slots per wave
    static_assert(RT <= 64 && LPE % U == 0 && EPW + U <= LANES_REC - LANES_CH,
                  "records must cover the reads past the range");
    constexpr uint32_t NONE = 0xFFFFFFFFu;   // no open run (row offsets are < 2^31)
    const uint32_t seg = blockIdx.x;
    const uint32_t row = blk_row[seg];
    const uint32_t start = blk_start[seg];
    const uint32_t cnt = blk_cnt[seg];

    const int tid = threadIdx.x;
    const int lane = tid & (WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / WAVE);
    const int slot = lane / LPE;
    const int r0 = (lane % LPE) * 2;
    const bool rank_ok = r0 < R;
    const uint32_t voff = uint32_t(rank_ok ? r0 : 0) * 8u;
    constexpr int sh0 = (MODE == 0) ? 15 : 30;
    constexpr int sh1 = (MODE == 2) ? 15 : 0;
    const __amdgpu_buffer_rsrc_t rs1 =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<double*>(F1), short(0), 0x7FFFFFFF, 0x00020000);
    const __amdgpu_buffer_rsrc_t rs2 =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<double*>(F2), short(0), 0x7FFFFFFF, 0x00020000);
    const uint32_t rowb = uint32_t(R) * 8u;
    auto row_load = [&](const __amdgpu_buffer_rsrc_t& rs, uint32_t off) {
        const auto w = __builtin_amdgcn_raw_buffer_load_b128(rs, voff + off, 0u, 0);
        return make_double2(
            __longlong_as_double((long long)((uint64_t(uint32_t(w[1])) << 32) | uint32_t(w[0]))),
            __longlong_as_double((long long)((uint64_t(uint32_t(w[3])) << 32) | uint32_t(w[2]))));
    };

    const uint32_t wchunk = (cnt + WAVES - 1) / WAVES;
    const uint32_t lo = start + min(cnt, uint32_t(wave) * wchunk);
    const uint32_t hi = start + min(cnt, uint32_t(wave + 1) * wchunk);

    double acc0 = 0.0, acc1 = 0.0, t0 = 0.0, t1 = 0.0;
    uint32_t cur = NONE;

    struct alignas(16) Rec
    {
        uint32_t off1, off2;
        double v;
    };
    // the records, reused for the cross-wave sums at the end; a wave's LDS
    // operations are processed in order, so its own record writes are
    // visible to its later reads
    __shared__ Rec recs[WAVES][LANES_REC];
    static_assert(sizeof(recs) >= sizeof(double) * WAVES * RT, "reduction space");
    Rec* const rw = recs[wave];

    // one batch of U elements at share position i; FULL: all exist
    auto batch = [&](auto full, const Rec* rsl, int i, int n_slot) {
        constexpr bool FULL = decltype(full)::value;
        Rec e[U];
#pragma unroll
        for (int u = 0; u < U; ++u) e[u] = rsl[i + u];
        double2 f1[U], f2[U];
        bool closes[U];
#pragma unroll
        for (int u = 0; u < U; ++u)
        {
            const bool live = FULL || i + u < n_slot;
            const uint32_t prev = (u == 0) ? cur : e[u - 1].off2;
            closes[u] = live && e[u].off2 != prev && prev != NONE;
            f1[u] = row_load(rs1, e[u].off1);   // records hold valid offsets
            if (closes[u]) f2[u] = row_load(rs2, prev);
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
        {
            if (FULL || i + u < n_slot)
            {
                if (closes[u])
                {
                    acc0 += t0 * f2[u].x;
                    acc1 += t1 * f2[u].y;
                    t0 = t1 = 0.0;
                }
                cur = e[u].off2;
                t0 += e[u].v * f1[u].x;
                t1 += e[u].v * f1[u].y;
            }
        }
    };
    for (uint32_t cb = lo; cb < hi; cb += LANES_CH)
    {
        const uint32_t m = min(uint32_t(LANES_CH), hi - cb);
        // every position of the pass at once: unconditional loads from
        // clamped positions, zeroed past the range
        constexpr int K = LANES_CH / WAVE;
        uint64_t pc[K];
        double v[K];
#pragma unroll
        for (int k = 0; k < K; ++k)
        {
            const uint32_t e = min(uint32_t(lane + WAVE * k), m - 1);
            pc[k] = __builtin_nontemporal_load(coords + cb + e);
            v[k] = __builtin_nontemporal_load(vals + cb + e);
        }
        asm volatile("" ::: "memory");   // the previous pass's reads come first
#pragma unroll
        for (int k = 0; k < K; ++k)
        {
            const bool ok = uint32_t(lane + WAVE * k) < m;
            const uint64_t p = ok ? pc[k] : uint64_t(0);
            rw[lane + WAVE * k] = Rec{(uint32_t(p >> sh0) & 0x7FFFu) * rowb,
                                      (uint32_t(p >> sh1) & 0x7FFFu) * rowb, ok ? v[k] : 0.0};
        }
        if (lane < LANES_REC - LANES_CH) rw[LANES_CH + lane] = Rec{0u, 0u, 0.0};
        asm volatile("" ::: "memory");
        const int q = int(m + EPW - 1) / EPW;   // share per slot
        const Rec* const rsl = rw + slot * q;
        if (int(m) == EPW * q && q % U == 0)
        {
#pragma nounroll
            for (int i = 0; i < q; i += U) batch(std::true_type{}, rsl, i, q);
        }
        else
        {
            const int left = int(m) - slot * q;
            const int n_slot = left < 0 ? 0 : (left > q ? q : left);
#pragma nounroll
            for (int i = 0; i < q; i += U) batch(std::false_type{}, rsl, i, n_slot);
        }
    }
    if (cur != NONE)
    {
        const double2 f2 = row_load(rs2, cur);
        acc0 += t0 * f2.x;
        acc1 += t1 * f2.y;
    }
    if (!rank_ok) acc0 = acc1 = 0.0;
    // reduce the slots of the wave (lanes l, l ^ LPE, l ^ 2 LPE, ...)
#pragma unroll
    for (int off = LPE; off < WAVE; off <<= 1)
    {
        acc0 += __shfl_xor(acc0, off, WAVE);
        acc1 += __shfl_xor(acc1, off, WAVE);
    }
    __syncthreads();   // every wave's record reads are done
    double* const red = reinterpret_cast<double*>(&recs[0][0]);   // [WAVES][RT]
    if (slot == 0)
    {
        red[wave * RT + r0] = acc0;
        red[wave * RT + r0 + 1] = acc1;
    }
    __syncthreads();
    for (int x = tid; x < RT; x += WAVE * WAVES)
    {
        if (x >= R) continue;
        double tot = 0.0;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) tot += red[w * RT + x];
        if (tot != 0.0) atomicAdd(FtV + size_t(row) * R + x, tot);
    }
}

template <int RT, int VEC>
hipError_t launch_rt(int mode, const uint64_t* coords, const double* vals, const uint32_t* br,
                     const uint32_t* bs, const uint32_t* bc, size_t nblocks, const double* F1,
                     const double* F2, double* FtV, int R, hipStream_t s)
{
    constexpr int WAVES = 4;
    constexpr int UNROLL = CPTC_SPARSE3_UNROLL;
    const unsigned ry = unsigned((R + RT - 1) / RT);
    dim3 grid(unsigned(nblocks), ry);
    // the wave-uniform kernel addresses rows by 32-bit byte offsets o * R * 8
    // (o < 2^15), so it needs R * 8 * 2^15 < 2^31
    if (RT <= 64 && VEC == 2)
    {
        constexpr int RL = RT <= 64 ? RT : 64;   // (the branch is dead for RT = 128)
        constexpr int UL = CPTC_SPARSE3_LANES_UNROLL;
        const dim3 block(WAVE * WAVES);
        if (mode == 0)
            hipLaunchKernelGGL((mttkrp3_seg_lanes_kernel<0, RL, WAVES, UL>), grid, block, 0, s,
                               coords, vals, br, bs, bc, F1, F2, FtV, R);
        else if (mode == 1)
            hipLaunchKernelGGL((mttkrp3_seg_lanes_kernel<1, RL, WAVES, UL>), grid, block, 0, s,
                               coords, vals, br, bs, bc, F1, F2, FtV, R);
        else
            hipLaunchKernelGGL((mttkrp3_seg_lanes_kernel<2, RL, WAVES, UL>), grid, block, 0, s,
                               coords, vals, br, bs, bc, F1, F2, FtV, R);
    }
    else if (RT == 128 && VEC == 2 && R <= 8000)
    {
        const dim3 block(WAVE * WAVES);
        if (mode == 0)
            hipLaunchKernelGGL((mttkrp3_seg_wave_kernel<0, WAVES, CPTC_SPARSE3_WAVE_UNROLL>), grid,
                               block, 0, s, coords, vals, br, bs, bc, F1, F2, FtV, R);
        else if (mode == 1)
            hipLaunchKernelGGL((mttkrp3_seg_wave_kernel<1, WAVES, CPTC_SPARSE3_WAVE_UNROLL>), grid,
                               block, 0, s, coords, vals, br, bs, bc, F1, F2, FtV, R);
        else
            hipLaunchKernelGGL((mttkrp3_seg_wave_kernel<2, WAVES, CPTC_SPARSE3_WAVE_UNROLL>), grid,
                               block, 0, s, coords, vals, br, bs, bc, F1, F2, FtV, R);
    }
    else
        hipLaunchKernelGGL((mttkrp3_seg_kernel<RT, VEC, WAVES, UNROLL>), grid,
                           dim3(WAVE * WAVES), 0, s, mode, coords, vals, br, bs, bc, F1, F2, FtV,
                           R);
    return hipGetLastError();
}

// Elements [start, start + count) of one mode's row-sorted view, each
// adding v * F1[o0, r] * F2[o1, r] (that product order) to FtV[target, r]
// with one atomic per (element, rank), as mttkrp_range_generic_kernel
// (sparse.cu:340-397).  One wave per element, lanes over ranks: the factor
// rows are read and the atomics issued 64 ranks at a time, coalesced.
__global__ __launch_bounds__(256) void mttkrp3_range_kernel(int mode,
                                                            const uint64_t* __restrict__ coords,
                                                            const double* __restrict__ vals,
                                                            size_t start, size_t count,
                                                            const double* __restrict__ F1,
                                                            const double* __restrict__ F2,
                                                            double* __restrict__ FtV, int R)
{
    const int lane = threadIdx.x & 63;
    const size_t waves = size_t(gridDim.x) * (blockDim.x / 64);
    for (size_t e = size_t(blockIdx.x) * (blockDim.x / 64) + threadIdx.x / 64; e < count;
         e += waves)
    {
        const uint64_t c = coords[start + e];
        const double v = vals[start + e];
        const uint32_t i = uint32_t(c >> 30), j = uint32_t(c >> 15) & 0x7FFFu,
                       k = uint32_t(c) & 0x7FFFu;
        const uint32_t t = mode == 0 ? i : (mode == 1 ? j : k);
        const uint32_t o0 = mode == 0 ? j : i;
        const uint32_t o1 = mode == 2 ? j : k;
        const double* __restrict__ f1 = F1 + size_t(o0) * R;
        const double* __restrict__ f2 = F2 + size_t(o1) * R;
        double* __restrict__ out = FtV + size_t(t) * R;
        for (int r = lane; r < R; r += 64) atomicAdd(out + r, v * f1[r] * f2[r]);
    }
}

}  // namespace

extern "C" int cptc_mttkrp_sparse3_range(int mode, const uint64_t* d_coords, const double* d_vals,
                                         size_t start, size_t count, const double* d_F1,
                                         const double* d_F2, double* d_FtV, int R, void* stream)
{
    CPTC_REQUIRE(mode >= 0 && mode < 3 && R >= 1, CPTC_ERR_ARG,
                 "cptc_mttkrp_sparse3_range: mode %d R %d", mode, R);
    if (count == 0) return CPTC_OK;
    CPTC_REQUIRE(d_coords && d_vals && d_F1 && d_F2 && d_FtV, CPTC_ERR_ARG,
                 "cptc_mttkrp_sparse3_range: null pointer");
    const unsigned grid = cptc::grid_for(count, 4, 1u << 16);
    hipLaunchKernelGGL(mttkrp3_range_kernel, dim3(grid), dim3(256), 0, cptc::as_stream(stream),
                       mode, d_coords, d_vals, start, count, d_F1, d_F2, d_FtV, R);
    CPTC_LAUNCHED();
    return CPTC_OK;
}

extern "C" int cptc_mttkrp_sparse3(int mode, const uint64_t* d_coords, const double* d_vals,
                                   const uint32_t* d_blk_row, const uint32_t* d_blk_start,
                                   const uint32_t* d_blk_cnt, size_t nblocks, const double* d_F1,
                                   const double* d_F2, double* d_FtV, int R, void* stream)
{
    CPTC_REQUIRE(mode >= 0 && mode < 3, CPTC_ERR_ARG, "cptc_mttkrp_sparse3: mode %d", mode);
    CPTC_REQUIRE(R >= 1, CPTC_ERR_ARG, "cptc_mttkrp_sparse3: R %d", R);
    if (nblocks == 0) return CPTC_OK;
    CPTC_REQUIRE(nblocks < (size_t(1) << 31), CPTC_ERR_ARG, "cptc_mttkrp_sparse3: %zu segments",
                 nblocks);
    CPTC_REQUIRE(d_coords && d_vals && d_blk_row && d_blk_start && d_blk_cnt && d_F1 && d_F2 &&
                     d_FtV,
                 CPTC_ERR_ARG, "cptc_mttkrp_sparse3: null pointer");
    hipStream_t s = cptc::as_stream(stream);
    // 16-byte rows need an even R and 16-byte aligned factor bases.
    const bool vec2 = (R % 2 == 0) && ((reinterpret_cast<uintptr_t>(d_F1) & 15) == 0) &&
                      ((reinterpret_cast<uintptr_t>(d_F2) & 15) == 0);
    hipError_t e;
    if (vec2)
    {
        if (R <= 8)
            e = launch_rt<8, 2>(mode, d_coords, d_vals, d_blk_row, d_blk_start, d_blk_cnt, nblocks,
                                d_F1, d_F2, d_FtV, R, s);
        else if (R <= 16)
            e = launch_rt<16, 2>(mode, d_coords, d_vals, d_blk_row, d_blk_start, d_blk_cnt,
                                 nblocks, d_F1, d_F2, d_FtV, R, s);
        else if (R <= 32)
            e = launch_rt<32, 2>(mode, d_coords, d_vals, d_blk_row, d_blk_start, d_blk_cnt,
                                 nblocks, d_F1, d_F2, d_FtV, R, s);
        else if (R <= 64)
            e = launch_rt<64, 2>(mode, d_coords, d_vals, d_blk_row, d_blk_start, d_blk_cnt,
                                 nblocks, d_F1, d_F2, d_FtV, R, s);
        else
            e = launch_rt<128, 2>(mode, d_coords, d_vals, d_blk_row, d_blk_start, d_blk_cnt,
                                  nblocks, d_F1, d_F2, d_FtV, R, s);
    }
    else
    {
        if (R <= 8)
            e = launch_rt<8, 1>(mode, d_coords, d_vals, d_blk_row, d_blk_start, d_blk_cnt, nblocks,
                                d_F1, d_F2, d_FtV, R, s);
        else if (R <= 16)
            e = launch_rt<16, 1>(mode, d_coords, d_vals, d_blk_row, d_blk_start, d_blk_cnt,
                                 nblocks, d_F1, d_F2, d_FtV, R, s);
        else if (R <= 32)
            e = launch_rt<32, 1>(mode, d_coords, d_vals, d_blk_row, d_blk_start, d_blk_cnt,
                                 nblocks, d_F1, d_F2, d_FtV, R, s);
        else
            e = launch_rt<64, 1>(mode, d_coords, d_vals, d_blk_row, d_blk_start, d_blk_cnt,
                                 nblocks, d_F1, d_F2, d_FtV, R, s);
    }
    CPTC_REQUIRE(e == hipSuccess, CPTC_ERR_HIP, "cptc_mttkrp_sparse3 launch: %s",
                 hipGetErrorString(e));
    return CPTC_OK;
}
