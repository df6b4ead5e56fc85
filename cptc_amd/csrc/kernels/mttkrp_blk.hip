// Order-3 FP64 sparse MTTKRP over the blocked residual layout, R in
// (64, 128], for CDNA4 wave64: the sum of the row-segment kernels in
// mttkrp_sparse.hip (sparse.cu:614-711), over the view of a mode re-sorted
// by (target row block, run-level block) so that a workgroup stages the
// run-level factor rows of a block pair in LDS.  blk_views3_device
// (layout.hip) builds the layout.
#include <hip/hip_runtime.h>

#include "../host/blk3_params.hpp"
#include "../host/hip_util.hpp"

#ifndef CPTC_BLK3_UNROLL
#define CPTC_BLK3_UNROLL 4   // gathers in flight per wave
#endif
#ifndef CPTC_BLK3_WPE
#define CPTC_BLK3_WPE 6      // resident waves per SIMD the registers are sized for
#endif

namespace {

constexpr int WAVE = 64;
// 8 waves per workgroup, 6 resident per SIMD (<= 80 VGPRs; 3 workgroups'
// 52 KB of LDS per CU): config 3 measured 2.45-2.48 ms per launch against
// 3.0 with 4 waves, 3 per SIMD and 8 gathers in flight per wave.
constexpr int BLK_WAVES = 8;

// Blocked residual view, R in (64, 128] (one element per wave, as the
// wave-uniform kernel).  The view of a mode is re-sorted by (target row
// block of TB rows, run-level block of KB rows, target, o1, o0) — inside a
// block pair the elements keep the reference view's (target, o1, o0) order
// — and cut into spans (one block pair, or several consecutive unstaged
// ones) and chunks (consecutive spans of one row block, one workgroup).
// For a staged span the KB run-level factor rows are copied into LDS once
// and every run of the span reads its row from there instead of gathering
// it (config 3: the per-run gathers, most of them L1 misses, drop to ~30 %).
// Per-row partial sums are added into a TB x 128 FP64 LDS accumulator (LDS
// atomics: a row can straddle two waves' ranges) and flushed to FtV with one
// global atomic per (row, rank) per chunk.  Same sum as mttkrp3_seg_kernel,
// reassociated: sum over runs of F2[o1] * sum over the run of v F1[o0].
template <int MODE, int LG_TB, int LG_KB, int WAVES, int UNROLL>
__global__ __launch_bounds__(WAVE* WAVES) __attribute__((amdgpu_waves_per_eu(CPTC_BLK3_WPE, CPTC_BLK3_WPE))) void mttkrp3_blk_kernel(
    const uint64_t* __restrict__ coords, const double* __restrict__ vals,
    const uint32_t* __restrict__ span_start, const uint32_t* __restrict__ span_cnt,
    const uint32_t* __restrict__ span_kb, const uint32_t* __restrict__ chunk_span0,
    const uint32_t* __restrict__ chunk_nspan, const uint32_t* __restrict__ chunk_tb,
    const double* __restrict__ F1, const double* __restrict__ F2, double* __restrict__ FtV,
    int R, uint32_t dimT, uint32_t dimF2)
{
    constexpr int RT = 128;
    constexpr int TB = 1 << LG_TB;
    constexpr int KB = 1 << LG_KB;
    constexpr int U = UNROLL;
    static_assert(WAVE % U == 0, "a full window is whole batches of U elements");
    constexpr uint32_t NONE = 0xFFFFFFFFu;
    constexpr int sh_t = (MODE == 0) ? 30 : (MODE == 1) ? 15 : 0;
    constexpr int sh0 = (MODE == 0) ? 15 : 30;
    constexpr int sh1 = (MODE == 2) ? 15 : 0;
    __shared__ double acc_l[TB * RT];
    __shared__ double stg[KB * RT];
    __shared__ double vbuf[WAVES][WAVE];

    const uint32_t ch = blockIdx.x;
    const uint32_t sp0 = chunk_span0[ch];
    const uint32_t nsp = chunk_nspan[ch];
    const uint32_t tb = chunk_tb[ch];
    const int tid = threadIdx.x;
    const int lane = tid & (WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / WAVE);
    const int r0 = lane * 2;
    const bool rank_ok = r0 < R;
    const int rr = rank_ok ? r0 : 0;
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
    auto lds_row = [&](const double* base, uint32_t off) {
        return *reinterpret_cast<const double2*>(reinterpret_cast<const char*>(base) + off + voff);
    };
    for (int x = tid; x < TB * RT; x += WAVE * WAVES) acc_l[x] = 0.0;
    double* const vw = vbuf[wave];

    for (uint32_t sp = sp0; sp < sp0 + nsp; ++sp)
    {
        const uint32_t st = span_start[sp];
        const uint32_t cnt = span_cnt[sp];
        const uint32_t kbw = span_kb[sp];
        const bool staged = (kbw >> 31) != 0;
        const uint32_t kb0 = (kbw & 0x7FFFFFFFu) << LG_KB;   // first staged row
        __syncthreads();   // the previous span's LDS rows are no longer read
        if (staged)
        {
            for (int x = tid; x < KB * (RT / 2); x += WAVE * WAVES)
            {
                const int row = x / (RT / 2);
                const int c = (x % (RT / 2)) * 2;
                const uint32_t g = kb0 + uint32_t(row);
                double2 f = make_double2(0.0, 0.0);
                if (g < dimF2 && c < R) f = *reinterpret_cast<const double2*>(F2 + size_t(g) * R + c);
                *reinterpret_cast<double2*>(stg + row * RT + c) = f;
            }
            __syncthreads();
        }
        const uint32_t wchunk = (cnt + WAVES - 1) / WAVES;
        const uint32_t lo = st + min(cnt, uint32_t(wave) * wchunk);
        const uint32_t hi = st + min(cnt, uint32_t(wave + 1) * wchunk);

        // The span's body, instantiated separately for staged and unstaged
        // spans: with one body for both, the compiler gives the run-level row
        // one register block whether it comes from LDS or from a global load,
        // and before each LDS read into it waits for every global load in
        // flight (s_waitcnt vmcnt(0)), the element gathers included.
        auto run_span = [&](auto staged_t) {
        constexpr bool STAGED = decltype(staged_t)::value;
        double acc0 = 0.0, acc1 = 0.0, t0 = 0.0, t1 = 0.0;
        uint32_t cur = NONE;      // run key (target row in block << 15 | o1) of the open run
        uint32_t cur_f2 = 0;      // byte offset of its F2 row (LDS when staged)
        auto flush = [&](uint32_t key) {
            // acc of the row in `key` into the LDS accumulator
            if (rank_ok)
            {
                double* a = acc_l + (key >> 15) * RT + r0;
                if (acc0 != 0.0) atomicAdd(a, acc0);
                if (acc1 != 0.0) atomicAdd(a + 1, acc1);
            }
            acc0 = acc1 = 0.0;
        };
        auto f2_row = [&](uint32_t off) {
            if constexpr (STAGED)
                return lds_row(stg, off);
            else
                return row_load(rs2, off);
        };

        uint64_t pc = 0;
        double v = 0.0;
        if (lo + uint32_t(lane) < hi)
        {
            pc = __builtin_nontemporal_load(coords + lo + lane);
            v = __builtin_nontemporal_load(vals + lo + lane);
        }
        auto batch = [&](auto full, int i, int n, uint32_t off1_l, uint32_t key_l,
                         uint32_t off2_l) {
            constexpr bool FULL = decltype(full)::value;
            uint32_t o0[U], k2[U], f2o[U];
            double ev[U];
#pragma unroll
            for (int u = 0; u < U; ++u)
            {
                const int j = i + u;
                o0[u] = uint32_t(__builtin_amdgcn_readlane(int(off1_l), j));
                k2[u] = uint32_t(__builtin_amdgcn_readlane(int(key_l), j));
                f2o[u] = uint32_t(__builtin_amdgcn_readlane(int(off2_l), j));
                ev[u] = vw[j];
            }
            double2 f1[U], f2[U];
            bool closes[U];
#pragma unroll
            for (int u = 0; u < U; ++u)
            {
                const bool live = FULL || i + u < n;
                const uint32_t prev = (u == 0) ? cur : k2[u - 1];
                const uint32_t prev_off = (u == 0) ? cur_f2 : f2o[u - 1];
                closes[u] = live && k2[u] != prev && (u > 0 || prev != NONE);
                if (live) f1[u] = row_load(rs1, o0[u]);
                if (closes[u]) f2[u] = f2_row(prev_off);
            }
#pragma unroll
            for (int u = 0; u < U; ++u)
            {
                if (FULL || i + u < n)
                {
                    const uint32_t prev = (u == 0) ? cur : k2[u - 1];
                    if (closes[u])
                    {
                        acc0 += t0 * f2[u].x;
                        acc1 += t1 * f2[u].y;
                        t0 = t1 = 0.0;
                        if ((prev >> 15) != (k2[u] >> 15)) flush(prev);
                    }
                    cur = k2[u];
                    cur_f2 = f2o[u];
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
            const uint32_t t = uint32_t(pc >> sh_t) & 0x7FFFu;
            const uint32_t o1 = uint32_t(pc >> sh1) & 0x7FFFu;
            const uint32_t off1_l = (uint32_t(pc >> sh0) & 0x7FFFu) * rowb;
            const uint32_t key_l = ((t & uint32_t(TB - 1)) << 15) | o1;
            const uint32_t off2_l = STAGED ? (o1 - kb0) * uint32_t(RT * 8) : o1 * rowb;
            asm volatile("" ::: "memory");   // the previous window's reads come first
            vw[lane] = v;
            asm volatile("" ::: "memory");
            if (n == WAVE)
            {
#pragma nounroll
                for (int i = 0; i < WAVE; i += U)
                    batch(std::true_type{}, i, n, off1_l, key_l, off2_l);
            }
            else
            {
#pragma nounroll
                for (int i = 0; i < n; i += U)
                    batch(std::false_type{}, i, n, off1_l, key_l, off2_l);
            }
            pc = pcn;
            v = vn;
        }
        if (cur != NONE)
        {
            const double2 f2 = f2_row(cur_f2);
            acc0 += t0 * f2.x;
            acc1 += t1 * f2.y;
            flush(cur);
        }
        };
        if (staged)
            run_span(std::true_type{});
        else
            run_span(std::false_type{});
}
    __syncthreads();
    for (int x = tid; x < TB * RT; x += WAVE * WAVES)
    {
        const uint32_t row = tb * uint32_t(TB) + uint32_t(x / RT);
        const int c = x % RT;
        const double a = acc_l[x];
        if (row < dimT && c < R && a != 0.0) atomicAdd(FtV + size_t(row) * R + c, a);
    }
}

template <int MODE>
hipError_t launch_blk(const uint64_t* coords, const double* vals, const uint32_t* ss,
                      const uint32_t* sc, const uint32_t* sk, const uint32_t* c0,
                      const uint32_t* cn, const uint32_t* ct, size_t nchunk, const double* F1,
                      const double* F2, double* FtV, int R, uint32_t dimT, uint32_t dimF2,
                      hipStream_t s)
{
    hipLaunchKernelGGL((mttkrp3_blk_kernel<MODE, CPTC_BLK3_LG_TB, CPTC_BLK3_LG_KB, BLK_WAVES,
                                           CPTC_BLK3_UNROLL>),
                       dim3(unsigned(nchunk)), dim3(WAVE * BLK_WAVES), 0, s, coords, vals, ss, sc, sk, c0,
                       cn, ct, F1, F2, FtV, R, dimT, dimF2);
    return hipGetLastError();
}
}  // namespace

extern "C" int cptc_mttkrp_sparse3_blk(int mode, const uint64_t* d_coords, const double* d_vals,
                                       const uint32_t* d_span_start, const uint32_t* d_span_cnt,
                                       const uint32_t* d_span_kb, const uint32_t* d_chunk_span0,
                                       const uint32_t* d_chunk_nspan, const uint32_t* d_chunk_tb,
                                       size_t nchunk, const double* d_F1, const double* d_F2,
                                       double* d_FtV, int R, uint64_t dim_target,
                                       uint64_t dim_f2, void* stream)
{
    CPTC_REQUIRE(mode >= 0 && mode < 3 && R > 64 && R <= 128 && R % 2 == 0, CPTC_ERR_ARG,
                 "cptc_mttkrp_sparse3_blk: mode %d R %d (even R in 65..128)", mode, R);
    if (nchunk == 0) return CPTC_OK;
    CPTC_REQUIRE(nchunk < (size_t(1) << 31) && dim_target < 32768 && dim_f2 < 32768,
                 CPTC_ERR_ARG, "cptc_mttkrp_sparse3_blk: sizes");
    CPTC_REQUIRE(d_coords && d_vals && d_span_start && d_span_cnt && d_span_kb && d_chunk_span0 &&
                     d_chunk_nspan && d_chunk_tb && d_F1 && d_F2 && d_FtV,
                 CPTC_ERR_ARG, "cptc_mttkrp_sparse3_blk: null pointer");
    CPTC_REQUIRE(((reinterpret_cast<uintptr_t>(d_F1) | reinterpret_cast<uintptr_t>(d_F2)) & 15) == 0,
                 CPTC_ERR_ARG, "cptc_mttkrp_sparse3_blk: factors must be 16-byte aligned");
    hipStream_t s = cptc::as_stream(stream);
    hipError_t e;
    const uint32_t dT = uint32_t(dim_target), dF = uint32_t(dim_f2);
    if (mode == 0)
        e = launch_blk<0>(d_coords, d_vals, d_span_start, d_span_cnt, d_span_kb, d_chunk_span0,
                          d_chunk_nspan, d_chunk_tb, nchunk, d_F1, d_F2, d_FtV, R, dT, dF, s);
    else if (mode == 1)
        e = launch_blk<1>(d_coords, d_vals, d_span_start, d_span_cnt, d_span_kb, d_chunk_span0,
                          d_chunk_nspan, d_chunk_tb, nchunk, d_F1, d_F2, d_FtV, R, dT, dF, s);
    else
        e = launch_blk<2>(d_coords, d_vals, d_span_start, d_span_cnt, d_span_kb, d_chunk_span0,
                          d_chunk_nspan, d_chunk_tb, nchunk, d_F1, d_F2, d_FtV, R, dT, dF, s);
    CPTC_REQUIRE(e == hipSuccess, CPTC_ERR_HIP, "cptc_mttkrp_sparse3_blk launch: %s",
                 hipGetErrorString(e));
    return CPTC_OK;
}
