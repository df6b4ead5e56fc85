// Element-gather probe of the blocked residual view: the element-level row
// gathers of mttkrp3_blk_kernel alone (mttkrp_blk.hip), in its work
// decomposition and order — the same chunks, spans and per-wave element
// ranges, one wave-uniform R-wide FP64 row per element, the same rows in
// flight per wave and resident waves per SIMD — with no run-level rows,
// LDS accumulation or atomics.  Its time is the floor those gathers set for
// the kernel on the same data (the L1/L2/MALL hits the real order gets
// included).  A measurement aid: the results are not used.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "../host/blk3_params.hpp"
#include "../host/hip_util.hpp"

namespace {

constexpr int WAVE = 64;
constexpr int PROBE_WAVES = 8;   // as mttkrp3_blk_kernel
constexpr int PROBE_U = 4;       // rows in flight per wave, as mttkrp3_blk_kernel
#define CPTC_PROBE_WPE 6         // resident waves per SIMD, as mttkrp3_blk_kernel
// the LDS of mttkrp3_blk_kernel (TB x 128 FP64 accumulator, KB staged rows,
// the waves' value buffers; TB, KB from blk3_params.hpp), reserved and
// unused, so that as many workgroups are resident per CU as for the kernel
// (more would widen the set of rows in flight and change the L2 hits the
// probe is there to see)
constexpr size_t PROBE_LDS =
    ((size_t(1) << CPTC_BLK3_LG_TB) * 128 + (size_t(1) << CPTC_BLK3_LG_KB) * 128 +
     PROBE_WAVES * WAVE) * sizeof(double);

template <int MODE>
__global__ __launch_bounds__(WAVE* PROBE_WAVES) __attribute__((amdgpu_waves_per_eu(CPTC_PROBE_WPE, CPTC_PROBE_WPE))) void gather_probe_kernel(
    const uint64_t* __restrict__ coords, const uint32_t* __restrict__ span_start,
    const uint32_t* __restrict__ span_cnt, const uint32_t* __restrict__ chunk_span0,
    const uint32_t* __restrict__ chunk_nspan, const double* __restrict__ F1, int R,
    double* __restrict__ sink)
{
    constexpr int sh0 = (MODE == 0) ? 15 : 30;   // element-level coordinate
    const uint32_t ch = blockIdx.x;
    const uint32_t sp0 = chunk_span0[ch];
    const uint32_t nsp = chunk_nspan[ch];
    const int lane = threadIdx.x & (WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) / WAVE);
    const int r0 = lane * 2;
    const uint32_t voff = uint32_t(r0 < R ? r0 : 0) * 8u;
    const uint32_t rowb = uint32_t(R) * 8u;
    const __amdgpu_buffer_rsrc_t rs1 =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<double*>(F1), short(0), 0x7FFFFFFF, 0x00020000);
    double a0 = 0.0, a1 = 0.0;
    for (uint32_t sp = sp0; sp < sp0 + nsp; ++sp)
    {
        const uint32_t st = span_start[sp];
        const uint32_t cnt = span_cnt[sp];
        const uint32_t wchunk = (cnt + PROBE_WAVES - 1) / PROBE_WAVES;
        const uint32_t lo = st + min(cnt, uint32_t(wave) * wchunk);
        const uint32_t hi = st + min(cnt, uint32_t(wave + 1) * wchunk);
        // the window's coordinates, and the next window's loading while this
        // one's rows are gathered (as in the kernel)
        uint64_t pc = (lo + uint32_t(lane) < hi) ? __builtin_nontemporal_load(coords + lo + lane)
                                                 : uint64_t(0);
        for (uint32_t base = lo; base < hi; base += WAVE)
        {
            const uint64_t pcn = (base + WAVE + uint32_t(lane) < hi)
                                     ? __builtin_nontemporal_load(coords + base + WAVE + lane)
                                     : uint64_t(0);
            const uint32_t n = min(uint32_t(WAVE), hi - base);
            const uint32_t off_l = (uint32_t(pc >> sh0) & 0x7FFFu) * rowb;
            for (uint32_t j = 0; j < n; j += PROBE_U)
            {
                decltype(__builtin_amdgcn_raw_buffer_load_b128(rs1, 0u, 0u, 0)) w[PROBE_U];
#pragma unroll
                for (int u = 0; u < PROBE_U; ++u)
                {
                    // lanes past n hold offset 0 (row 0): an in-bounds row
                    const uint32_t off = uint32_t(__builtin_amdgcn_readlane(int(off_l), int(j) + u));
                    w[u] = __builtin_amdgcn_raw_buffer_load_b128(rs1, voff, off, 0);
                }
#pragma unroll
                for (int u = 0; u < PROBE_U; ++u)
                {
                    if (j + uint32_t(u) >= n) break;
                    a0 += __longlong_as_double(
                        (long long)((uint64_t(uint32_t(w[u][1])) << 32) | uint32_t(w[u][0])));
                    a1 += __longlong_as_double(
                        (long long)((uint64_t(uint32_t(w[u][3])) << 32) | uint32_t(w[u][2])));
                }
            }
            pc = pcn;
        }
    }
    // a store the compiler cannot drop (the sums are never this value for
    // finite factors), so every gather above stays
    if (a0 + a1 == -1.25e300) sink[0] = a0;
}

}  // namespace

extern "C" int cptc_gather_probe3_blk(int mode, const uint64_t* d_coords,
                                      const uint32_t* d_span_start, const uint32_t* d_span_cnt,
                                      const uint32_t* d_chunk_span0, const uint32_t* d_chunk_nspan,
                                      size_t nchunk, const double* d_F1, int R, double* d_sink,
                                      void* stream)
{
    CPTC_REQUIRE(mode >= 0 && mode < 3 && R > 64 && R <= 128 && R % 2 == 0, CPTC_ERR_ARG,
                 "cptc_gather_probe3_blk: mode %d R %d (even R in 65..128)", mode, R);
    if (nchunk == 0) return CPTC_OK;
    CPTC_REQUIRE(nchunk < (size_t(1) << 31), CPTC_ERR_ARG, "cptc_gather_probe3_blk: sizes");
    CPTC_REQUIRE(d_coords && d_span_start && d_span_cnt && d_chunk_span0 && d_chunk_nspan && d_F1 &&
                     d_sink,
                 CPTC_ERR_ARG, "cptc_gather_probe3_blk: null pointer");
    CPTC_REQUIRE((reinterpret_cast<uintptr_t>(d_F1) & 15) == 0, CPTC_ERR_ARG,
                 "cptc_gather_probe3_blk: the factor must be 16-byte aligned");
    hipStream_t s = cptc::as_stream(stream);
    const dim3 grid{unsigned(nchunk)}, block{unsigned(WAVE * PROBE_WAVES)};
    if (mode == 0)
        hipLaunchKernelGGL(gather_probe_kernel<0>, grid, block, PROBE_LDS, s, d_coords, d_span_start,
                           d_span_cnt, d_chunk_span0, d_chunk_nspan, d_F1, R, d_sink);
    else if (mode == 1)
        hipLaunchKernelGGL(gather_probe_kernel<1>, grid, block, PROBE_LDS, s, d_coords, d_span_start,
                           d_span_cnt, d_chunk_span0, d_chunk_nspan, d_F1, R, d_sink);
    else
        hipLaunchKernelGGL(gather_probe_kernel<2>, grid, block, PROBE_LDS, s, d_coords, d_span_start,
                           d_span_cnt, d_chunk_span0, d_chunk_nspan, d_F1, R, d_sink);
    CPTC_LAUNCHED();
    return CPTC_OK;
}
