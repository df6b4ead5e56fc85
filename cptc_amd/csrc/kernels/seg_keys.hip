// FP64 segment MTTKRP of the generic N-order path over packed level keys.
//
// Same contract as the segment kernel over SoA coordinates
// (g_mttkrp_seg_pack_kernel, generic.cu:271-343): for each row segment of a
// mode's view, acc_r = sum_e v_e prod_{m != mode} F_m[c_m(e), r], stored
// when the segment is its row's only one, else added atomically.  The view
// is the driver's own kernel view (dense-covered elements dropped, rows
// sorted over the other modes, smallest dimension first), so its element
// layout is free: each element's other coordinates are packed into one
// 32- or 64-bit key in level order (level 0 in the top bits), which
//   * halves the bytes streamed per element (key + value instead of N - 1
//     coordinate words + value) and makes them one load each;
//   * turns "which levels changed" into one XOR and a few shifts.
//
// Work split: one workgroup (4 waves) per segment; a lane owns 2 ranks, so
// LPE = RT / 2 lanes evaluate one element and a wave carries EPW = 64 / LPE
// element slots, each walking a contiguous chunk of the segment.  Keys and
// values arrive in windows of WIN elements per slot: every lane loads
// WIN / LPE of them (consecutive per slot), the next window is prefetched
// into registers while the current one is consumed from LDS, where each
// slot's lanes read the same word (a broadcast).  Within a window, batches
// of U elements first issue all their gathers (the last level's row, and
// the deepest run level's row for every element that closes a run), then
// fold them in order; shallower levels, whose runs are long, load their row
// when the run closes.
//
// The sum is evaluated as a tree over equal coordinate prefixes (the CSF
// form): t[l] is the open partial sum under the prefix o_0..o_l; when o_k
// changes the levels k..NL-1 close (t[l] * F_l[o_l] moves one level up).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "../host/hip_util.hpp"

namespace {

constexpr int WAVE = 64;
constexpr int WAVES = 4;
constexpr int WIN = 16;
constexpr int MAXM = CPTC_MAX_MODES;

struct KeyLevels
{
    const double* F[MAXM];  // factor of each level, level order; F[NO-1] = last level
    uint32_t shift[MAXM];   // bit offset of each level in the key
    uint64_t mask[MAXM];    // field mask of each level (after the shift)
};

__device__ __forceinline__ void wave_sync()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The two ranks r, r + 1 of row idx.  OFF32: the element offset idx R + r
// fits 28 bits for every level (launch_rt checks it before choosing either
// OFF32 kernel, the leaf-in-LDS one included), so it is formed in 32-bit
// arithmetic from the wave-uniform factor base.
template <bool OFF32>
__device__ __forceinline__ double2 row2(const double* __restrict__ base, uint32_t idx, int R, int r)
{
    if constexpr (OFF32)
        return *reinterpret_cast<const double2*>(base + (idx * uint32_t(R) + uint32_t(r)));
    else
        return *reinterpret_cast<const double2*>(base + uint64_t(idx) * uint64_t(R) + r);
}

// One row segment (one workgroup).  LEAF_LDS: the last level's factor is
// read from fleaf (LDS) instead of global memory.
template <int NO, int RT, typename KEY, int U, bool OFF32, bool LEAF_LDS>
__device__ __forceinline__ void seg_keys_segment(
    const KeyLevels& lv, const KEY* __restrict__ keys, const double* __restrict__ vals,
    const uint32_t* __restrict__ seg_row, const uint32_t* __restrict__ seg_start,
    const uint32_t* __restrict__ seg_cnt, const uint8_t* __restrict__ single,
    double* __restrict__ FtV, int R, uint32_t seg, const double* __restrict__ fleaf)
{
    constexpr int VEC = 2;
    constexpr int LPE = RT / VEC;            // lanes per element
    constexpr int EPW = WAVE / LPE;          // element slots per wave
    constexpr int SLOTS = EPW * WAVES;
    constexpr int K = WIN / LPE;             // window elements each lane loads
    constexpr int NL = (NO > 1) ? NO - 1 : 1; // run levels 0 .. NO-2
    static_assert(K >= 1 && WIN % LPE == 0, "window must cover the slot's lanes");

    __shared__ KEY lkey[WAVES][EPW][WIN];
    __shared__ double lval[WAVES][EPW][WIN];
    __shared__ double red[WAVES][RT];

    const uint32_t row = seg_row[seg];
    const uint32_t start = seg_start[seg];
    const uint32_t cnt = seg_cnt[seg];

    const int tid = threadIdx.x;
    const int lane = tid & (WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / WAVE);   // uniform per wave
    const int slot = lane / LPE;
    const int j = lane % LPE;
    const int r0 = j * VEC;
    const bool rank_ok = r0 < R;
    const int rr = rank_ok ? r0 : 0;

    const uint32_t g = uint32_t(wave * EPW + slot);
    const uint32_t chunk = (cnt + SLOTS - 1) / SLOTS;
    uint32_t lo = start + g * chunk;
    const uint32_t hi = (g * chunk + chunk < cnt) ? lo + chunk : start + cnt;
    if (lo > hi) lo = hi;
    const uint32_t nwin = (chunk + WIN - 1) / WIN;   // same for every lane of the block

    const double* __restrict__ Fleaf = lv.F[NO - 1];
    const uint32_t sh_leaf = lv.shift[NO - 1];
    const KEY mk_leaf = KEY(lv.mask[NO - 1]);
    // field of level l (in the key's own width: 32-bit operations for u32 keys)
    auto level = [&](KEY k, int l) -> uint32_t { return uint32_t((k >> lv.shift[l]) & KEY(lv.mask[l])); };
    // a change above the last level closes at least the deepest run level
    const uint32_t sh_deep = lv.shift[NO > 1 ? NO - 2 : 0];

    double acc0 = 0.0, acc1 = 0.0;
    double t0[NL], t1[NL];
#pragma unroll
    for (int l = 0; l < NL; ++l) t0[l] = t1[l] = 0.0;
    KEY cur = 0;
    bool open = false;

    // close run levels NL-1 .. `to`; the deepest level's row is given
    auto close_from = [&](int to, const double2 fdeep) {
#pragma unroll
        for (int l = NL - 1; l >= 0; --l)
        {
            if (l < to) break;
            const double2 f = (l == NL - 1) ? fdeep : row2<OFF32>(lv.F[l], level(cur, l), R, rr);
            const double x0 = t0[l] * f.x, x1 = t1[l] * f.y;
            if (l == 0)
            {
                acc0 += x0;
                acc1 += x1;
            }
            else
            {
                t0[l - 1] += x0;
                t1[l - 1] += x1;
            }
            t0[l] = t1[l] = 0.0;
        }
    };

    KEY nk[K];
    double nv[K];
    auto fetch = [&](uint32_t w) {
#pragma unroll
        for (int k = 0; k < K; ++k)
        {
            const uint32_t e = lo + w * WIN + uint32_t(j + k * LPE);
            const bool ok = e < hi;
            nk[k] = ok ? __builtin_nontemporal_load(keys + e) : KEY(0);
            nv[k] = ok ? __builtin_nontemporal_load(vals + e) : 0.0;
        }
    };
    fetch(0);

    for (uint32_t w = 0; w < nwin; ++w)
    {
        wave_sync();   // the previous window has been read
#pragma unroll
        for (int k = 0; k < K; ++k)
        {
            lkey[wave][slot][j + k * LPE] = nk[k];
            lval[wave][slot][j + k * LPE] = nv[k];
        }
        wave_sync();
        if (w + 1 < nwin) fetch(w + 1);
        const uint32_t base = lo + w * WIN;
        const int nvalid = (base < hi) ? int(hi - base < uint32_t(WIN) ? hi - base : WIN) : 0;

#pragma unroll
        for (int i0 = 0; i0 < WIN; i0 += U)
        {
            if (i0 >= nvalid) break;
            KEY kk[U];
            double vv[U];
            double2 gl[U], cl[U];
#pragma unroll
            for (int u = 0; u < U; ++u)
            {
                const bool live = i0 + u < nvalid;
                kk[u] = live ? lkey[wave][slot][i0 + u] : KEY(0);
                vv[u] = live ? lval[wave][slot][i0 + u] : 0.0;
            }
#pragma unroll
            for (int u = 0; u < U; ++u)
            {
                gl[u] = make_double2(0.0, 0.0);
                if (i0 + u < nvalid)
                {
                    const uint32_t li = uint32_t((kk[u] >> sh_leaf) & mk_leaf);
                    if constexpr (LEAF_LDS)
                        gl[u] = *reinterpret_cast<const double2*>(
                            fleaf + (li * uint32_t(R) + uint32_t(rr)));
                    else
                        gl[u] = row2<OFF32>(Fleaf, li, R, rr);
                }
            }
            if constexpr (NO > 1)
            {
#pragma unroll
                for (int u = 0; u < U; ++u)
                {
                    cl[u] = make_double2(0.0, 0.0);
                    const KEY prev = (u == 0) ? cur : kk[u - 1];
                    const bool has_prev = (u == 0) ? open : true;
                    if (i0 + u < nvalid && has_prev && ((kk[u] ^ prev) >> sh_deep) != 0)
                        cl[u] = row2<OFF32>(lv.F[NL - 1], level(prev, NL - 1), R, rr);
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u)
            {
                if (i0 + u >= nvalid) break;
                if constexpr (NO == 1)
                {
                    acc0 += vv[u] * gl[u].x;
                    acc1 += vv[u] * gl[u].y;
                }
                else
                {
                    if (!open)
                    {
                        open = true;
                        cur = kk[u];
                    }
                    else
                    {
                        const KEY d = kk[u] ^ cur;
                        if ((d >> sh_deep) != 0)
                        {
                            int L = NL - 1;
#pragma unroll
                            for (int l = NL - 2; l >= 0; --l)
                                if ((d >> lv.shift[l]) != 0) L = l;
                            close_from(L, cl[u]);
                            cur = kk[u];
                        }
                    }
                    t0[NL - 1] += vv[u] * gl[u].x;
                    t1[NL - 1] += vv[u] * gl[u].y;
                }
            }
        }
    }
    if constexpr (NO > 1)
        if (open) close_from(0, row2<OFF32>(lv.F[NL - 1], level(cur, NL - 1), R, rr));
    if (!rank_ok) acc0 = acc1 = 0.0;

#pragma unroll
    for (int off = LPE; off < WAVE; off <<= 1)
    {
        acc0 += __shfl_xor(acc0, off, WAVE);
        acc1 += __shfl_xor(acc1, off, WAVE);
    }
    if (slot == 0 && rank_ok)
    {
        red[wave][r0] = acc0;
        red[wave][r0 + 1] = acc1;
    }
    __syncthreads();
    const bool store = single && single[seg] != 0;
    for (int x = tid; x < R; x += WAVE * WAVES)
    {
        double tot = 0.0;
#pragma unroll
        for (int q = 0; q < WAVES; ++q) tot += red[q][x];
        double* out = FtV + size_t(row) * R + x;
        if (store)
            *out = tot;
        else if (tot != 0.0)
            atomicAdd(out, tot);
    }
}

// One workgroup per segment, leaf factor from global memory.
template <int NO, int RT, typename KEY, int U, bool OFF32>
__global__ __launch_bounds__(256) void seg_keys_kernel(
    KeyLevels lv, const KEY* __restrict__ keys, const double* __restrict__ vals,
    const uint32_t* __restrict__ seg_row, const uint32_t* __restrict__ seg_start,
    const uint32_t* __restrict__ seg_cnt, const uint8_t* __restrict__ single,
    double* __restrict__ FtV, int R)
{
    seg_keys_segment<NO, RT, KEY, U, OFF32, false>(lv, keys, vals, seg_row, seg_start, seg_cnt,
                                                   single, FtV, R, blockIdx.x, nullptr);
}

// Persistent grid (workgroup b takes segments b, b + grid, ...): the last
// level's factor (leaf_n doubles) is copied into LDS once per workgroup, so
// the per-element row gathers read LDS instead of the L1 / texture path.
template <int NO, int RT, typename KEY, int U>
__global__ __launch_bounds__(256) void seg_keys_leaf_lds_kernel(
    KeyLevels lv, const KEY* __restrict__ keys, const double* __restrict__ vals,
    const uint32_t* __restrict__ seg_row, const uint32_t* __restrict__ seg_start,
    const uint32_t* __restrict__ seg_cnt, const uint8_t* __restrict__ single,
    double* __restrict__ FtV, int R, uint32_t nseg, uint32_t leaf_n)
{
    extern __shared__ double fleaf[];
    const double* __restrict__ src = lv.F[NO - 1];
    for (uint32_t x = threadIdx.x; x < leaf_n; x += blockDim.x) fleaf[x] = src[x];
    __syncthreads();
    for (uint32_t seg = blockIdx.x; seg < nseg; seg += gridDim.x)
    {
        seg_keys_segment<NO, RT, KEY, U, true, true>(lv, keys, vals, seg_row, seg_start, seg_cnt,
                                                     single, FtV, R, seg, fleaf);
        __syncthreads();   // lkey / lval / red are reused by the next segment
    }
}

// Leaf-in-LDS plan: the leaf factor takes at most LEAF_LDS_MAX bytes, so
// that five workgroups (the register-limited occupancy) still share a CU's
// LDS; the grid is LEAF_LDS_WG_PER_CU workgroups per CU, used when there
// are at least LEAF_LDS_MIN_SEGS segments per workgroup to amortise the copy,
// every level's row offsets fit 32 bits, and five workgroups' leaf plus
// static LDS fit a CU (launch_rt checks the last two).
constexpr size_t LEAF_LDS_MAX = 24 * 1024;
constexpr size_t CU_LDS_BYTES = 160 * 1024;   // LDS per CU on gfx950
constexpr unsigned LEAF_LDS_WG_PER_CU = 5;
constexpr uint64_t LEAF_LDS_MIN_SEGS = 4;

struct LeafPlan
{
    unsigned grid = 0;      // 0: global-memory kernel
    uint32_t n = 0;         // leaf factor size in doubles
};

template <int NO, int RT, typename KEY>
void launch_rt(const KeyLevels& lv, const void* keys, const double* vals, const uint32_t* row,
               const uint32_t* st, const uint32_t* cn, const uint8_t* single, uint64_t nseg,
               double* FtV, int R, const LeafPlan& lp, hipStream_t s)
{
    constexpr int U = (NO <= 2) ? 8 : 4;
    // 32-bit row offsets when every level's (field range x R) stays below 2^28
    bool off32 = true;
    for (int l = 0; l < NO; ++l)
        if ((lv.mask[l] + 1) * uint64_t(R) >= (uint64_t(1) << 28)) off32 = false;
    // the leaf-in-LDS kernel reads its non-leaf rows with 32-bit offsets, and
    // LEAF_LDS_WG_PER_CU of its workgroups (leaf + static LDS) must share a CU
    if (lp.grid > 0 && off32)
    {
        static const size_t static_lds = [] {
            hipFuncAttributes a{};
            const void* k = reinterpret_cast<const void*>(seg_keys_leaf_lds_kernel<NO, RT, KEY, U>);
            return hipFuncGetAttributes(&a, k) == hipSuccess ? size_t(a.sharedSizeBytes)
                                                              : CU_LDS_BYTES;
        }();
        if (LEAF_LDS_WG_PER_CU * (static_lds + size_t(lp.n) * sizeof(double)) <= CU_LDS_BYTES)
        {
            hipLaunchKernelGGL((seg_keys_leaf_lds_kernel<NO, RT, KEY, U>), dim3(lp.grid),
                               dim3(256), size_t(lp.n) * sizeof(double), s, lv,
                               static_cast<const KEY*>(keys), vals, row, st, cn, single, FtV, R,
                               uint32_t(nseg), lp.n);
            return;
        }
    }
    if (off32)
        hipLaunchKernelGGL((seg_keys_kernel<NO, RT, KEY, U, true>), dim3(unsigned(nseg)),
                           dim3(256), 0, s, lv, static_cast<const KEY*>(keys), vals, row, st, cn,
                           single, FtV, R);
    else
        hipLaunchKernelGGL((seg_keys_kernel<NO, RT, KEY, U, false>), dim3(unsigned(nseg)),
                           dim3(256), 0, s, lv, static_cast<const KEY*>(keys), vals, row, st, cn,
                           single, FtV, R);
}

template <int NO, typename KEY>
void launch_r(const KeyLevels& lv, const void* keys, const double* vals, const uint32_t* row,
              const uint32_t* st, const uint32_t* cn, const uint8_t* single, uint64_t nseg,
              double* FtV, int R, const LeafPlan& lp, hipStream_t s)
{
    if (R <= 8)
        launch_rt<NO, 8, KEY>(lv, keys, vals, row, st, cn, single, nseg, FtV, R, lp, s);
    else if (R <= 16)
        launch_rt<NO, 16, KEY>(lv, keys, vals, row, st, cn, single, nseg, FtV, R, lp, s);
    else
        launch_rt<NO, 32, KEY>(lv, keys, vals, row, st, cn, single, nseg, FtV, R, lp, s);
}

template <typename KEY>
void launch_n(int NO, const KeyLevels& lv, const void* keys, const double* vals,
              const uint32_t* row, const uint32_t* st, const uint32_t* cn, const uint8_t* single,
              uint64_t nseg, double* FtV, int R, const LeafPlan& lp, hipStream_t s)
{
    switch (NO)
    {
    case 1: launch_r<1, KEY>(lv, keys, vals, row, st, cn, single, nseg, FtV, R, lp, s); break;
    case 2: launch_r<2, KEY>(lv, keys, vals, row, st, cn, single, nseg, FtV, R, lp, s); break;
    case 3: launch_r<3, KEY>(lv, keys, vals, row, st, cn, single, nseg, FtV, R, lp, s); break;
    case 4: launch_r<4, KEY>(lv, keys, vals, row, st, cn, single, nseg, FtV, R, lp, s); break;
    case 5: launch_r<5, KEY>(lv, keys, vals, row, st, cn, single, nseg, FtV, R, lp, s); break;
    case 6: launch_r<6, KEY>(lv, keys, vals, row, st, cn, single, nseg, FtV, R, lp, s); break;
    default: launch_r<7, KEY>(lv, keys, vals, row, st, cn, single, nseg, FtV, R, lp, s); break;
    }
}

template <typename KEY>
__global__ void pack_keys_kernel(const uint32_t* __restrict__ sc, uint64_t nnz, int nlev,
                                 KeyLevels lv, KEY* __restrict__ out)
{
    const uint64_t stride = uint64_t(gridDim.x) * blockDim.x;
    for (uint64_t e = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; e < nnz; e += stride)
    {
        uint64_t k = 0;
        for (int q = 0; q < nlev; ++q) k |= uint64_t(sc[uint64_t(q) * nnz + e]) << lv.shift[q];
        out[e] = KEY(k);
    }
}

// shifts / masks from the field widths; total bits into *total
bool make_levels(int nlev, const int* bits, KeyLevels& lv, int* total)
{
    int sum = 0;
    for (int q = 0; q < nlev; ++q)
    {
        if (bits[q] < 1 || bits[q] > 32) return false;
        sum += bits[q];
    }
    if (sum > 64) return false;
    int off = sum;
    for (int q = 0; q < nlev; ++q)
    {
        off -= bits[q];
        lv.shift[q] = uint32_t(off);
        lv.mask[q] = (bits[q] >= 64) ? ~uint64_t(0) : ((uint64_t(1) << bits[q]) - 1);
    }
    *total = sum;
    return true;
}

}  // namespace

extern "C" int cptc_level_key_bytes(int nlev, const int* level_bits)
{
    if (nlev < 1 || nlev > MAXM - 1 || !level_bits) return 0;
    KeyLevels lv{};
    int total = 0;
    if (!make_levels(nlev, level_bits, lv, &total)) return 0;
    return total <= 32 ? 4 : 8;
}

extern "C" int cptc_pack_level_keys(int nlev, const uint32_t* d_scoords, uint64_t nnz,
                                    const int* level_bits, void* d_keys, int key_bytes,
                                    void* stream)
{
    CPTC_REQUIRE(nlev >= 1 && nlev <= MAXM - 1 && level_bits, CPTC_ERR_ARG,
                 "cptc_pack_level_keys: %d levels", nlev);
    KeyLevels lv{};
    int total = 0;
    CPTC_REQUIRE(make_levels(nlev, level_bits, lv, &total), CPTC_ERR_ARG,
                 "cptc_pack_level_keys: level widths must be 1..32 bits and sum to <= 64");
    CPTC_REQUIRE((key_bytes == 4 && total <= 32) || key_bytes == 8, CPTC_ERR_ARG,
                 "cptc_pack_level_keys: %d-byte keys for %d bits", key_bytes, total);
    if (nnz == 0) return CPTC_OK;
    CPTC_REQUIRE(d_scoords && d_keys, CPTC_ERR_ARG, "cptc_pack_level_keys: null pointer");
    hipStream_t s = cptc::as_stream(stream);
    const unsigned g = cptc::grid_for(nnz, 256, 8192);
    if (key_bytes == 4)
        hipLaunchKernelGGL(pack_keys_kernel<uint32_t>, dim3(g), dim3(256), 0, s, d_scoords, nnz,
                           nlev, lv, static_cast<uint32_t*>(d_keys));
    else
        hipLaunchKernelGGL(pack_keys_kernel<uint64_t>, dim3(g), dim3(256), 0, s, d_scoords, nnz,
                           nlev, lv, static_cast<uint64_t*>(d_keys));
    CPTC_LAUNCHED();
    return CPTC_OK;
}

extern "C" int cptc_mttkrp_seg_nd_keys(int nmodes, int mode, const void* d_keys, int key_bytes,
                                       const int* level_modes, const int* level_bits,
                                       const double* d_vals, uint64_t nnz,
                                       const uint32_t* d_seg_row, const uint32_t* d_seg_start,
                                       const uint32_t* d_seg_cnt, const uint8_t* d_single,
                                       uint64_t nseg, const double* const* h_F, double* d_FtV,
                                       int R, void* stream)
{
    return cptc_mttkrp_seg_nd_keys_dims(nmodes, mode, d_keys, key_bytes, level_modes, level_bits,
                                        d_vals, nnz, d_seg_row, d_seg_start, d_seg_cnt, d_single,
                                        nseg, h_F, nullptr, d_FtV, R, stream);
}

extern "C" int cptc_mttkrp_seg_nd_keys_dims(int nmodes, int mode, const void* d_keys,
                                            int key_bytes, const int* level_modes,
                                            const int* level_bits, const double* d_vals,
                                            uint64_t nnz, const uint32_t* d_seg_row,
                                            const uint32_t* d_seg_start,
                                            const uint32_t* d_seg_cnt, const uint8_t* d_single,
                                            uint64_t nseg, const double* const* h_F,
                                            const uint64_t* h_dims, double* d_FtV, int R,
                                            void* stream)
{
    CPTC_REQUIRE(nmodes >= 2 && nmodes <= MAXM && mode >= 0 && mode < nmodes, CPTC_ERR_ARG,
                 "cptc_mttkrp_seg_nd_keys: nmodes %d mode %d", nmodes, mode);
    CPTC_REQUIRE(R >= 2 && R <= 32 && R % 2 == 0, CPTC_ERR_ARG,
                 "cptc_mttkrp_seg_nd_keys: R %d (even, 2..32)", R);
    CPTC_REQUIRE(key_bytes == 4 || key_bytes == 8, CPTC_ERR_ARG,
                 "cptc_mttkrp_seg_nd_keys: key_bytes %d", key_bytes);
    if (nseg == 0) return CPTC_OK;
    CPTC_REQUIRE(nseg < (uint64_t(1) << 31) && nnz <= 0x7FFFFFFFull, CPTC_ERR_ARG,
                 "cptc_mttkrp_seg_nd_keys: %llu segments / %llu nnz", (unsigned long long)nseg,
                 (unsigned long long)nnz);
    CPTC_REQUIRE(d_keys && d_vals && d_seg_row && d_seg_start && d_seg_cnt && d_FtV && h_F &&
                     level_modes && level_bits,
                 CPTC_ERR_ARG, "cptc_mttkrp_seg_nd_keys: null pointer");
    const int nlev = nmodes - 1;
    KeyLevels lv{};
    int total = 0;
    CPTC_REQUIRE(make_levels(nlev, level_bits, lv, &total), CPTC_ERR_ARG,
                 "cptc_mttkrp_seg_nd_keys: level widths must be 1..32 bits and sum to <= 64");
    CPTC_REQUIRE(key_bytes == 8 || total <= 32, CPTC_ERR_ARG,
                 "cptc_mttkrp_seg_nd_keys: %d key bits in 4-byte keys", total);
    unsigned seen = 1u << mode;
    for (int q = 0; q < nlev; ++q)
    {
        const int m = level_modes[q];
        CPTC_REQUIRE(m >= 0 && m < nmodes && !(seen & (1u << m)) && h_F[m], CPTC_ERR_ARG,
                     "cptc_mttkrp_seg_nd_keys: level_modes is not a permutation of the other "
                     "modes, or a factor is null");
        seen |= 1u << m;
        CPTC_REQUIRE((reinterpret_cast<uintptr_t>(h_F[m]) & 15) == 0, CPTC_ERR_ARG,
                     "cptc_mttkrp_seg_nd_keys: factor %d is not 16-byte aligned", m);
        lv.F[q] = h_F[m];
    }
    hipStream_t s = cptc::as_stream(stream);
    // the last level's factor in LDS when its size is known and small
    LeafPlan lp;
    if (h_dims)
    {
        const uint64_t rows = h_dims[level_modes[nlev - 1]];
        const uint64_t bytes = rows * uint64_t(R) * sizeof(double);
        // the key field bounds every leaf coordinate by its width, the dims by rows
        if (rows >= 1 && rows <= lv.mask[nlev - 1] + 1 && bytes <= LEAF_LDS_MAX)
        {
            int dev = 0;
            CPTC_HIP(hipGetDevice(&dev));
            const int cus = cptc::cu_count(dev);
            const uint64_t grid = uint64_t(LEAF_LDS_WG_PER_CU) * uint64_t(cus);
            if (nseg >= LEAF_LDS_MIN_SEGS * grid)
            {
                lp.grid = unsigned(grid);
                lp.n = uint32_t(rows * uint64_t(R));
            }
        }
    }
    if (key_bytes == 4)
        launch_n<uint32_t>(nlev, lv, d_keys, d_vals, d_seg_row, d_seg_start, d_seg_cnt, d_single,
                           nseg, d_FtV, R, lp, s);
    else
        launch_n<uint64_t>(nlev, lv, d_keys, d_vals, d_seg_row, d_seg_start, d_seg_cnt, d_single,
                           nseg, d_FtV, R, lp, s);
    CPTC_LAUNCHED();
    return CPTC_OK;
}
