// Host-side helpers shared by the generators, the loader and the drivers.
#pragma once

#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <vector>

#include <omp.h>

namespace cptc {

inline uint64_t mix64(uint64_t z)
{
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Counter-based stream: independent 64-bit words for any (seed, stream, ctr).
inline uint64_t rng_u64(uint64_t seed, uint64_t stream, uint64_t ctr)
{
    return mix64(mix64(seed ^ (stream * 0xD1B54A32D192ED03ull)) + ctr);
}

// [0, 1) with 53 random bits.
inline double u01(uint64_t x) { return double(x >> 11) * (1.0 / 9007199254740992.0); }

// Stable LSD radix sort of (key, payload) pairs on the low `key_bits` bits,
// 11 bits per pass, OpenMP-parallel with per-thread histograms.
template <class V>
void radix_sort_pairs_u64(std::vector<uint64_t>& keys, std::vector<V>& vals, int key_bits)
{
    const size_t n = keys.size();
    if (n < 2 || key_bits <= 0) return;
    constexpr int DB = 11;
    constexpr int NB = 1 << DB;
    std::vector<uint64_t> k2(n);
    std::vector<V> v2(n);
    const int nt = std::max(1, omp_get_max_threads());
    std::vector<size_t> hist(size_t(nt) * NB);
    for (int shift = 0; shift < key_bits; shift += DB)
    {
        std::fill(hist.begin(), hist.end(), 0);
        #pragma omp parallel num_threads(nt)
        {
            const int t = omp_get_thread_num();
            const size_t lo = n * t / nt, hi = n * (t + 1) / nt;
            size_t* h = &hist[size_t(t) * NB];
            for (size_t i = lo; i < hi; ++i) ++h[(keys[i] >> shift) & (NB - 1)];
        }
        size_t run = 0;
        for (int d = 0; d < NB; ++d)
            for (int t = 0; t < nt; ++t)
            {
                const size_t c = hist[size_t(t) * NB + d];
                hist[size_t(t) * NB + d] = run;
                run += c;
            }
        #pragma omp parallel num_threads(nt)
        {
            const int t = omp_get_thread_num();
            const size_t lo = n * t / nt, hi = n * (t + 1) / nt;
            size_t* h = &hist[size_t(t) * NB];
            for (size_t i = lo; i < hi; ++i)
            {
                const size_t p = h[(keys[i] >> shift) & (NB - 1)]++;
                k2[p] = keys[i];
                v2[p] = vals[i];
            }
        }
        keys.swap(k2);
        vals.swap(v2);
    }
}

// Group cap for the grouped MFMA tile / unit launches: a group of up to
// `cap` tiles with one target row block is one wave, which sums the group in
// LDS and issues one atomic per (row, rank) per group.  Large groups save
// atomics; enough groups keep the SIMDs busy: the cap is the number of
// tile x rank-block items per SIMD (16-rank blocks for the FP32 kernel,
// 32-rank blocks for the split-bf16 one), clamped to [1, cap].  Measured: config
// 4 (3847 units, R = 16) 0.518 -> 0.406 ms per iteration at 4 instead of 16;
// config 5 (32768 units) slows at anything below 16 (atomic contention on
// 64-row targets).  CPTC_TILE_GROUP=<n> fixes it (tuning).
// Smallest tile (unit) x 32-rank-block count for which the drivers take the
// split-bf16 tile kernel: config 5's 32 768 units at R = 32 gain, and since
// the order-3 update runs in one launch, config 1's 4096 tiles at R = 32 do
// too (0.167-0.169 -> 0.163 ms per iteration; before it, its extra
// operand-image launch cost more than the kernel saved).
constexpr size_t TILE_B3_MIN_ITEMS = 4096;

// Tile kernel choice from a switch (ALS_TILE_KERNEL / GEN_TILE_KERNEL):
// "fp32" -> 0, "bf16x3" -> 1, unset or anything else -> -1 (automatic).
inline int tile_kernel_switch(const char* name)
{
    const char* e = std::getenv(name);
    if (!e) return -1;
    if (std::strcmp(e, "fp32") == 0) return 0;
    if (std::strcmp(e, "bf16x3") == 0) return 1;
    return -1;
}

// The automatic choice: the split-bf16 kernel for R > 16 and at least
// TILE_B3_MIN_ITEMS tile x 32-rank-block items.
inline bool tile_b3_auto(size_t ntiles, int R)
{
    return R > 16 && ntiles * size_t((R + 31) / 32) >= TILE_B3_MIN_ITEMS;
}

// The merged grid's experiment switches (dense.cu:2277-2283, 2350-2352):
// ALS_MERGED_STRIDE=<k> makes every k-th workgroup a tile workgroup (unset or
// <= 0: spread evenly); ALS_MERGED_NO_DENSE / ALS_MERGED_NO_SPARSE, on when
// set (the reference tests getenv != nullptr), leave the tiles / the
// residual segments out -> flags bits 0 / 1 of cptc_mttkrp_merged3_ex.
inline void merged_switches(int& every, int& flags)
{
    const char* s = std::getenv("ALS_MERGED_STRIDE");
    every = s ? std::atoi(s) : 0;
    flags = (std::getenv("ALS_MERGED_NO_DENSE") ? 1 : 0) |
            (std::getenv("ALS_MERGED_NO_SPARSE") ? 2 : 0);
}

inline int tile_group_cap(size_t ntiles, int R, int num_cus, int cap, int rank_block = 16)
{
    if (const char* e = std::getenv("CPTC_TILE_GROUP"))
    {
        const int g = std::atoi(e);
        if (g >= 1) return g;
    }
    const size_t simds = size_t(num_cus > 0 ? num_cus : 256) * 4;
    const size_t items = ntiles * size_t((R + rank_block - 1) / rank_block);
    const size_t g = (items + simds - 1) / simds;
    return int(std::max<size_t>(1, std::min<size_t>(g, size_t(cap))));
}

}  // namespace cptc
