// Deterministic synthetic tensors for the five benchmark configurations.
//
// Every random draw is a pure function of (seed, stream, counter): a
// SplitMix64-style finaliser over a counter, so generation parallelises over
// OpenMP threads and gives identical bytes for any thread count.  Indices are
// 0-based, stored mode-major (idx[m * nnz + e]).
//
// Decisions fixed here (the configuration text leaves them open):
//   * N(0, 0.01) noise means variance 0.01 (sigma = 0.1).
//   * Zipf(s) is bounded to the mode length D: P(n) ~ n^-s, n = 1..D, and the
//     rank n maps to index perm[n-1] of a seeded permutation of [0, D).
//   * "De-duplicate" keeps the first occurrence of each coordinate in draw
//     order and draws until exactly `nnz` distinct coordinates exist (the
//     first `nnz` distinct coordinates of the draw sequence); a value is a
//     function of its coordinate's first draw index.  Elements are emitted in
//     a fixed pseudo-random order (hash clusters in slot order, keys sorted
//     inside a cluster); no duplicates exist, so the layout built from the
//     tensor does not depend on this order.
//   * Config-2 blocks sit on the 16^3 tile grid at distinct tile positions;
//     background cells inside a block are not drawn again.
//   * Config-5 units sit on the 16^3 grid of modes 0-2 at distinct (tile,
//     outer tuple) slots; the uniform background is drawn until the total
//     reaches 20,000,000 distinct coordinates.
#include "cptc_hip.h"
#include "host_util.hpp"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <numeric>
#include <vector>

#include <omp.h>
#include <sys/mman.h>

namespace {

using cptc::mix64;
using cptc::rng_u64;
using cptc::u01;

double normal01(uint64_t seed, uint64_t stream, uint64_t ctr)
{
    // Box-Muller on two independent uniforms; u1 in (0, 1].
    const double u1 = 1.0 - u01(rng_u64(seed, stream, 2 * ctr));
    const double u2 = u01(rng_u64(seed, stream, 2 * ctr + 1));
    return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
}

int poisson(double lam, uint64_t x)
{
    // Inversion by sequential search (small lambda).
    const double u = u01(x);
    double p = std::exp(-lam), c = p;
    int k = 0;
    while (u >= c && k < 1000)
    {
        ++k;
        p *= lam / k;
        c += p;
    }
    return k;
}

// Vose alias table for a bounded Zipf law over ranks 1..D.
struct Alias
{
    std::vector<double> prob;
    std::vector<uint32_t> alias;
    uint32_t D = 0;

    void build_zipf(uint32_t d, double s)
    {
        D = d;
        std::vector<double> w(d);
        double tot = 0.0;
        for (uint32_t n = 0; n < d; ++n)
        {
            w[n] = (s == 0.0) ? 1.0 : std::pow(double(n + 1), -s);
            tot += w[n];
        }
        prob.assign(d, 0.0);
        alias.assign(d, 0);
        std::vector<double> q(d);
        std::vector<uint32_t> small, large;
        for (uint32_t n = 0; n < d; ++n)
        {
            q[n] = w[n] * d / tot;
            (q[n] < 1.0 ? small : large).push_back(n);
        }
        while (!small.empty() && !large.empty())
        {
            const uint32_t l = small.back(); small.pop_back();
            const uint32_t g = large.back(); large.pop_back();
            prob[l] = q[l];
            alias[l] = g;
            q[g] = (q[g] + q[l]) - 1.0;
            (q[g] < 1.0 ? small : large).push_back(g);
        }
        for (uint32_t g : large) { prob[g] = 1.0; alias[g] = g; }
        for (uint32_t l : small) { prob[l] = 1.0; alias[l] = l; }
    }

    // rank in [0, D)
    uint32_t sample(uint64_t x) const
    {
        const uint32_t col = uint32_t(((x >> 32) * uint64_t(D)) >> 32);
        const double f = double(uint32_t(x)) * (1.0 / 4294967296.0);
        return f < prob[col] ? col : alias[col];
    }
};

std::vector<uint32_t> seeded_perm(uint32_t d, uint64_t seed, uint64_t stream)
{
    std::vector<uint32_t> p(d);
    std::iota(p.begin(), p.end(), 0u);
    for (uint32_t i = d; i > 1; --i)
    {
        const uint64_t x = rng_u64(seed, stream, i);
        const uint32_t j = uint32_t(((x >> 32) * uint64_t(i)) >> 32);
        std::swap(p[i - 1], p[j]);
    }
    return p;
}

// Packs an N-mode coordinate into a 64-bit key (bits per mode = ceil(log2 dim)).
struct KeyPack
{
    int n = 0;
    int shift[8] = {};
    int bits[8] = {};
    int total = 0;

    bool init(int nmodes, const uint64_t* dims)
    {
        n = nmodes;
        total = 0;
        for (int m = nmodes - 1; m >= 0; --m)
        {
            int b = 1;
            while ((uint64_t(1) << b) < dims[m]) ++b;
            bits[m] = b;
            shift[m] = total;
            total += b;
        }
        return total <= 64;
    }
    uint64_t pack(const uint32_t* c) const
    {
        uint64_t k = 0;
        for (int m = 0; m < n; ++m) k |= uint64_t(c[m]) << shift[m];
        return k;
    }
    uint32_t get(uint64_t k, int m) const
    {
        return uint32_t((k >> shift[m]) & ((uint64_t(1) << bits[m]) - 1));
    }
};

// First-occurrence set of packed coordinates: open addressing (linear
// probing) over 64-bit slots holding key + 1, plus the smallest draw index t
// seen for the key (atomic min).  Insertion is lock-free and its final
// contents do not depend on thread interleaving.
void* big_alloc(size_t bytes)
{
    constexpr size_t HUGE = size_t(2) << 20;
    bytes = (bytes + HUGE - 1) / HUGE * HUGE;
    void* p = std::aligned_alloc(HUGE, bytes);
    if (p) madvise(p, bytes, MADV_HUGEPAGE);
    return p;
}

struct FirstSet
{
    uint64_t* key = nullptr;
    uint64_t* tmin = nullptr;
    uint64_t mask = 0;
    uint64_t count = 0;  // distinct keys (atomic)

    explicit FirstSet(uint64_t expect)
    {
        uint64_t cap = 1;
        while (cap < expect) cap <<= 1;
        mask = cap - 1;
        // 2 MiB-aligned and THP-advised: random probes over GiB-sized tables
        // otherwise miss the TLB on almost every access
        key = static_cast<uint64_t*>(big_alloc(cap * sizeof(uint64_t)));
        tmin = static_cast<uint64_t*>(big_alloc(cap * sizeof(uint64_t)));
        if (key && tmin)
        {
            // parallel first touch
            #pragma omp parallel for schedule(static)
            for (int64_t x = 0; x < int64_t(cap); ++x)
            {
                key[x] = 0;
                tmin[x] = 0;
            }
        }
    }
    ~FirstSet()
    {
        std::free(key);
        std::free(tmin);
    }
    bool ok() const { return key && tmin; }
    uint64_t capacity() const { return mask + 1; }

    void insert(uint64_t k, uint64_t t)
    {
        const uint64_t want = k + 1;
        const uint64_t tv = t + 1;  // tmin slot: 0 = none yet, else first t + 1
        uint64_t h = mix64(k) & mask;
        for (;;)
        {
            uint64_t cur = __atomic_load_n(&key[h], __ATOMIC_ACQUIRE);
            if (cur == 0)
            {
                uint64_t expected = 0;
                if (__atomic_compare_exchange_n(&key[h], &expected, want, false, __ATOMIC_ACQ_REL,
                                                __ATOMIC_ACQUIRE))
                {
                    __atomic_fetch_add(&count, 1, __ATOMIC_RELAXED);
                    cur = want;
                }
                else
                    cur = expected;
            }
            if (cur == want)
            {
                uint64_t old = __atomic_load_n(&tmin[h], __ATOMIC_ACQUIRE);
                while (old == 0 || old > tv)
                    if (__atomic_compare_exchange_n(&tmin[h], &old, tv, false, __ATOMIC_ACQ_REL,
                                                    __ATOMIC_ACQUIRE))
                        return;
                return;
            }
            h = (h + 1) & mask;
        }
    }

    // The `target` distinct keys with the smallest first-draw index t, with
    // their t, in a canonical order: under linear probing the set of occupied
    // slots, and the keys of every maximal occupied run, do not depend on the
    // insertion order; runs are visited in slot order (circularly from the
    // first empty slot) and each run's keys are emitted in key order.
    void extract(uint64_t target, std::vector<uint64_t>& keys, std::vector<uint64_t>& ts) const
    {
        const int nt = std::max(1, omp_get_max_threads());
        const uint64_t cap = mask + 1;
        std::vector<uint64_t> tall;
        tall.reserve(count);
        for (uint64_t h = 0; h < cap; ++h)
            if (key[h]) tall.push_back(tmin[h] - 1);
        uint64_t cut = ~uint64_t(0);  // keep t < cut
        if (tall.size() > target)
        {
            std::nth_element(tall.begin(), tall.begin() + target, tall.end());
            cut = tall[target];
        }
        std::vector<uint64_t>().swap(tall);
        uint64_t e0 = 0;
        while (e0 < cap && key[e0]) ++e0;  // the table is never full
        auto slot = [&](uint64_t x) { return (e0 + x) & mask; };
        // chunk starts on empty slots so no run straddles two chunks
        std::vector<uint64_t> beg(size_t(nt) + 1, cap);
        for (int th = 0; th < nt; ++th)
        {
            uint64_t x = cap * th / nt;
            while (x < cap && key[slot(x)]) ++x;
            beg[th] = x;
        }
        for (int th = nt - 1; th > 0; --th) beg[th] = std::min(beg[th], beg[th + 1]);
        std::vector<uint64_t> cnt(size_t(nt) + 1, 0);
        auto walk = [&](int th, bool emit, uint64_t w) {
            std::vector<std::pair<uint64_t, uint64_t>> run;
            uint64_t c = 0;
            uint64_t x = beg[th];
            while (x < beg[th + 1])
            {
                if (!key[slot(x)])
                {
                    ++x;
                    continue;
                }
                run.clear();
                while (x < cap && key[slot(x)])
                {
                    const uint64_t h = slot(x);
                    if (tmin[h] - 1 < cut) run.emplace_back(key[h] - 1, tmin[h] - 1);
                    ++x;
                }
                if (emit)
                {
                    std::sort(run.begin(), run.end());
                    for (auto& kt : run)
                    {
                        keys[w] = kt.first;
                        ts[w] = kt.second;
                        ++w;
                    }
                }
                c += run.size();
            }
            return c;
        };
        #pragma omp parallel for schedule(static, 1) num_threads(nt)
        for (int th = 0; th < nt; ++th) cnt[th + 1] = walk(th, false, 0);
        for (int th = 0; th < nt; ++th) cnt[th + 1] += cnt[th];
        keys.resize(cnt[nt]);
        ts.resize(cnt[nt]);
        #pragma omp parallel for schedule(static, 1) num_threads(nt)
        for (int th = 0; th < nt; ++th) walk(th, true, cnt[th]);
    }
};

int alloc_coo(cptc_coo* out, int nmodes, const uint64_t* dims, uint64_t nnz)
{
    std::memset(out, 0, sizeof(*out));
    out->nmodes = nmodes;
    for (int m = 0; m < nmodes; ++m) out->dims[m] = dims[m];
    out->nnz = nnz;
    out->idx = static_cast<uint32_t*>(std::malloc(sizeof(uint32_t) * nmodes * (nnz ? nnz : 1)));
    out->val = static_cast<double*>(std::malloc(sizeof(double) * (nnz ? nnz : 1)));
    return (out->idx && out->val) ? 0 : -1;
}

// Draws coordinates with `draw(t, coord)`, t = t0, t0 + 1, ..., until
// `target` distinct coordinates exist (counting those already in `set`);
// returns the first `target` distinct keys of the draw sequence (in the
// canonical order of FirstSet::extract) with the draw index of their first
// occurrence.
template <class Draw>
int draw_distinct(const KeyPack& kp, uint64_t target, uint64_t t0, Draw draw, FirstSet& set,
                  std::vector<uint64_t>& keys, std::vector<uint64_t>& ts)
{
    uint64_t t_next = t0;
    for (int round = 0; round < 256 && set.count < target; ++round)
    {
        const uint64_t missing = target - set.count;
        const uint64_t batch = std::max<uint64_t>(missing + missing / 4, 1u << 14);
        if (set.count + batch > set.capacity() / 10 * 7) return -1;
        #pragma omp parallel for schedule(static)
        for (int64_t b = 0; b < int64_t(batch); ++b)
        {
            uint32_t c[8] = {};
            const uint64_t t = t_next + uint64_t(b);
            draw(t, c);
            set.insert(kp.pack(c), t);
        }
        t_next += batch;
    }
    if (set.count < target) return -1;
    set.extract(target, keys, ts);
    return keys.size() == target ? 0 : -1;
}

}  // namespace

extern "C" void cptc_coo_free(cptc_coo* c)
{
    if (!c) return;
    std::free(c->idx);
    std::free(c->val);
    c->idx = nullptr;
    c->val = nullptr;
    c->nnz = 0;
}

extern "C" int cptc_synth_zipf(int nmodes, const uint64_t* dims, const double* exponents,
                               uint64_t nnz, int value_kind, uint64_t seed, cptc_coo* out)
{
    if (nmodes < 2 || nmodes > CPTC_MAX_MODES || !dims || !exponents || !out) return -1;
    KeyPack kp;
    if (!kp.init(nmodes, dims)) return -2;
    double cells = 1.0;
    for (int m = 0; m < nmodes; ++m) cells *= double(dims[m]);
    if (double(nnz) > 0.5 * cells) return -3;

    std::vector<Alias> al(nmodes);
    std::vector<std::vector<uint32_t>> perm(nmodes);
    for (int m = 0; m < nmodes; ++m)
    {
        al[m].build_zipf(uint32_t(dims[m]), exponents[m]);
        perm[m] = seeded_perm(uint32_t(dims[m]), seed, 100 + m);
    }
    auto draw = [&](uint64_t t, uint32_t* c) {
        for (int m = 0; m < nmodes; ++m)
            c[m] = perm[m][al[m].sample(rng_u64(seed, m, t))];
    };
    std::vector<uint64_t> keys, ts;
    {
        FirstSet set(nnz * 2);
        if (!set.ok()) return -5;
        if (draw_distinct(kp, nnz, 0, draw, set, keys, ts) != 0) return -4;
    }
    if (alloc_coo(out, nmodes, dims, nnz) != 0) return -5;
    #pragma omp parallel for schedule(static)
    for (int64_t e = 0; e < int64_t(nnz); ++e)
    {
        for (int m = 0; m < nmodes; ++m) out->idx[uint64_t(m) * nnz + e] = kp.get(keys[e], m);
        const uint64_t t = ts[e];
        double v;
        if (value_kind == CPTC_VAL_POISSON1P2)
            v = 1.0 + poisson(2.0, rng_u64(seed, 20, t));
        else if (value_kind == CPTC_VAL_NORMAL)
            v = normal01(seed, 21, t);
        else
            v = std::exp(normal01(seed, 22, t));
        out->val[e] = v;
    }
    return 0;
}

extern "C" int cptc_synth_lowrank3(uint64_t n, int rank, double keep_p, double noise_sigma,
                                   uint64_t seed, cptc_coo* out)
{
    if (n == 0 || n > 4096 || rank <= 0 || !out) return -1;
    std::vector<double> f(3 * n * rank);
    for (size_t x = 0; x < f.size(); ++x) f[x] = u01(rng_u64(seed, 30, x));
    const uint64_t cells = n * n * n;
    // count kept cells per i-slab, then fill in lexicographic order
    std::vector<uint64_t> cnt(n + 1, 0);
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < int64_t(n); ++i)
    {
        uint64_t c = 0;
        for (uint64_t jk = 0; jk < n * n; ++jk)
            c += u01(rng_u64(seed, 31, uint64_t(i) * n * n + jk)) < keep_p;
        cnt[i + 1] = c;
    }
    for (uint64_t i = 0; i < n; ++i) cnt[i + 1] += cnt[i];
    const uint64_t dims[3] = {n, n, n};
    if (alloc_coo(out, 3, dims, cnt[n]) != 0) return -5;
    const uint64_t nnz = cnt[n];
    const double* A = f.data();
    const double* B = A + n * rank;
    const double* C = B + n * rank;
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < int64_t(n); ++i)
    {
        uint64_t w = cnt[i];
        for (uint64_t j = 0; j < n; ++j)
            for (uint64_t k = 0; k < n; ++k)
            {
                const uint64_t cell = (uint64_t(i) * n + j) * n + k;
                if (!(u01(rng_u64(seed, 31, cell)) < keep_p)) continue;
                double s = 0.0;
                for (int r = 0; r < rank; ++r)
                    s += A[i * rank + r] * B[j * rank + r] * C[k * rank + r];
                out->idx[w] = uint32_t(i);
                out->idx[nnz + w] = uint32_t(j);
                out->idx[2 * nnz + w] = uint32_t(k);
                out->val[w] = s + noise_sigma * normal01(seed, 32, cell);
                ++w;
            }
    }
    (void)cells;
    return 0;
}

extern "C" int cptc_synth_blocks3(uint64_t n, int nblocks, double fill_lo, double fill_hi,
                                  double bg_density, uint64_t seed, cptc_coo* out)
{
    if (n == 0 || n % 16 || n > 16384 || !out) return -1;
    const uint64_t nb = n / 16, ntiles = nb * nb * nb;
    if (uint64_t(nblocks) > ntiles) return -2;
    // distinct tile positions: partial Fisher-Yates over tile ids
    std::vector<uint64_t> tiles(ntiles);
    std::iota(tiles.begin(), tiles.end(), uint64_t(0));
    for (int b = 0; b < nblocks; ++b)
    {
        const uint64_t x = rng_u64(seed, 40, b);
        const uint64_t j = b + uint64_t(((x >> 32) * (ntiles - b)) >> 32);
        std::swap(tiles[b], tiles[j]);
    }
    std::vector<uint8_t> in_block(ntiles, 0);
    std::vector<double> fill(ntiles, 0.0);
    for (int b = 0; b < nblocks; ++b)
    {
        in_block[tiles[b]] = 1;
        fill[tiles[b]] = fill_lo + (fill_hi - fill_lo) * u01(rng_u64(seed, 41, b));
    }
    // every cell decides independently: block cells keep with the block fill,
    // other cells with bg_density.  Counter = cell index -> deterministic.
    auto keep = [&](uint64_t cell) -> bool {
        const uint64_t k = cell % n, j = (cell / n) % n, i = cell / (n * n);
        const uint64_t t = ((i / 16) * nb + (j / 16)) * nb + (k / 16);
        const double p = in_block[t] ? fill[t] : bg_density;
        return u01(rng_u64(seed, 42, cell)) < p;
    };
    std::vector<uint64_t> cnt(n + 1, 0);
    #pragma omp parallel for schedule(dynamic, 4)
    for (int64_t i = 0; i < int64_t(n); ++i)
    {
        uint64_t c = 0;
        for (uint64_t jk = 0; jk < n * n; ++jk) c += keep(uint64_t(i) * n * n + jk);
        cnt[i + 1] = c;
    }
    for (uint64_t i = 0; i < n; ++i) cnt[i + 1] += cnt[i];
    const uint64_t dims[3] = {n, n, n};
    const uint64_t nnz = cnt[n];
    if (alloc_coo(out, 3, dims, nnz) != 0) return -5;
    #pragma omp parallel for schedule(dynamic, 4)
    for (int64_t i = 0; i < int64_t(n); ++i)
    {
        uint64_t w = cnt[i];
        for (uint64_t jk = 0; jk < n * n; ++jk)
        {
            const uint64_t cell = uint64_t(i) * n * n + jk;
            if (!keep(cell)) continue;
            out->idx[w] = uint32_t(i);
            out->idx[nnz + w] = uint32_t(jk / n);
            out->idx[2 * nnz + w] = uint32_t(jk % n);
            out->val[w] = std::exp(normal01(seed, 43, cell));
            ++w;
        }
    }
    return 0;
}

extern "C" int cptc_synth_units5(const uint64_t* dims, int nunits, double fill_lo, double fill_hi,
                                 uint64_t total_nnz, int signal_rank, uint64_t seed, cptc_coo* out)
{
    if (!dims || !out || nunits < 0) return -1;
    for (int m = 0; m < 3; ++m)
        if (dims[m] % 16) return -1;
    KeyPack kp;
    if (!kp.init(5, dims)) return -2;
    const uint64_t nb0 = dims[0] / 16, nb1 = dims[1] / 16, nb2 = dims[2] / 16;
    const uint64_t slots = nb0 * nb1 * nb2 * dims[3] * dims[4];
    if (uint64_t(nunits) > slots) return -3;
    std::vector<uint64_t> slot(slots);
    std::iota(slot.begin(), slot.end(), uint64_t(0));
    for (int u = 0; u < nunits; ++u)
    {
        const uint64_t x = rng_u64(seed, 50, u);
        const uint64_t j = u + uint64_t(((x >> 32) * (slots - u)) >> 32);
        std::swap(slot[u], slot[j]);
    }
    // unit cells, unit by unit, cell order (a, b, c) inside the unit
    FirstSet set(total_nnz * 2);
    if (!set.ok()) return -5;
    std::vector<uint64_t> keys, ts;
    uint64_t t = 0;
    for (int u = 0; u < nunits; ++u)
    {
        uint64_t s = slot[u];
        const uint64_t o4 = s % dims[4]; s /= dims[4];
        const uint64_t o3 = s % dims[3]; s /= dims[3];
        const uint64_t t2 = s % nb2; s /= nb2;
        const uint64_t t1 = s % nb1; s /= nb1;
        const uint64_t t0 = s;
        const double f = fill_lo + (fill_hi - fill_lo) * u01(rng_u64(seed, 51, u));
        for (uint32_t cell = 0; cell < 4096; ++cell)
        {
            if (!(u01(rng_u64(seed, 52, uint64_t(u) * 4096 + cell)) < f)) continue;
            uint32_t c[5] = {uint32_t(t0 * 16 + (cell >> 8)), uint32_t(t1 * 16 + ((cell >> 4) & 15)),
                             uint32_t(t2 * 16 + (cell & 15)), uint32_t(o3), uint32_t(o4)};
            set.insert(kp.pack(c), t++);
        }
    }
    if (set.count > total_nnz) return -4;
    // uniform background until total_nnz distinct coordinates
    auto draw = [&](uint64_t tt, uint32_t* c) {
        for (int m = 0; m < 5; ++m)
        {
            const uint64_t x = rng_u64(seed, 53 + m, tt);
            c[m] = uint32_t(((x >> 32) * dims[m]) >> 32);
        }
    };
    if (draw_distinct(kp, total_nnz, t, draw, set, keys, ts) != 0) return -5;
    // rank-`signal_rank` CP signal with U(0,1) factors
    std::vector<std::vector<double>> fac(5);
    for (int m = 0; m < 5; ++m)
    {
        fac[m].resize(dims[m] * signal_rank);
        for (size_t x = 0; x < fac[m].size(); ++x) fac[m][x] = u01(rng_u64(seed, 60 + m, x));
    }
    const uint64_t nnz = keys.size();
    if (alloc_coo(out, 5, dims, nnz) != 0) return -6;
    #pragma omp parallel for schedule(static)
    for (int64_t e = 0; e < int64_t(nnz); ++e)
    {
        uint32_t c[5];
        for (int m = 0; m < 5; ++m)
        {
            c[m] = kp.get(keys[e], m);
            out->idx[uint64_t(m) * nnz + e] = c[m];
        }
        double s = 0.0;
        for (int r = 0; r < signal_rank; ++r)
        {
            double p = 1.0;
            for (int m = 0; m < 5; ++m) p *= fac[m][uint64_t(c[m]) * signal_rank + r];
            s += p;
        }
        out->val[e] = s + normal01(seed, 65, ts[e]);
    }
    return 0;
}

extern "C" int cptc_synth_config(int config, uint64_t seed, cptc_coo* out)
{
    switch (config)
    {
        case 1:
            return cptc_synth_lowrank3(256, 8, 0.9, 0.1, seed, out);
        case 2:
            return cptc_synth_blocks3(512, 2000, 0.1, 0.6, 2e-4, seed, out);
        case 3:
        {
            const uint64_t d[3] = {12092, 9184, 28818};
            const double s[3] = {1.1, 1.1, 1.1};
            return cptc_synth_zipf(3, d, s, 76879419ull, CPTC_VAL_LOGNORMAL, seed, out);
        }
        case 4:
        {
            const uint64_t d[4] = {183, 24, 1140, 1717};
            const double s[4] = {0.0, 0.0, 1.2, 1.2};
            return cptc_synth_zipf(4, d, s, 3300000ull, CPTC_VAL_POISSON1P2, seed, out);
        }
        case 5:
        {
            const uint64_t d[5] = {64, 64, 64, 32, 16};
            return cptc_synth_units5(d, 4000, 0.05, 0.5, 20000000ull, 4, seed, out);
        }
        default:
            return -1;
    }
}
