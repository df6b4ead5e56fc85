// Generic N-order CP-ALS driver (run_generic_cp, generic.cu:1639-2366), the
// host reordering (apply_reordering, generic.cu:1176-1376), the factor dump
// and the dense-unit self-test (run_dense_selftest, generic.cu:1389-1637).
//
// Device work goes through the C ABI's kernels on one stream; layout through
// layout_nd.  Host reordering reproduces the reference's floating-point
// sums bit for bit: HITS sums every (mode, row) in element order, so the
// rows are summed in parallel, each in its element order.
#include <hip/hip_runtime.h>
#include <omp.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <numeric>
#include <random>
#include <string>
#include <vector>

#include "hip_util.hpp"
#include "host_util.hpp"
#include "layout_nd.hpp"
#include "split_img.hpp"

namespace {

using Clock = std::chrono::high_resolution_clock;

double ms_since(Clock::time_point t0)
{
    return std::chrono::duration<double, std::milli>(Clock::now() - t0).count();
}

constexpr uint64_t GOLDEN = 0x9E3779B97F4A7C15ull;

// ------------------------------------------------------------ reordering --

struct HostCoo
{
    int N = 0;
    std::vector<uint64_t> dims;
    uint64_t nnz = 0;
    std::vector<uint32_t> idx;   // N x nnz
    const double* val = nullptr;
    uint32_t* c(int m) { return idx.data() + uint64_t(m) * nnz; }
    const uint32_t* c(int m) const { return idx.data() + uint64_t(m) * nnz; }
};

using Ranks = std::vector<std::vector<uint32_t>>;

// Elements e = 0, stride, 2*stride, ... grouped by coordinate of mode m, each
// group in element order (a stable counting sort of the sample).
struct SampleCsr
{
    std::vector<uint64_t> off;
    std::vector<uint32_t> el;
};

void sample_csr(const HostCoo& t, int m, uint64_t stride, SampleCsr& out)
{
    const uint64_t dim = t.dims[m];
    const uint32_t* cm = t.c(m);
    out.off.assign(dim + 1, 0);
    for (uint64_t e = 0; e < t.nnz; e += stride) ++out.off[cm[e] + 1];
    for (uint64_t i = 1; i <= dim; ++i) out.off[i] += out.off[i - 1];
    out.el.resize(out.off[dim]);
    std::vector<uint64_t> cur(out.off.begin(), out.off.end() - 1);
    for (uint64_t e = 0; e < t.nnz; e += stride) out.el[cur[cm[e]]++] = uint32_t(e);
}

void rank_by_score(const std::vector<double>& s, std::vector<uint32_t>& rank)
{
    std::vector<uint32_t> ord(s.size());
    std::iota(ord.begin(), ord.end(), 0u);
    std::sort(ord.begin(), ord.end(), [&](uint32_t a, uint32_t b) {
        return (s[a] != s[b]) ? (s[a] > s[b]) : (a < b);
    });
    rank.assign(s.size(), 0);
    for (size_t i = 0; i < ord.size(); ++i) rank[ord[i]] = uint32_t(i);
}

// generic.cu:1290-1341
void hits_ranks(const HostCoo& t, int rounds, uint64_t budget, Ranks& rank)
{
    const int N = t.N;
    const uint64_t stride = (t.nnz > budget && budget > 0) ? (t.nnz / budget) : 1;
    std::vector<SampleCsr> csr(N);
    for (int m = 0; m < N; ++m) sample_csr(t, m, stride, csr[m]);
    std::vector<std::vector<double>> s(N), ns(N);
    for (int m = 0; m < N; ++m) s[m].assign(t.dims[m], 1.0);
    // (mode, row) tasks
    std::vector<std::pair<int, uint32_t>> tasks;
    for (int m = 0; m < N; ++m)
        for (uint64_t x = 0; x < t.dims[m]; ++x)
            if (csr[m].off[x + 1] > csr[m].off[x]) tasks.emplace_back(m, uint32_t(x));
    for (int it = 0; it < rounds; ++it)
    {
        for (int m = 0; m < N; ++m) ns[m].assign(t.dims[m], 0.0);
#pragma omp parallel for schedule(dynamic, 4)
        for (size_t k = 0; k < tasks.size(); ++k)
        {
            const int m = tasks[k].first;
            const uint32_t x = tasks[k].second;
            double acc = 0.0;
            for (uint64_t j = csr[m].off[x]; j < csr[m].off[x + 1]; ++j)
            {
                const uint64_t e = csr[m].el[j];
                double p = 1.0;
                for (int q = 0; q < N; ++q)
                    if (q != m) p *= s[q][t.c(q)[e]];
                acc += p;
            }
            ns[m][x] = acc;
        }
        for (int m = 0; m < N; ++m)
        {
            double mx = 0.0;
            for (double v : ns[m]) mx = std::max(mx, v);
            if (mx > 0.0)
                for (double& v : ns[m]) v /= mx;
            s[m].swap(ns[m]);
        }
    }
    rank.assign(N, {});
    for (int m = 0; m < N; ++m) rank_by_score(s[m], rank[m]);
}

// generic.cu:1342-1357
void cadr_ranks(const HostCoo& t, Ranks& rank)
{
    rank.assign(t.N, {});
    for (int m = 0; m < t.N; ++m)
    {
        std::vector<uint32_t> deg(t.dims[m], 0);
        const uint32_t* cm = t.c(m);
        for (uint64_t e = 0; e < t.nnz; ++e) ++deg[cm[e]];
        std::vector<uint32_t> ord(t.dims[m]);
        std::iota(ord.begin(), ord.end(), 0u);
        std::sort(ord.begin(), ord.end(), [&](uint32_t a, uint32_t b) {
            return deg[a] != deg[b] ? deg[a] > deg[b] : a < b;
        });
        rank[m].assign(t.dims[m], 0);
        for (size_t i = 0; i < ord.size(); ++i) rank[m][ord[i]] = uint32_t(i);
    }
}

// generic.cu:1208-1237: sampled fill of 16^3 tiles x outer tuples (modes 0, 1, 2
// inner); `rk` (may be null) maps every coordinate first.
double probe_fill(const HostCoo& t, const Ranks* rk)
{
    const uint64_t budget = 2000000;
    const uint64_t st = (t.nnz > budget) ? (t.nnz / budget) : 1;
    const uint64_t nbj = (t.dims[1] + 15) / 16, nbk = (t.dims[2] + 15) / 16;
    auto co = [&](int m, uint64_t e) -> uint64_t {
        const uint32_t x = t.c(m)[e];
        return rk ? (*rk)[m][x] : x;
    };
    std::vector<uint64_t> keys;
    keys.reserve(t.nnz / st + 1);
    for (uint64_t e = 0; e < t.nnz; e += st)
    {
        const uint64_t a = co(0, e), b = co(1, e), c = co(2, e);
        const uint64_t tile = ((a / 16) * nbj + b / 16) * nbk + c / 16;
        uint64_t o = 0;
        for (int m = 3; m < t.N; ++m) o = o * 1000003ull + co(m, e);
        keys.push_back(cptc_gen_hash(tile ^ (o * GOLDEN)));
    }
    std::sort(keys.begin(), keys.end());
    long long tiles = 0, in = 0;
    for (size_t i = 0; i < keys.size();)
    {
        size_t j = i;
        while (j < keys.size() && keys[j] == keys[i]) ++j;
        const long long n = (long long)(j - i) * (long long)st;
        if (n >= 122)
        {
            ++tiles;
            in += n;
        }
        i = j;
    }
    return tiles ? double(in) / (double(tiles) * 4096.0) : 0.0;
}

void relabel(HostCoo& t, const Ranks& rank)
{
    for (int m = 0; m < t.N; ++m)
    {
        uint32_t* cm = t.c(m);
        const uint32_t* rk = rank[m].data();
#pragma omp parallel for schedule(static)
        for (int64_t e = 0; e < int64_t(t.nnz); ++e) cm[e] = rk[cm[e]];
    }
}

// Returns the method actually applied ("hits", "cadr" or "none").
std::string reorder(HostCoo& t, std::string how, int rounds, uint64_t budget, Ranks& rank,
                    bool verbose)
{
    rank.clear();
    if (rounds < 1) rounds = 1;
    if (budget == 0) budget = 8000000;
    if (how != "hits" && how != "cadr" && how != "none" && how != "auto")
    {
        if (verbose)
            std::printf("[GEN] unknown GEN_REORDER=%s -> falling back to cadr\n", how.c_str());
        how = "cadr";
    }
    if (how == "none" || t.nnz == 0) return "none";
    if (how == "cadr")
    {
        cadr_ranks(t, rank);
        relabel(t, rank);
        return "cadr";
    }
    if (how == "hits")
    {
        hits_ranks(t, rounds, budget, rank);
        relabel(t, rank);
        return "hits";
    }
    // auto (generic.cu:1201-1288)
    if (t.N < 3)
    {
        if (verbose) std::printf("[GEN] reorder=auto -> none (order %d < 3)\n", t.N);
        return "none";
    }
    const double f_raw = probe_fill(t, nullptr);
    if (f_raw < 0.02)
    {
        if (verbose)
            std::printf("[GEN] reorder=auto -> none (raw probe fill %g < 0.02)\n", f_raw);
        return "none";
    }
    Ranks rk;
    hits_ranks(t, rounds, budget, rk);
    // The reference relabels before probing and then maps the relabelled
    // coordinates through the ranks once more; the probe here reads the same
    // coordinates: rank[rank[c]].
    Ranks twice(t.N);
    for (int m = 0; m < t.N; ++m)
    {
        twice[m].resize(t.dims[m]);
        for (uint64_t a = 0; a < t.dims[m]; ++a) twice[m][a] = rk[m][rk[m][a]];
    }
    const double f_hits = probe_fill(t, &twice);
    if (f_hits >= 0.11)
    {
        if (verbose)
            std::printf("[GEN] reorder=auto -> hits (probe fill %g -> %g >= 0.11)\n", f_raw,
                        f_hits);
        rank = rk;
        relabel(t, rank);
        return "hits";
    }
    if (verbose)
        std::printf("[GEN] reorder=auto -> none (probe fill %g -> %g < 0.11)\n", f_raw, f_hits);
    return "none";
}

bool coo_ok(const cptc_coo* c)
{
    if (!c || c->nmodes < 1 || c->nmodes > CPTC_MAX_MODES) return false;
    if (c->nnz && (!c->idx || !c->val)) return false;
    return true;
}

int check_indices(const cptc_coo* c)
{
    for (int m = 0; m < c->nmodes; ++m)
    {
        const uint32_t* cm = c->idx + uint64_t(m) * c->nnz;
        uint32_t mx = 0;
#pragma omp parallel for reduction(max : mx)
        for (int64_t e = 0; e < int64_t(c->nnz); ++e) mx = std::max(mx, cm[e]);
        CPTC_REQUIRE(c->nnz == 0 || uint64_t(mx) < c->dims[m], CPTC_ERR_ARG,
                     "coordinate %u of mode %d outside dim %llu", mx, m,
                     (unsigned long long)c->dims[m]);
    }
    return CPTC_OK;
}

HostCoo host_copy(const cptc_coo* c)
{
    HostCoo t;
    t.N = c->nmodes;
    t.dims.assign(c->dims, c->dims + c->nmodes);
    t.nnz = c->nnz;
    t.idx.assign(c->idx, c->idx + uint64_t(c->nmodes) * c->nnz);
    t.val = c->val;
    return t;
}

// ---------------------------------------------------------------- driver --

template <class T>
int dmalloc(T** p, size_t n)
{
    *p = nullptr;
    if (n == 0) return CPTC_OK;
    CPTC_HIP(hipMalloc(reinterpret_cast<void**>(p), n * sizeof(T)));
    return CPTC_OK;
}

template <class T>
void dfree(T*& p)
{
    if (p) (void)hipFree(p);
    p = nullptr;
}

struct Gen
{
    int N = 0;
    int R = 0;
    uint64_t nnz = 0;
    std::vector<uint64_t> dims;
    uint64_t maxdim = 0;
    cptc_gen_opts opts{};
    std::string method = "none";
    Ranks rank;   // empty when no relabel
    double prep_ms[3] = {0, 0, 0};
    double x2 = 0.0;

    hipStream_t s = nullptr;
    double* d_L = nullptr;          // R x R Cholesky factor of FtF + eps I
    uint32_t* d_coords = nullptr;   // N x nnz (reordered)
    double* d_vals = nullptr;
    std::vector<double*> d_F;
    double* d_lambda = nullptr;
    double* d_grams = nullptr;      // N x R x R
    double* d_FtF = nullptr;
    double* d_FtV = nullptr;        // maxdim x R
    double* d_out2 = nullptr;       // fit scalars / residual

    bool dense = false;
    unsigned inner_mask = 0;
    cptc::DevUnitsN units;
    float* d_tiles = nullptr;
    double* d_W = nullptr;
    // split-bf16 unit kernel (GEN_TILE_KERNEL / the automatic rule)
    bool tile_b3 = false;
    void* d_tile_ws = nullptr;
    size_t tile_ws_bytes = 0;
    // compacted unit image (GEN_TILE_COMPACT=0: the dense one)
    cptc::SplitImg uimg[3];   // compacted split unit image per inner slot
    // per-slot unit groups (one target row block each) for the grouped MFMA launch
    uint32_t* d_uorder[3] = {nullptr, nullptr, nullptr};
    uint32_t* d_ugoff[3] = {nullptr, nullptr, nullptr};
    size_t ungroups[3] = {0, 0, 0};
    bool w_dirty = true;
    // every element in a dense unit (config 5): the outer modes' MTTKRP from
    // per-unit inner sums (cptc_gen_unit_sums, formed once after the inner
    // factors change) instead of the segment kernel over the same elements;
    // GEN_UNIT_SUMS=0 keeps the segment kernel
    bool unit_sums = false;
    bool usum_ok = false;
    double* d_usum = nullptr;          // nunits x R
    double* d_uimg64 = nullptr;        // the units' FP64 images for cptc_gen_unit_sums_img
    double** d_Fo = nullptr;           // the outer modes' factors, device array of pointers
    uint32_t* d_us_order = nullptr;    // cptc_gen_unit_sums_plan: units by inner block triple
    uint32_t* d_us_chunk = nullptr;    // chunk offsets into d_us_order
    size_t us_nchunks = 0;
    std::vector<cptc::DevViewN> views;   // kernel views (dense elements dropped, rows sorted)
    std::vector<uint64_t> ref_nseg;      // segments of the reference-layout views

    // per-kernel timing: seg / unit kernel of each mode, summed over iterations
    hipEvent_t kev[4 * CPTC_MAX_MODES] = {};
    hipEvent_t* kev_cur = kev;   // the event block of the iteration being queued
    bool timing = false;
    // queued runs (no host wait per iteration): per-iteration fit scalars on
    // the device and a pool of timing events, both grown on first use
    double* d_fit_hist = nullptr;
    size_t fit_hist_cap = 0;
    std::vector<hipEvent_t> ev_pool;
    double k_seg[CPTC_MAX_MODES] = {}, k_unit[CPTC_MAX_MODES] = {};
    int k_iters = 0;

    // GEN_PROFILE: gram, mttkrp, solve, norm, fit
    std::vector<hipEvent_t> ev;
    double prof[5] = {0, 0, 0, 0, 0};
    int prof_iters = 0;

    ~Gen()
    {
        if (s) (void)hipStreamSynchronize(s);
        dfree(d_coords);
        dfree(d_vals);
        for (auto& p : d_F) dfree(p);
        dfree(d_lambda);
        dfree(d_grams);
        dfree(d_FtF);
        dfree(d_FtV);
        dfree(d_out2);
        dfree(d_tiles);
        dfree(d_tile_ws);
        for (cptc::SplitImg& u : uimg) cptc::free_split_img(u);
        dfree(d_W);
        for (int q = 0; q < 3; ++q)
        {
            dfree(d_uorder[q]);
            dfree(d_ugoff[q]);
        }
        cptc::free_units(units);
        for (auto& v : views) cptc::free_view(v);
        for (auto& e : ev) (void)hipEventDestroy(e);
        for (auto& e : kev)
            if (e) (void)hipEventDestroy(e);
        for (auto& e : ev_pool) (void)hipEventDestroy(e);
        dfree(d_fit_hist);
        dfree(d_L);
        dfree(d_usum);
        dfree(d_uimg64);
        if (d_Fo) (void)hipFree(d_Fo);
        if (d_us_order) (void)hipFree(d_us_order);
        if (d_us_chunk) (void)hipFree(d_us_chunk);
        if (s) (void)hipStreamDestroy(s);
    }

    int slot_of(int n) const
    {
        for (int q = 0; q < 3; ++q)
            if (units.inner[q] == n) return q;
        return -1;
    }

    const double* const* F() const { return d_F.data(); }

    // FtV = MTTKRP of mode n (zeroed first, unless `zeroed`).  With `timing`,
    // events bracket the unit kernel (kev 0-1) and the segment kernel (kev 2-3).
    int mttkrp(int n, bool zeroed = false)
    {
        if (!zeroed) CPTC_HIP(hipMemsetAsync(d_FtV, 0, dims[n] * size_t(R) * sizeof(double), s));
        const bool in = dense && (inner_mask & (1u << n));
        hipEvent_t* ke = kev_cur + 4 * n;
        if (timing) CPTC_HIP(hipEventRecord(ke[0], s));
        if (in)
        {
            if (w_dirty)
            {
                std::vector<int> om(units.outer.begin(), units.outer.end());
                CPTC_TRY(cptc_units_weights_nd(units.d_unit6, units.nunits, units.d_outer_coords,
                                               int(om.size()), om.data(), F(), R, d_W, s));
                w_dirty = false;
            }
            const int* in3 = units.inner;
            const int sl = slot_of(n);
            if (tile_b3 && uimg[sl].ready())
                CPTC_TRY(cptc_mttkrp_units_nd_cws(
                    sl, units.d_unit6, units.nunits, uimg[sl].cmask, uimg[sl].segoff,
                    uimg[sl].seg, uimg[sl].nseg, d_W,
                    d_uorder[sl], d_ugoff[sl], ungroups[sl], d_F[in3[0]], d_F[in3[1]],
                    d_F[in3[2]], int(dims[in3[0]]), int(dims[in3[1]]), int(dims[in3[2]]), d_FtV, R,
                    d_tile_ws, tile_ws_bytes, s));
            else if (tile_b3)
                CPTC_TRY(cptc_mttkrp_units_nd_ws(
                    sl, units.d_unit6, units.nunits, d_tiles, d_W, d_uorder[sl], d_ugoff[sl],
                    ungroups[sl], d_F[in3[0]], d_F[in3[1]], d_F[in3[2]], int(dims[in3[0]]),
                    int(dims[in3[1]]), int(dims[in3[2]]), d_FtV, R, d_tile_ws, tile_ws_bytes, s));
            else
                CPTC_TRY(cptc_mttkrp_units_nd(sl, units.d_unit6, units.nunits, d_tiles, d_W,
                                              d_uorder[sl], d_ugoff[sl], ungroups[sl],
                                              d_F[in3[0]], d_F[in3[1]], d_F[in3[2]],
                                              int(dims[in3[0]]), int(dims[in3[1]]),
                                              int(dims[in3[2]]), d_FtV, R, s));
        }
        const bool usum_path = unit_sums && !in;
        if (timing && !usum_path)
        {
            CPTC_HIP(hipEventRecord(ke[1], s));
            CPTC_HIP(hipEventRecord(ke[2], s));
        }
        if (usum_path)
        {
            // events: kev 0-1 the per-unit sums (when formed), kev 2-3 the scatter
            const int* in3 = units.inner;
            if (!usum_ok)
            {
                if (d_uimg64)
                    CPTC_TRY(cptc_gen_unit_sums_img(units.d_unit6, units.nunits, d_uimg64,
                                                    d_us_order, d_us_chunk, us_nchunks,
                                                    d_F[in3[0]], d_F[in3[1]], d_F[in3[2]],
                                                    int(dims[in3[0]]), int(dims[in3[1]]),
                                                    int(dims[in3[2]]), R, d_usum, s));
                else
                    CPTC_TRY(cptc_gen_unit_sums(units.d_unit6, units.nunits, units.d_lid,
                                                units.d_val, d_us_order, d_us_chunk, us_nchunks,
                                                d_F[in3[0]], d_F[in3[1]], d_F[in3[2]],
                                                int(dims[in3[0]]), int(dims[in3[1]]),
                                                int(dims[in3[2]]), R, d_usum, s));
                usum_ok = true;
            }
            if (timing)
            {
                CPTC_HIP(hipEventRecord(ke[1], s));
                CPTC_HIP(hipEventRecord(ke[2], s));
            }
            int pos = 0;
            while (units.outer[size_t(pos)] != n) ++pos;
            CPTC_TRY(cptc_gen_unit_scatter(units.d_outer_coords, units.nunits,
                                           int(units.outer.size()), pos,
                                           const_cast<const double* const*>(d_Fo), d_usum, R, dims[n],
                                           d_FtV, s));
            if (timing) CPTC_HIP(hipEventRecord(ke[3], s));
            return CPTC_OK;
        }
        const cptc::DevViewN& v = views[n];
        if (v.key_bytes > 0 && R % 2 == 0)
            CPTC_TRY(cptc_mttkrp_seg_nd_keys_dims(
                N, n, v.d_key, v.key_bytes, v.level_modes.data(), v.level_bits.data(), v.d_vals,
                v.nnz, v.d_row, v.d_start, v.d_cnt, v.d_single, v.nseg, F(), dims.data(), d_FtV,
                R, s));
        else
            CPTC_TRY(cptc_mttkrp_seg_nd(N, n, v.d_sc, v.level_modes.data(), v.d_vals, nullptr,
                                        v.nnz, v.d_row, v.d_start, v.d_cnt, v.d_single, v.nseg,
                                        F(), d_FtV, R, s));
        if (timing) CPTC_HIP(hipEventRecord(ke[3], s));
        return CPTC_OK;
    }

    // accumulate every mode's kernel events (after the iteration's sync)
    int collect_kernel_times()
    {
        for (int n = 0; n < N; ++n)
        {
            float a = 0.0f, b = 0.0f;
            CPTC_HIP(hipEventElapsedTime(&a, kev_cur[4 * n], kev_cur[4 * n + 1]));
            CPTC_HIP(hipEventElapsedTime(&b, kev_cur[4 * n + 2], kev_cur[4 * n + 3]));
            k_unit[n] += a;
            k_seg[n] += b;
        }
        ++k_iters;
        return CPTC_OK;
    }

    void mark(int i)
    {
        if (opts.profile && i < int(ev.size())) (void)hipEventRecord(ev[i], s);
    }

    // one iteration's updates and the fit scalars into d_out (no host wait)
    int enqueue_iteration(double* d_out, int& mk)
    {
        const size_t RR = size_t(R) * R;
        // a small factor's update (cptc_gen_normalize_gram) also forms the
        // next mode's FtF and zeroes its FtV
        bool ftf_ready = false, ftv_zeroed = false;
        for (int n = 0; n < N; ++n)
        {
            if (!ftf_ready) CPTC_TRY(cptc_gram_hadamard(d_grams, N, n, R, d_FtF, s));
            mark(mk++);
            CPTC_TRY(mttkrp(n, ftv_zeroed));
            ftf_ready = ftv_zeroed = false;
            mark(mk++);
            // One stream: factoring FtF on a second stream beside the MTTKRP
            // measured slower (configs 4 and 5: 0.545 -> 0.60 and 1.54 ->
            // 1.58 ms per iteration) because the cross-stream waits cost
            // more than the factorization.
            if (opts.svd)
                CPTC_TRY(cptc_solve_pinv(d_FtF, d_FtV, d_F[n], dims[n], R, nullptr, s));
            else
            {
                CPTC_TRY(cptc_chol_ridge_solve(d_FtF, d_FtV, d_F[n], dims[n], R, s));
            }
            mark(mk++);
            // one workgroup pays while its Gram loop is short: <= 256 rows
            // per row group (1024 / R^2 groups)
            if (R <= 32 && dims[n] <= size_t(256) * size_t(1024 / (R * R)) &&
                dims[n] * size_t(R) <= (size_t(1) << 16))
            {
                const int next = n + 1 < N ? n + 1 : -1;
                const size_t nz = next >= 0 && dims[next] * size_t(R) <= (size_t(1) << 18)
                                      ? dims[next] * size_t(R)
                                      : 0;
                CPTC_TRY(cptc_gen_normalize_gram(d_F[n], dims[n], R, d_lambda, d_grams, N, n, next,
                                                 d_FtF, d_FtV, nz, s));
                ftf_ready = next >= 0;
                ftv_zeroed = nz > 0;
            }
            else
            {
                CPTC_TRY(cptc_gen_normalize(d_F[n], dims[n], R, d_lambda, s));
                CPTC_TRY(cptc_gram(d_F[n], dims[n], R, d_grams + size_t(n) * RR, s));
            }
            if (dense && !(inner_mask & (1u << n))) w_dirty = true;
            if (dense && (inner_mask & (1u << n))) usum_ok = false;
            mark(mk++);
        }
        return cptc_fit_gram(d_F[N - 1], d_FtV, dims[N - 1], d_lambda, d_grams, N, R, d_out, s);
    }

    double fit_of(double iprod, double model2) const
    {
        const double res = std::max(x2 - 2.0 * iprod + model2, 0.0);
        const double xn = std::sqrt(x2);
        return (xn > 0.0) ? 1.0 - std::sqrt(res) / xn : 0.0;
    }

    // Queued runs time the segment / unit kernels (4 events per mode) on
    // every KSAMPLE-th iteration and the last one only: recording them on
    // every iteration cost 60 us of a 0.42 ms config-4 iteration and 81 us
    // of a 1.42 ms config-5 iteration.
    static constexpr int KSAMPLE = 8;
    static bool kernel_sampled(int it, int iters)
    {
        return it % KSAMPLE == KSAMPLE - 1 || it == iters - 1;
    }

    // `iters` iterations queued back to back; one wait at the end.  Fits,
    // per-iteration GPU times and kernel times are read afterwards.
    int run_queued(int iters, double* fit, double* iprod, double* model2, double* ms_iter)
    {
        if (iters <= 0) return CPTC_OK;
        if (fit_hist_cap < size_t(iters))
        {
            dfree(d_fit_hist);
            CPTC_TRY(dmalloc(&d_fit_hist, size_t(2) * iters));
            fit_hist_cap = size_t(iters);
        }
        const size_t per = size_t(1 + 4 * N);   // iteration end + kernel events
        const size_t need = 1 + per * size_t(iters);
        while (ev_pool.size() < need)
        {
            hipEvent_t e = nullptr;
            CPTC_HIP(hipEventCreate(&e));
            ev_pool.push_back(e);
        }
        CPTC_HIP(hipEventRecord(ev_pool[0], s));
        const bool want = timing;
        for (int it = 0; it < iters; ++it)
        {
            hipEvent_t* blk = ev_pool.data() + 1 + per * size_t(it);
            kev_cur = blk + 1;
            int mk = 0;
            timing = want && kernel_sampled(it, iters);
            const int rc = enqueue_iteration(d_fit_hist + 2 * it, mk);
            timing = want;
            kev_cur = kev;
            CPTC_TRY(rc);
            CPTC_HIP(hipEventRecord(blk[0], s));
        }
        std::vector<double> h(size_t(2) * iters);
        CPTC_HIP(hipMemcpyAsync(h.data(), d_fit_hist, h.size() * sizeof(double),
                                hipMemcpyDeviceToHost, s));
        CPTC_HIP(hipStreamSynchronize(s));
        hipEvent_t prev = ev_pool[0];
        for (int it = 0; it < iters; ++it)
        {
            hipEvent_t* blk = ev_pool.data() + 1 + per * size_t(it);
            if (fit) fit[it] = fit_of(h[2 * it], h[2 * it + 1]);
            if (iprod) iprod[it] = h[2 * it];
            if (model2) model2[it] = h[2 * it + 1];
            float ms = 0.0f;
            CPTC_HIP(hipEventElapsedTime(&ms, prev, blk[0]));
            if (ms_iter) ms_iter[it] = ms;
            prev = blk[0];
            if (timing && kernel_sampled(it, iters))
            {
                kev_cur = blk + 1;
                const int rc = collect_kernel_times();
                kev_cur = kev;
                CPTC_TRY(rc);
            }
        }
        return CPTC_OK;
    }

    int iterate(double* fit, double* iprod, double* model2)
    {
        int mk = 0;
        mark(mk++);
        CPTC_TRY(enqueue_iteration(d_out2, mk));
        double h[2] = {0.0, 0.0};
        CPTC_HIP(hipMemcpyAsync(h, d_out2, sizeof(h), hipMemcpyDeviceToHost, s));
        CPTC_HIP(hipStreamSynchronize(s));
        mark(mk++);
        if (timing) CPTC_TRY(collect_kernel_times());
        if (fit) *fit = fit_of(h[0], h[1]);
        if (iprod) *iprod = h[0];
        if (model2) *model2 = h[1];
        if (opts.profile)
        {
            CPTC_HIP(hipEventSynchronize(ev[mk - 1]));
            double d[5] = {0, 0, 0, 0, 0};
            for (int i = 0; i + 1 < mk; ++i)
            {
                float t = 0.0f;
                CPTC_HIP(hipEventElapsedTime(&t, ev[i], ev[i + 1]));
                d[(i < 4 * N) ? (i % 4) : 4] += t;
            }
            for (int q = 0; q < 5; ++q) prof[q] += d[q];
            ++prof_iters;
            if (opts.verbose)
                std::printf("[GEN][profile] iter %d gram=%g mttkrp=%g solve=%g norm=%g fit=%g "
                            "sum=%g ms\n",
                            prof_iters, d[0], d[1], d[2], d[3], d[4],
                            d[0] + d[1] + d[2] + d[3] + d[4]);
        }
        return CPTC_OK;
    }
};

Gen* as_gen(void* h) { return static_cast<Gen*>(h); }

// Units of each slot grouped by target row block for the grouped MFMA
// launch (UNIT_GROUP units per wave at most, fewer when the units are few).
// Device arrays are allocated here; the caller frees them.
constexpr int UNIT_GROUP = 16;

int build_unit_groups(const cptc::DevUnitsN& u, int R, hipStream_t s, uint32_t* order[3],
                      uint32_t* goff[3], size_t ng[3], int rank_block)
{
    for (int q = 0; q < 3; ++q)
    {
        order[q] = goff[q] = nullptr;
        ng[q] = 0;
    }
    const size_t nu = u.nunits;
    if (nu == 0) return CPTC_OK;
    std::vector<int32_t> hdr(nu * 6);
    CPTC_HIP(hipMemcpyAsync(hdr.data(), u.d_unit6, hdr.size() * sizeof(int32_t),
                            hipMemcpyDeviceToHost, s));
    CPTC_HIP(hipStreamSynchronize(s));
    std::vector<uint32_t> ord(nu), off(nu + 1);
    int dev = 0, cus = 0;
    CPTC_HIP(hipGetDevice(&dev));
    CPTC_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    const int cap = cptc::tile_group_cap(nu, R, cus, UNIT_GROUP, rank_block);
    for (int q = 0; q < 3; ++q)
    {
        CPTC_TRY(cptc_dense_groups(hdr.data(), 6, nu, q, cap, ord.data(), off.data(), &ng[q]));
        CPTC_HIP(hipMalloc(&order[q], nu * sizeof(uint32_t)));
        CPTC_HIP(hipMalloc(&goff[q], (ng[q] + 1) * sizeof(uint32_t)));
        CPTC_HIP(hipMemcpyAsync(order[q], ord.data(), nu * sizeof(uint32_t), hipMemcpyHostToDevice, s));
        CPTC_HIP(hipMemcpyAsync(goff[q], off.data(), (ng[q] + 1) * sizeof(uint32_t),
                                hipMemcpyHostToDevice, s));
        CPTC_HIP(hipStreamSynchronize(s));
    }
    return CPTC_OK;
}

// Units sorted by inner block triple, in chunks of <= 8 (a workgroup of the
// unit-sum kernel stages the chunk's three factor blocks once; its 4 waves
// take 2 units each).
int build_unit_sums_plan(const cptc::DevUnitsN& u, hipStream_t s, uint32_t*& d_order,
                         uint32_t*& d_chunk, size_t& nchunks)
{
    const size_t nu = u.nunits;
    std::vector<uint32_t> hdr(nu * 6), ord(nu), off(nu + 1);
    CPTC_HIP(hipMemcpyAsync(hdr.data(), u.d_unit6, hdr.size() * sizeof(uint32_t),
                            hipMemcpyDeviceToHost, s));
    CPTC_HIP(hipStreamSynchronize(s));
    CPTC_TRY(cptc_gen_unit_sums_plan(hdr.data(), nu, 8, ord.data(), off.data(), &nchunks));
    CPTC_HIP(hipMalloc(&d_order, nu * sizeof(uint32_t)));
    CPTC_HIP(hipMalloc(&d_chunk, (nchunks + 1) * sizeof(uint32_t)));
    CPTC_HIP(hipMemcpyAsync(d_order, ord.data(), nu * sizeof(uint32_t), hipMemcpyHostToDevice, s));
    CPTC_HIP(hipMemcpyAsync(d_chunk, off.data(), (nchunks + 1) * sizeof(uint32_t),
                            hipMemcpyHostToDevice, s));
    CPTC_HIP(hipStreamSynchronize(s));
    return CPTC_OK;
}

bool env_set(const char* k) { return std::getenv(k) != nullptr; }

// generic.cu:1743-1782: U[0,1) draws in mode order; row a of the data keeps
// the vector it would have had without reordering.
void init_factors(const std::vector<uint64_t>& dims, int R, unsigned seed, const Ranks& rank,
                  std::vector<std::vector<double>>& F)
{
    std::mt19937 gen(seed);
    std::uniform_real_distribution<double> dis(0.0, 1.0);
    F.assign(dims.size(), {});
    for (size_t m = 0; m < dims.size(); ++m)
    {
        const uint64_t dim = dims[m];
        std::vector<double> u(dim * R);
        for (auto& x : u) x = dis(gen);
        F[m].assign(dim * R, 0.0);
        const bool has = m < rank.size() && rank[m].size() == dim;
        for (uint64_t a = 0; a < dim; ++a)
        {
            const uint64_t nw = has ? rank[m][a] : a;
            std::memcpy(&F[m][nw * R], &u[a * R], size_t(R) * sizeof(double));
        }
    }
}

}  // namespace

extern "C" int cptc_gen_reorder(cptc_coo* t, const char* how, int rounds, uint64_t sample_budget,
                                uint32_t* rank_out, int* applied)
{
    CPTC_REQUIRE(coo_ok(t), CPTC_ERR_ARG, "cptc_gen_reorder: bad tensor");
    CPTC_TRY(check_indices(t));
    HostCoo h = host_copy(t);
    std::string m = how ? how : (t->nmodes >= 4 ? "hits" : "cadr");
    Ranks rank;
    const std::string used = reorder(h, m, rounds, sample_budget, rank, false);
    const bool did = !rank.empty();
    if (did) std::memcpy(t->idx, h.idx.data(), h.idx.size() * sizeof(uint32_t));
    if (applied) *applied = did ? 1 : 0;
    if (rank_out)
    {
        uint64_t off = 0;
        for (int q = 0; q < t->nmodes; ++q)
        {
            for (uint64_t a = 0; a < t->dims[q]; ++a)
                rank_out[off + a] = did ? rank[q][a] : uint32_t(a);
            off += t->dims[q];
        }
    }
    (void)used;
    return CPTC_OK;
}

extern "C" void cptc_gen_default_opts(cptc_gen_opts* o)
{
    if (!o) return;
    std::memset(o, 0, sizeof(*o));
    o->R = 32;
    o->seed = env_set("GEN_SEED") ? unsigned(std::atoi(std::getenv("GEN_SEED"))) : 42u;
    if (const char* e = std::getenv("GEN_REORDER")) std::snprintf(o->reorder, sizeof(o->reorder), "%s", e);
    o->reorder_rounds = env_set("GEN_REORDER_T") ? std::atoi(std::getenv("GEN_REORDER_T")) : 3;
    o->reorder_sample = env_set("GEN_REORDER_SAMPLE")
                            ? std::strtoull(std::getenv("GEN_REORDER_SAMPLE"), nullptr, 10)
                            : 8000000ull;
    o->dense = env_set("GEN_DENSE") ? (std::atoi(std::getenv("GEN_DENSE")) != 0) : 1;
    o->threshold = env_set("GEN_DENSE_THRESHOLD") ? std::atof(std::getenv("GEN_DENSE_THRESHOLD")) : 0.03;
    o->inner[0] = 0;
    o->inner[1] = 1;
    o->inner[2] = 2;
    if (const char* e = std::getenv("GEN_DENSE_INNER"))
    {
        int k = 0;
        const char* q = e;
        while (*q && k < 3)
        {
            o->inner[k++] = std::atoi(q);
            while (*q && *q != ',') ++q;
            if (*q == ',') ++q;
        }
    }
    o->svd = env_set("GEN_SOLVER") && std::string(std::getenv("GEN_SOLVER")) == "svd";
    o->profile = env_set("GEN_PROFILE") ? 1 : 0;
    o->verbose = 0;
}

extern "C" int cptc_gen_create(const cptc_coo* coo, const cptc_gen_opts* opts, void** handle)
{
    CPTC_REQUIRE(handle && opts, CPTC_ERR_ARG, "cptc_gen_create: null argument");
    *handle = nullptr;
    CPTC_REQUIRE(coo_ok(coo) && coo->nmodes >= 2, CPTC_ERR_ARG,
                 "cptc_gen_create: invalid tensor (nmodes 2..%d)", CPTC_MAX_MODES);
    const int R = opts->R;
    CPTC_REQUIRE(coo->nnz > 0 && R >= 1 && R <= 32, CPTC_ERR_UNSUPPORTED,
                 "[GEN] invalid run config (nmodes=%d nnz=%llu R=%d)", coo->nmodes,
                 (unsigned long long)coo->nnz, R);
    CPTC_REQUIRE(coo->nnz <= 0x7FFFFFFFull, CPTC_ERR_UNSUPPORTED,
                 "[GEN] nnz too large for 1D grid (%llu)", (unsigned long long)coo->nnz);
    for (int m = 0; m < coo->nmodes; ++m)
        CPTC_REQUIRE(coo->dims[m] >= 1 && coo->dims[m] <= 0xFFFFFFFFull, CPTC_ERR_ARG,
                     "cptc_gen_create: dim %d = %llu", m, (unsigned long long)coo->dims[m]);
    CPTC_TRY(check_indices(coo));
    auto* g = new Gen();
    auto fail = [&](int rc) {
        delete g;
        return rc;
    };
    g->opts = *opts;
    g->N = coo->nmodes;
    g->R = R;
    g->nnz = coo->nnz;
    g->dims.assign(coo->dims, coo->dims + coo->nmodes);
    for (auto d : g->dims) g->maxdim = std::max(g->maxdim, d);
    const int N = g->N;
    const bool verbose = opts->verbose != 0;

    for (uint64_t e = 0; e < g->nnz; ++e) g->x2 += coo->val[e] * coo->val[e];

    int rc;
#define GEN_TRY(expr)                     \
    do                                    \
    {                                     \
        if ((rc = (expr)) != CPTC_OK)     \
            return fail(rc);              \
    } while (0)
#define GEN_HIP(call)                                                                      \
    do                                                                                     \
    {                                                                                      \
        hipError_t e_ = (call);                                                            \
        if (e_ != hipSuccess)                                                              \
        {                                                                                  \
            cptc::set_error("%s:%d %s -> %s", __FILE__, __LINE__, #call,                   \
                            hipGetErrorString(e_));                                        \
            return fail(CPTC_ERR_HIP);                                                     \
        }                                                                                  \
    } while (0)

    GEN_HIP(hipStreamCreateWithFlags(&g->s, hipStreamNonBlocking));
    hipStream_t s = g->s;
    const size_t RR = size_t(R) * R;
    const uint64_t ncoords = uint64_t(N) * g->nnz;
    GEN_TRY(dmalloc(&g->d_coords, ncoords));
    GEN_TRY(dmalloc(&g->d_vals, g->nnz));
    GEN_HIP(hipMemcpyAsync(g->d_coords, coo->idx, ncoords * sizeof(uint32_t),
                           hipMemcpyHostToDevice, s));
    GEN_HIP(hipMemcpyAsync(g->d_vals, coo->val, g->nnz * sizeof(double), hipMemcpyHostToDevice, s));

    // reorder on the device (relabels d_coords; ranks come back for the factors)
    auto t0 = Clock::now();
    std::string how = opts->reorder[0] ? std::string(opts->reorder, strnlen(opts->reorder, 8))
                                       : (N >= 4 ? "hits" : "cadr");
    GEN_TRY(cptc::reorder_nd_device(N, g->dims.data(), g->d_coords, g->nnz, how,
                                    opts->reorder_rounds, opts->reorder_sample, g->rank,
                                    g->method, verbose, s));
    GEN_HIP(hipStreamSynchronize(s));
    g->prep_ms[0] = ms_since(t0);
    if (verbose)
    {
        std::printf("[GEN] reorder=%s", g->method.c_str());
        if (g->method == "hits") std::printf("(T=%d)", std::max(opts->reorder_rounds, 1));
        std::printf(" prep=%g ms (device)\n", g->prep_ms[0]);
        std::printf("[GEN] N-order CP-ALS: order=%d R=%d nnz=%llu\n[GEN] dims = ", N, R,
                    (unsigned long long)g->nnz);
        for (int m = 0; m < N; ++m)
            std::printf("%s%llu", m ? " x " : "", (unsigned long long)g->dims[m]);
        std::printf("\n");
    }

    std::vector<std::vector<double>> F0;
    init_factors(g->dims, R, opts->seed, g->rank, F0);
    g->d_F.assign(N, nullptr);
    for (int m = 0; m < N; ++m)
    {
        GEN_TRY(dmalloc(&g->d_F[m], g->dims[m] * R));
        GEN_HIP(hipMemcpyAsync(g->d_F[m], F0[m].data(), F0[m].size() * sizeof(double),
                               hipMemcpyHostToDevice, s));
    }
    GEN_TRY(dmalloc(&g->d_lambda, size_t(R)));
    {
        std::vector<double> ones(R, 1.0);
        GEN_HIP(hipMemcpyAsync(g->d_lambda, ones.data(), R * sizeof(double), hipMemcpyHostToDevice, s));
        GEN_HIP(hipStreamSynchronize(s));
    }
    GEN_TRY(dmalloc(&g->d_grams, RR * N));
    GEN_TRY(dmalloc(&g->d_FtF, RR));
    GEN_TRY(dmalloc(&g->d_L, RR));
    GEN_TRY(dmalloc(&g->d_FtV, g->maxdim * R));
    GEN_TRY(dmalloc(&g->d_out2, size_t(2)));

    // dense units
    t0 = Clock::now();
    const int* in = opts->inner;
    const bool inner_ok = N >= 3 && in[0] >= 0 && in[1] >= 0 && in[2] >= 0 && in[0] < N &&
                          in[1] < N && in[2] < N && in[0] != in[1] && in[0] != in[2] &&
                          in[1] != in[2];
    if (opts->dense && N >= 4 && opts->threshold > 0.0 && !inner_ok && verbose)
        std::printf("[GEN] dense path disabled: GEN_DENSE_INNER=%d,%d,%d is not a set of three "
                    "distinct modes\n",
                    in[0], in[1], in[2]);
    if (opts->dense && N >= 4 && opts->threshold > 0.0 && inner_ok)
    {
        GEN_TRY(cptc::units_nd_device(N, g->dims.data(), g->d_coords, g->d_vals, g->nnz,
                                      opts->threshold, in, g->units, s));
        g->dense = g->units.nunits > 0;
        if (g->dense)
        {
            for (int q = 0; q < 3; ++q) g->inner_mask |= 1u << in[q];
            GEN_TRY(dmalloc(&g->d_tiles, g->units.nunits * 4096));
            GEN_TRY(dmalloc(&g->d_W, g->units.nunits * R));
            GEN_TRY(cptc_units_pack_nd(g->units.d_unit6, g->units.nunits, g->units.d_lid,
                                       g->units.d_val, g->d_tiles, s));
            // split-bf16 units for R > 16 and enough units (the order-3
            // driver's rule); GEN_TILE_KERNEL=fp32 / bf16x3 forces the choice
            const int sw = cptc::tile_kernel_switch("GEN_TILE_KERNEL");
            g->tile_b3 = sw < 0 ? cptc::tile_b3_auto(g->units.nunits, R) : sw == 1;
            GEN_TRY(build_unit_groups(g->units, R, s, g->d_uorder, g->d_ugoff, g->ungroups,
                                      g->tile_b3 ? 32 : 16));
            // every element in a unit: the outer modes' MTTKRP from per-unit sums
            const char* us = std::getenv("GEN_UNIT_SUMS");
            if (g->units.dense_nnz == g->nnz && R <= 32 && !g->units.outer.empty() &&
                !(us && std::atoi(us) == 0))
            {
                GEN_TRY(dmalloc(&g->d_usum, g->units.nunits * size_t(R)));
                GEN_TRY(build_unit_sums_plan(g->units, s, g->d_us_order, g->d_us_chunk,
                                             g->us_nchunks));
                // the sums from FP64 unit images on the matrix cores (32 KB
                // per unit, up to 8 GiB) when the units are at least a fifth
                // full: the image path streams every cell (HBM bound, ~6.7 ns
                // per unit) whatever the fill, the pool path reads three
                // factor rows from LDS per element (LDS bound, ~10 ps per
                // element).  Config 5 (fill 0.149): 0.220 against 0.203 ms
                // per call.  GEN_UNIT_SUMS_IMG=1 / 0 forces the choice.
                const char* ui = std::getenv("GEN_UNIT_SUMS_IMG");
                const double fill = double(g->units.dense_nnz) /
                                    (double(g->units.nunits) * 4096.0);
                const bool img = ui ? std::strcmp(ui, "0") != 0 : fill >= 0.2;
                if (img && g->units.nunits <= (size_t(8) << 30) / (4096 * sizeof(double)))
                {
                    GEN_TRY(dmalloc(&g->d_uimg64, g->units.nunits * 4096));
                    GEN_TRY(cptc_units_pack_nd_f64(g->units.d_unit6, g->units.nunits,
                                                   g->units.d_lid, g->units.d_val, g->d_uimg64, s));
                }
                std::vector<const double*> fo;
                for (int o : g->units.outer) fo.push_back(g->d_F[o]);
                GEN_HIP(hipMalloc(&g->d_Fo, fo.size() * sizeof(double*)));
                GEN_HIP(hipMemcpy(g->d_Fo, fo.data(), fo.size() * sizeof(double*),
                                  hipMemcpyHostToDevice));
                g->unit_sums = true;
            }
            if (g->tile_b3)
            {
                const uint64_t md = std::max({g->dims[in[0]], g->dims[in[1]], g->dims[in[2]]});
                g->tile_ws_bytes = cptc_tile_operands_bytes(md, R);
                GEN_HIP(hipMalloc(&g->d_tile_ws, g->tile_ws_bytes));
                // compacted split unit images, one per inner slot (the order-3
                // tiles' format)
                const char* ce = std::getenv("GEN_TILE_COMPACT");
                if (!(ce && std::strcmp(ce, "0") == 0))
                    for (int sl = 0; sl < 3; ++sl)
                        GEN_TRY(cptc::build_split_img(g->d_tiles, g->units.nunits, sl, g->uimg[sl], s));
            }
        }
        g->prep_ms[1] = ms_since(t0);
        if (verbose)
            std::printf("[GEN] dense: units=%llu dense_nnz=%llu (%g%% of nnz) cutoff=%d "
                        "prep=%g ms\n",
                        (unsigned long long)g->units.nunits,
                        (unsigned long long)g->units.dense_nnz,
                        100.0 * double(g->units.dense_nnz) / double(g->nnz), g->units.cutoff,
                        g->prep_ms[1]);
    }
    else
    {
        for (int q = 0; q < 3; ++q) g->units.inner[q] = in[q];
    }

    // views: the kernel's (dense elements of the inner modes dropped, rows
    // sorted over the other modes) and the reference layout's segment counts
    t0 = Clock::now();
    g->views.resize(N);
    g->ref_nseg.assign(N, 0);
    for (int n = 0; n < N; ++n)
    {
        const bool in = g->dense && (g->inner_mask & (1u << n));
        GEN_TRY(cptc::work_view_nd_device(N, g->dims.data(), n, g->d_coords, g->d_vals,
                                          in ? g->units.d_is_dense : nullptr, in, g->nnz,
                                          g->views[n], s));
        std::vector<uint64_t> deg(g->dims[n], 0);
        // the degree multiset does not change under relabelling
        const uint32_t* cn = coo->idx + uint64_t(n) * g->nnz;
        for (uint64_t e = 0; e < g->nnz; ++e) ++deg[cn[e]];
        for (uint64_t d : deg) g->ref_nseg[n] += (d + CPTC_SEG - 1) / CPTC_SEG;
        if (verbose)
            std::printf("[GEN] mode %d view: %llu segments (%llu nnz; kernel view %llu nnz in "
                        "%llu segments)\n",
                        n, (unsigned long long)g->ref_nseg[n], (unsigned long long)g->nnz,
                        (unsigned long long)g->views[n].nnz,
                        (unsigned long long)g->views[n].nseg);
    }
    g->prep_ms[2] = ms_since(t0);

    for (int m = 0; m < N; ++m) GEN_TRY(cptc_gram(g->d_F[m], g->dims[m], R, g->d_grams + m * RR, s));
    if (opts->profile)
    {
        g->ev.resize(size_t(2 + 4 * N));
        for (auto& e : g->ev) GEN_HIP(hipEventCreate(&e));
    }
    for (auto& e : g->kev) GEN_HIP(hipEventCreate(&e));
    GEN_HIP(hipStreamSynchronize(s));
#undef GEN_TRY
#undef GEN_HIP
    *handle = g;
    return CPTC_OK;
}

extern "C" int cptc_gen_info_get(void* handle, cptc_gen_info* info)
{
    CPTC_REQUIRE(handle && info, CPTC_ERR_ARG, "cptc_gen_info_get: null argument");
    Gen* g = as_gen(handle);
    std::memset(info, 0, sizeof(*info));
    info->nmodes = g->N;
    for (int m = 0; m < g->N; ++m)
    {
        info->dims[m] = g->dims[m];
        info->nseg[m] = g->ref_nseg[m];
    }
    info->nnz = g->nnz;
    info->R = g->R;
    std::snprintf(info->reorder, sizeof(info->reorder), "%s", g->method.c_str());
    info->reordered = g->rank.empty() ? 0 : 1;
    info->dense_enabled = g->dense ? 1 : 0;
    info->cutoff = g->units.cutoff;
    for (int q = 0; q < 3; ++q) info->inner[q] = g->units.inner[q];
    info->n_units = g->units.nunits;
    info->dense_nnz = g->units.dense_nnz;
    for (int m = 0; m < g->N; ++m) info->kernel_nnz[m] = g->views[m].nnz;
    info->tile_bf16x3 = (g->dense && g->tile_b3) ? 1 : 0;
    for (int sl = 0; sl < 3; ++sl) info->unit_segments[sl] = g->uimg[sl].ready() ? g->uimg[sl].nseg : 0;
    info->unit_sums = g->unit_sums ? 1 : 0;
    info->unit_sums_img = (g->unit_sums && g->d_uimg64) ? 1 : 0;
    for (int q = 0; q < 3; ++q) info->prep_ms[q] = g->prep_ms[q];
    return CPTC_OK;
}

extern "C" int cptc_gen_run(void* handle, int iters, double* fit, double* iprod, double* model2,
                            double* ms_iter)
{
    CPTC_REQUIRE(handle && iters >= 0, CPTC_ERR_ARG, "cptc_gen_run: bad arguments");
    Gen* g = as_gen(handle);
    struct Timing
    {
        Gen* g;
        ~Timing() { g->timing = false; }
    } timing_guard{g};
    g->timing = true;
    // Quiet runs queue every iteration and wait once (ms_iter = GPU time per
    // iteration); verbose or profiled runs wait per iteration for the log
    // line, as the reference does (generic.cu:2174-2230).
    if (!g->opts.verbose && !g->opts.profile)
        return g->run_queued(iters, fit, iprod, model2, ms_iter);
    for (int it = 0; it < iters; ++it)
    {
        const auto t0 = Clock::now();
        double f = 0, ip = 0, m2 = 0;
        CPTC_TRY(g->iterate(&f, &ip, &m2));
        const double ms = ms_since(t0);
        if (fit) fit[it] = f;
        if (iprod) iprod[it] = ip;
        if (model2) model2[it] = m2;
        if (ms_iter) ms_iter[it] = ms;
        if (g->opts.verbose)
            std::printf("[GEN] iter %d/%d time=%g ms iprod=%g model2=%g fit=%g\n", it + 1, iters,
                        ms, ip, m2, f);
    }
    return CPTC_OK;
}

extern "C" int cptc_gen_profile(void* handle, double* out5, int* iters, int reset)
{
    CPTC_REQUIRE(handle && out5, CPTC_ERR_ARG, "cptc_gen_profile: null argument");
    Gen* g = as_gen(handle);
    for (int q = 0; q < 5; ++q) out5[q] = g->prof[q];
    if (iters) *iters = g->prof_iters;
    if (reset)
    {
        for (double& x : g->prof) x = 0.0;
        g->prof_iters = 0;
    }
    return CPTC_OK;
}

extern "C" int cptc_gen_kernel_times(void* handle, double* out16, int* iters, int reset)
{
    CPTC_REQUIRE(handle && out16, CPTC_ERR_ARG, "cptc_gen_kernel_times: null argument");
    Gen* g = as_gen(handle);
    for (int m = 0; m < CPTC_MAX_MODES; ++m)
    {
        out16[m] = g->k_seg[m];
        out16[CPTC_MAX_MODES + m] = g->k_unit[m];
    }
    if (iters) *iters = g->k_iters;
    if (reset)
    {
        for (int m = 0; m < CPTC_MAX_MODES; ++m) g->k_seg[m] = g->k_unit[m] = 0.0;
        g->k_iters = 0;
    }
    return CPTC_OK;
}

extern "C" int cptc_gen_mttkrp(void* handle, int mode, double* host_out)
{
    CPTC_REQUIRE(handle && host_out, CPTC_ERR_ARG, "cptc_gen_mttkrp: null argument");
    Gen* g = as_gen(handle);
    CPTC_REQUIRE(mode >= 0 && mode < g->N, CPTC_ERR_ARG, "cptc_gen_mttkrp: mode %d", mode);
    g->w_dirty = true;
    g->usum_ok = false;
    CPTC_TRY(g->mttkrp(mode));
    CPTC_HIP(hipMemcpyAsync(host_out, g->d_FtV, g->dims[mode] * size_t(g->R) * sizeof(double),
                            hipMemcpyDeviceToHost, g->s));
    CPTC_HIP(hipStreamSynchronize(g->s));
    return CPTC_OK;
}

extern "C" int cptc_gen_factor(void* handle, int mode, double* host_out)
{
    CPTC_REQUIRE(handle && host_out, CPTC_ERR_ARG, "cptc_gen_factor: null argument");
    Gen* g = as_gen(handle);
    CPTC_REQUIRE(mode >= 0 && mode < g->N, CPTC_ERR_ARG, "cptc_gen_factor: mode %d", mode);
    CPTC_HIP(hipMemcpyAsync(host_out, g->d_F[mode], g->dims[mode] * size_t(g->R) * sizeof(double),
                            hipMemcpyDeviceToHost, g->s));
    CPTC_HIP(hipStreamSynchronize(g->s));
    return CPTC_OK;
}

extern "C" int cptc_gen_set_factor(void* handle, int mode, const double* host_in)
{
    CPTC_REQUIRE(handle && host_in, CPTC_ERR_ARG, "cptc_gen_set_factor: null argument");
    Gen* g = as_gen(handle);
    CPTC_REQUIRE(mode >= 0 && mode < g->N, CPTC_ERR_ARG, "cptc_gen_set_factor: mode %d", mode);
    const size_t RR = size_t(g->R) * g->R;
    CPTC_HIP(hipMemcpyAsync(g->d_F[mode], host_in, g->dims[mode] * size_t(g->R) * sizeof(double),
                            hipMemcpyHostToDevice, g->s));
    CPTC_TRY(cptc_gram(g->d_F[mode], g->dims[mode], g->R, g->d_grams + mode * RR, g->s));
    g->w_dirty = true;
    g->usum_ok = false;
    CPTC_HIP(hipStreamSynchronize(g->s));
    return CPTC_OK;
}

extern "C" int cptc_gen_lambda(void* handle, double* host_out)
{
    CPTC_REQUIRE(handle && host_out, CPTC_ERR_ARG, "cptc_gen_lambda: null argument");
    Gen* g = as_gen(handle);
    CPTC_HIP(hipMemcpyAsync(host_out, g->d_lambda, size_t(g->R) * sizeof(double),
                            hipMemcpyDeviceToHost, g->s));
    CPTC_HIP(hipStreamSynchronize(g->s));
    return CPTC_OK;
}

extern "C" int cptc_gen_residual(void* handle, double* res_sq, double* x_sq)
{
    CPTC_REQUIRE(handle, CPTC_ERR_ARG, "cptc_gen_residual: null handle");
    Gen* g = as_gen(handle);
    CPTC_HIP(hipMemsetAsync(g->d_out2, 0, 2 * sizeof(double), g->s));
    CPTC_TRY(cptc_residual_nd(g->N, g->d_coords, g->d_vals, g->nnz, g->F(), g->d_lambda, g->R,
                              g->d_out2, g->s));
    double h[2] = {0, 0};
    CPTC_HIP(hipMemcpyAsync(h, g->d_out2, sizeof(h), hipMemcpyDeviceToHost, g->s));
    CPTC_HIP(hipStreamSynchronize(g->s));
    if (res_sq) *res_sq = h[0];
    if (x_sq) *x_sq = h[1];
    return CPTC_OK;
}

extern "C" int cptc_gen_rank(void* handle, int mode, uint32_t* host_out)
{
    CPTC_REQUIRE(handle && host_out, CPTC_ERR_ARG, "cptc_gen_rank: null argument");
    Gen* g = as_gen(handle);
    CPTC_REQUIRE(mode >= 0 && mode < g->N, CPTC_ERR_ARG, "cptc_gen_rank: mode %d", mode);
    for (uint64_t a = 0; a < g->dims[mode]; ++a)
        host_out[a] = g->rank.empty() ? uint32_t(a) : g->rank[mode][a];
    return CPTC_OK;
}

extern "C" int cptc_gen_coords(void* handle, uint32_t* idx)
{
    CPTC_REQUIRE(handle && idx, CPTC_ERR_ARG, "cptc_gen_coords: null argument");
    Gen* g = as_gen(handle);
    CPTC_HIP(hipMemcpyAsync(idx, g->d_coords, size_t(g->N) * g->nnz * sizeof(uint32_t),
                            hipMemcpyDeviceToHost, g->s));
    CPTC_HIP(hipStreamSynchronize(g->s));
    return CPTC_OK;
}

extern "C" int cptc_gen_view(void* handle, int mode, uint32_t* scoords, double* vals,
                             uint8_t* skip, uint32_t* seg_row, uint32_t* seg_start,
                             uint32_t* seg_cnt, uint8_t* single)
{
    CPTC_REQUIRE(handle, CPTC_ERR_ARG, "cptc_gen_view: null handle");
    Gen* g = as_gen(handle);
    CPTC_REQUIRE(mode >= 0 && mode < g->N, CPTC_ERR_ARG, "cptc_gen_view: mode %d", mode);
    hipStream_t s = g->s;
    // the reference layout, built for this copy (the kernel keeps its own views)
    const bool in = g->dense && (g->inner_mask & (1u << mode));
    cptc::DevViewN v;
    struct VFree
    {
        cptc::DevViewN* v;
        ~VFree() { cptc::free_view(*v); }
    } vfree{&v};
    CPTC_TRY(cptc::view_nd_device(g->N, g->dims.data(), mode, g->d_coords, g->d_vals,
                                  g->dense ? g->units.d_is_dense : nullptr, in, g->nnz, v, s));
    CPTC_REQUIRE(v.nseg == g->ref_nseg[mode], CPTC_ERR_STATE,
                 "cptc_gen_view: %llu segments, expected %llu", (unsigned long long)v.nseg,
                 (unsigned long long)g->ref_nseg[mode]);
    auto get = [&](void* dst, const void* src, size_t bytes) -> int {
        if (!dst || bytes == 0) return CPTC_OK;
        if (!src)
        {
            std::memset(dst, 0, bytes);
            return CPTC_OK;
        }
        CPTC_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s));
        return CPTC_OK;
    };
    CPTC_TRY(get(scoords, v.d_sc, size_t(g->N - 1) * g->nnz * sizeof(uint32_t)));
    CPTC_TRY(get(vals, v.d_vals, g->nnz * sizeof(double)));
    CPTC_TRY(get(skip, v.d_skip, g->nnz));
    CPTC_TRY(get(seg_row, v.d_row, v.nseg * sizeof(uint32_t)));
    CPTC_TRY(get(seg_start, v.d_start, v.nseg * sizeof(uint32_t)));
    CPTC_TRY(get(seg_cnt, v.d_cnt, v.nseg * sizeof(uint32_t)));
    CPTC_TRY(get(single, v.d_single, v.nseg));
    CPTC_HIP(hipStreamSynchronize(s));
    return CPTC_OK;
}

extern "C" int cptc_gen_units(void* handle, uint32_t* unit6, uint32_t* outer_coords,
                              uint32_t* lid, double* val, uint8_t* is_dense)
{
    CPTC_REQUIRE(handle, CPTC_ERR_ARG, "cptc_gen_units: null handle");
    Gen* g = as_gen(handle);
    const cptc::DevUnitsN& u = g->units;
    hipStream_t s = g->s;
    auto get = [&](void* dst, const void* src, size_t bytes) -> int {
        if (!dst || bytes == 0) return CPTC_OK;
        if (!src)
        {
            std::memset(dst, 0, bytes);
            return CPTC_OK;
        }
        CPTC_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s));
        return CPTC_OK;
    };
    CPTC_TRY(get(unit6, u.d_unit6, u.nunits * 6 * sizeof(uint32_t)));
    CPTC_TRY(get(outer_coords, u.d_outer_coords, u.nunits * u.outer.size() * sizeof(uint32_t)));
    CPTC_TRY(get(lid, u.d_lid, u.dense_nnz * sizeof(uint32_t)));
    CPTC_TRY(get(val, u.d_val, u.dense_nnz * sizeof(double)));
    CPTC_TRY(get(is_dense, u.d_is_dense, g->nnz));
    CPTC_HIP(hipStreamSynchronize(s));
    return CPTC_OK;
}

extern "C" int cptc_gen_dump(void* handle, const char* base)
{
    return cptc_gen_dump_ex(handle, base, 0);
}

extern "C" int cptc_gen_dump_ex(void* handle, const char* base, int input_order)
{
    CPTC_REQUIRE(handle && base, CPTC_ERR_ARG, "cptc_gen_dump: null argument");
    Gen* g = as_gen(handle);
    const std::string path = std::string(base) + ".factors.txt";
    FILE* f = std::fopen(path.c_str(), "w");
    CPTC_REQUIRE(f, CPTC_ERR_IO, "cptc_gen_dump: cannot open %s", path.c_str());
    const int R = g->R;
    std::fprintf(f, "# cpTC factor dump (factors are column-normalised; lambda holds the norms)\n");
    if (input_order) std::fprintf(f, "# rows in the input tensor's index order\n");
    std::fprintf(f, "order %d\nrank %d\ndims", g->N, R);
    for (int m = 0; m < g->N; ++m) std::fprintf(f, " %llu", (unsigned long long)g->dims[m]);
    std::fprintf(f, "\n");
    std::vector<double> buf;
    int rc = CPTC_OK;
    for (int m = 0; m < g->N && rc == CPTC_OK; ++m)
    {
        buf.assign(g->dims[m] * R, 0.0);
        rc = cptc_gen_factor(handle, m, buf.data());
        if (rc != CPTC_OK) break;
        std::fprintf(f, "mode %d %llu %d\n", m, (unsigned long long)g->dims[m], R);
        for (uint64_t i = 0; i < g->dims[m]; ++i)
        {
            // row i of the input tensor is row rank[i] of the relabelled factor
            const uint64_t src = (input_order && !g->rank.empty()) ? g->rank[m][i] : i;
            for (int r = 0; r < R; ++r)
                std::fprintf(f, r ? " %.17g" : "%.17g", buf[src * R + r]);
            std::fprintf(f, "\n");
        }
    }
    if (rc == CPTC_OK)
    {
        std::vector<double> lam(R, 1.0);
        rc = cptc_gen_lambda(handle, lam.data());
        std::fprintf(f, "lambda %d\n", R);
        for (int r = 0; r < R; ++r) std::fprintf(f, r ? " %.17g" : "%.17g", lam[r]);
        std::fprintf(f, "\n");
    }
    std::fclose(f);
    return rc;
}

extern "C" int cptc_gen_destroy(void* handle)
{
    delete as_gen(handle);
    return CPTC_OK;
}

// ------------------------------------------------------------- self-test --

namespace {

struct SelfTensor
{
    int dims[4] = {40, 24, 36, 3};
    std::vector<std::vector<uint32_t>> co = std::vector<std::vector<uint32_t>>(4);
    std::vector<double> vals;
    std::vector<std::vector<double>> F;
};

// generic.cu:1389-1441 (two ~half-full 16^3 blocks per outer slice, a
// partial boundary block, 4000 scattered elements; R = 8 factors).
void build_self_tensor(SelfTensor& T, int R)
{
    std::mt19937 gen(1234);
    std::uniform_real_distribution<double> uv(0.0, 1.0);
    const int* dims = T.dims;
    auto push = [&](int i, int j, int k, int l, double v) {
        T.co[0].push_back(uint32_t(i));
        T.co[1].push_back(uint32_t(j));
        T.co[2].push_back(uint32_t(k));
        T.co[3].push_back(uint32_t(l));
        T.vals.push_back(v);
    };
    const int tiles[2][3] = {{0, 0, 0}, {1, 0, 1}};
    for (int l = 0; l < dims[3]; ++l)
        for (int t = 0; t < 2; ++t)
            for (int a = 0; a < 16; ++a)
                for (int b = 0; b < 16; ++b)
                    for (int c = 0; c < 16; ++c)
                        if (uv(gen) < 0.5)
                            push(tiles[t][0] * 16 + a, tiles[t][1] * 16 + b, tiles[t][2] * 16 + c,
                                 l, 1.0 + uv(gen));
    for (int l = 0; l < dims[3]; ++l)
        for (int a = 32; a < dims[0]; ++a)
            for (int b = 16; b < dims[1]; ++b)
                for (int c = 32; c < dims[2]; ++c)
                    if (uv(gen) < 0.6) push(a, b, c, l, 1.0 + uv(gen));
    // the argument evaluation order of this call is the host compiler's
    for (int e = 0; e < 4000; ++e)
        push((int)(uv(gen) * dims[0]) % dims[0], (int)(uv(gen) * dims[1]) % dims[1],
             (int)(uv(gen) * dims[2]) % dims[2], (int)(uv(gen) * dims[3]) % dims[3],
             1.0 + uv(gen));
    T.F.assign(4, {});
    for (int m = 0; m < 4; ++m)
    {
        T.F[m].resize(size_t(dims[m]) * R);
        for (auto& x : T.F[m]) x = uv(gen);
    }
}

}  // namespace

extern "C" int cptc_gen_selftest(int verbose, int* failures)
{
    const int N = 4, R = 8;
    SelfTensor T;
    build_self_tensor(T, R);
    const size_t nnz = T.vals.size();
    if (verbose)
        std::printf("[SELFTEST] N=%d dims=%d,%d,%d,%d nnz=%zu R=%d\n", N, T.dims[0], T.dims[1],
                    T.dims[2], T.dims[3], nnz, R);
    // exact FP64 reference per mode
    std::vector<std::vector<double>> ref(N);
    for (int n = 0; n < N; ++n)
    {
        ref[n].assign(size_t(R) * T.dims[n], 0.0);
        for (size_t e = 0; e < nnz; ++e)
            for (int r = 0; r < R; ++r)
            {
                double q = T.vals[e];
                for (int m = 0; m < N; ++m)
                    if (m != n) q *= T.F[m][size_t(T.co[m][e]) * R + r];
                ref[n][size_t(T.co[n][e]) * R + r] += q;
            }
    }

    hipStream_t s = nullptr;
    CPTC_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    struct Owned
    {
        std::vector<void*> p;
        hipStream_t s = nullptr;
        ~Owned()
        {
            if (s) (void)hipStreamSynchronize(s);
            for (void* x : p) (void)hipFree(x);
            if (s) (void)hipStreamDestroy(s);
        }
    } own;
    own.s = s;
    auto dal = [&](void** d, size_t bytes) -> int {
        CPTC_HIP(hipMalloc(d, bytes));
        own.p.push_back(*d);
        return CPTC_OK;
    };
    uint32_t* d_co = nullptr;
    double* d_va = nullptr;
    double* d_FtV = nullptr;
    int maxd = 0;
    for (int m = 0; m < N; ++m) maxd = std::max(maxd, T.dims[m]);
    CPTC_TRY(dal(reinterpret_cast<void**>(&d_co), size_t(N) * nnz * sizeof(uint32_t)));
    CPTC_TRY(dal(reinterpret_cast<void**>(&d_va), nnz * sizeof(double)));
    CPTC_TRY(dal(reinterpret_cast<void**>(&d_FtV), size_t(maxd) * R * sizeof(double)));
    for (int m = 0; m < N; ++m)
        CPTC_HIP(hipMemcpyAsync(d_co + size_t(m) * nnz, T.co[m].data(), nnz * sizeof(uint32_t),
                                hipMemcpyHostToDevice, s));
    CPTC_HIP(hipMemcpyAsync(d_va, T.vals.data(), nnz * sizeof(double), hipMemcpyHostToDevice, s));
    std::vector<double*> dF(N);
    for (int m = 0; m < N; ++m)
    {
        CPTC_TRY(dal(reinterpret_cast<void**>(&dF[m]), T.F[m].size() * sizeof(double)));
        CPTC_HIP(hipMemcpyAsync(dF[m], T.F[m].data(), T.F[m].size() * sizeof(double),
                                hipMemcpyHostToDevice, s));
    }
    const uint64_t dims64[4] = {40, 24, 36, 3};

    int fails = 0;
    const int inner_sets[4][3] = {{0, 1, 2}, {1, 2, 3}, {0, 1, 3}, {0, 2, 3}};
    for (int iset = 0; iset < 4; ++iset)
        for (int pass = 0; pass < 2; ++pass)
        {
            const int* inner = inner_sets[iset];
            const double thr = (pass == 0) ? 0.0 : 0.01;
            if (verbose)
                std::printf("[SELFTEST] --- inner=(%d,%d,%d) pass %d (%s) ---\n", inner[0],
                            inner[1], inner[2], pass,
                            pass == 0 ? "dense-only" : "mixed dense+FP64");
            cptc::DevUnitsN u;
            struct UFree
            {
                cptc::DevUnitsN* u;
                ~UFree() { cptc::free_units(*u); }
            } ufree{&u};
            CPTC_TRY(cptc::units_nd_device(N, dims64, d_co, d_va, nnz, thr, inner, u, s));
            if (verbose)
                std::printf("[SELFTEST]   units=%llu dense_nnz=%llu (%.1f%%)\n",
                            (unsigned long long)u.nunits, (unsigned long long)u.dense_nnz,
                            100.0 * double(u.dense_nnz) / double(nnz));
            float* d_tiles = nullptr;
            double* d_W = nullptr;
            void* d_ws = nullptr;   // split-bf16 operand images (the driver's kernel)
            size_t ws_bytes = 0;
            const int tsw = cptc::tile_kernel_switch("GEN_TILE_KERNEL");
            const bool b3 = tsw < 0 ? cptc::tile_b3_auto(u.nunits, R) : tsw == 1;
            uint32_t* gorder[3] = {nullptr, nullptr, nullptr};
            uint32_t* ggoff[3] = {nullptr, nullptr, nullptr};
            size_t gn[3] = {0, 0, 0};
            if (u.nunits)
            {
                CPTC_TRY(dal(reinterpret_cast<void**>(&d_tiles), u.nunits * 4096 * sizeof(float)));
                if (b3)
                {
                    ws_bytes = cptc_tile_operands_bytes(
                        uint64_t(std::max({T.dims[inner[0]], T.dims[inner[1]], T.dims[inner[2]]})), R);
                    CPTC_TRY(dal(&d_ws, ws_bytes));
                }
                CPTC_TRY(dal(reinterpret_cast<void**>(&d_W), u.nunits * R * sizeof(double)));
                CPTC_TRY(cptc_units_pack_nd(u.d_unit6, u.nunits, u.d_lid, u.d_val, d_tiles, s));
                const int rcg = build_unit_groups(u, R, s, gorder, ggoff, gn, b3 ? 32 : 16);
                for (int q = 0; q < 3; ++q)
                {
                    own.p.push_back(gorder[q]);
                    own.p.push_back(ggoff[q]);
                }
                CPTC_TRY(rcg);
                const int om = u.outer.empty() ? 0 : u.outer[0];
                CPTC_TRY(cptc_units_weights_nd(u.d_unit6, u.nunits, u.d_outer_coords,
                                               int(u.outer.size()), &om, dF.data(), R, d_W, s));
            }
            for (int ii = 0; ii < 3; ++ii)
            {
                const int n = inner[ii];
                CPTC_HIP(hipMemsetAsync(d_FtV, 0, size_t(maxd) * R * sizeof(double), s));
                if (u.nunits && b3)
                    CPTC_TRY(cptc_mttkrp_units_nd_ws(ii, u.d_unit6, u.nunits, d_tiles, d_W,
                                                     gorder[ii], ggoff[ii], gn[ii],
                                                     dF[inner[0]], dF[inner[1]], dF[inner[2]],
                                                     T.dims[inner[0]], T.dims[inner[1]],
                                                     T.dims[inner[2]], d_FtV, R, d_ws, ws_bytes,
                                                     s));
                else if (u.nunits)
                    CPTC_TRY(cptc_mttkrp_units_nd(ii, u.d_unit6, u.nunits, d_tiles, d_W,
                                                  gorder[ii], ggoff[ii], gn[ii],
                                                  dF[inner[0]], dF[inner[1]], dF[inner[2]],
                                                  T.dims[inner[0]], T.dims[inner[1]],
                                                  T.dims[inner[2]], d_FtV, R, s));
                if (pass == 1)
                {
                    cptc::DevViewN v;
                    struct VFree
                    {
                        cptc::DevViewN* v;
                        ~VFree() { cptc::free_view(*v); }
                    } vfree{&v};
                    CPTC_TRY(cptc::work_view_nd_device(N, dims64, n, d_co, d_va, u.d_is_dense,
                                                       true, nnz, v, s));
                    CPTC_TRY(cptc_mttkrp_seg_nd(N, n, v.d_sc, v.level_modes.data(), v.d_vals,
                                                nullptr, v.nnz, v.d_row, v.d_start, v.d_cnt,
                                                v.d_single, v.nseg, dF.data(), d_FtV, R, s));
                    CPTC_HIP(hipStreamSynchronize(s));
                }
                std::vector<double> got(size_t(R) * T.dims[n]);
                CPTC_HIP(hipMemcpyAsync(got.data(), d_FtV, got.size() * sizeof(double),
                                        hipMemcpyDeviceToHost, s));
                CPTC_HIP(hipStreamSynchronize(s));
                double num = 0.0, den = 0.0;
                for (size_t i = 0; i < got.size(); ++i)
                {
                    const double d = got[i] - ref[n][i];
                    num += d * d;
                    den += ref[n][i] * ref[n][i];
                }
                const double rel = den > 0.0 ? std::sqrt(num / den) : 0.0;
                const bool ok = rel < 2e-3;
                if (verbose)
                    std::printf("[SELFTEST]   mode %d: relative L2 error = %.3e  %s\n", n, rel,
                                ok ? "OK" : "FAIL");
                if (!ok) ++fails;
            }
        }
    if (verbose) std::printf("[SELFTEST] %s (%d failures)\n", fails ? "FAILED" : "PASSED", fails);
    if (failures) *failures = fails;
    return CPTC_OK;
}
