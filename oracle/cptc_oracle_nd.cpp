// CPU oracle for the generic N-order CP-ALS path — TEST INFRASTRUCTURE ONLY
// (see cptc_oracle_nd.hpp).  Follows src/generic.cu of the reference.
#include "cptc_oracle_nd.hpp"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <numeric>
#include <random>
#include <stdexcept>
#include <unordered_map>

#include "cptc_oracle.hpp"

namespace oracle {

// generic.cu:39-45
uint64_t splitbit_hash(uint64_t x)
{
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

namespace {

void relabel(CooN& t, const std::vector<std::vector<uint32_t>>& rank)
{
    for (int m = 0; m < t.N; ++m)
        for (auto& x : t.c[m]) x = rank[m][x];
}

// generic.cu:1201-1230 (the sampled fill probe of reorder=auto)
double probe_fill(const CooN& t, const std::vector<std::vector<uint32_t>>* rk)
{
    const size_t nnz = t.nnz();
    const size_t budget = 2000000;
    const size_t st = (nnz > budget) ? (nnz / budget) : 1;
    const uint64_t nbj = (t.dims[1] + 15) / 16;
    const uint64_t nbk = (t.dims[2] + 15) / 16;
    auto co = [&](int m, size_t e) -> uint64_t {
        return rk ? (*rk)[m][t.c[m][e]] : t.c[m][e];
    };
    std::unordered_map<uint64_t, uint32_t> cnt;
    for (size_t e = 0; e < nnz; e += st)
    {
        const uint64_t a = co(0, e), b = co(1, e), c = co(2, e);
        const uint64_t tile = ((a / 16) * nbj + b / 16) * nbk + c / 16;
        uint64_t o = 0;
        for (int m = 3; m < t.N; ++m) o = o * 1000003ull + co(m, e);
        ++cnt[splitbit_hash(tile ^ (o * 0x9E3779B97F4A7C15ull))];
    }
    long long tiles = 0, in = 0;
    for (const auto& kv : cnt)
        if ((long long)kv.second * (long long)st >= 122)
        {
            ++tiles;
            in += (long long)kv.second * (long long)st;
        }
    return tiles ? double(in) / (double(tiles) * 4096.0) : 0.0;
}

}  // namespace

// generic.cu:1180-1376
void reorder_nd(CooN& t, const std::string& how, int rounds, size_t sample_budget,
                std::vector<std::vector<uint32_t>>& rank_out)
{
    const int N = t.N;
    const size_t nnz = t.nnz();
    rank_out.clear();
    std::vector<std::vector<uint32_t>> rank(N);
    for (int m = 0; m < N; ++m)
    {
        rank[m].resize(t.dims[m]);
        std::iota(rank[m].begin(), rank[m].end(), 0u);
    }
    if (how == "auto")
    {
        const double f_raw = probe_fill(t, nullptr);
        if (f_raw < 0.02) return;
        std::vector<std::vector<uint32_t>> rk_try;
        reorder_nd(t, "hits", rounds, sample_budget, rk_try);
        bool ok = int(rk_try.size()) == N;
        // the probe maps the already relabelled coordinates once more
        // (generic.cu:1255: fill_of(rk_try, true) after the relabel)
        const double f_hits = ok ? probe_fill(t, &rk_try) : 0.0;
        if (ok && f_hits >= 0.11)
        {
            rank_out = rk_try;
            return;
        }
        for (int m = 0; m < N; ++m)
        {
            std::vector<uint32_t> inv(t.dims[m]);
            for (size_t a = 0; a < t.dims[m]; ++a) inv[rk_try[m][a]] = uint32_t(a);
            for (auto& x : t.c[m]) x = inv[x];
        }
        return;
    }
    if (how == "hits")
    {
        const size_t stride =
            (nnz > sample_budget && sample_budget > 0) ? (nnz / sample_budget) : 1;
        std::vector<std::vector<double>> s(N), ns(N);
        for (int m = 0; m < N; ++m) s[m].assign(t.dims[m], 1.0);
        for (int it = 0; it < rounds; ++it)
        {
            for (int m = 0; m < N; ++m) ns[m].assign(t.dims[m], 0.0);
            for (size_t e = 0; e < nnz; e += stride)
                for (int m = 0; m < N; ++m)
                {
                    double p = 1.0;
                    for (int q = 0; q < N; ++q)
                        if (q != m) p *= s[q][t.c[q][e]];
                    ns[m][t.c[m][e]] += p;
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
        for (int m = 0; m < N; ++m)
        {
            std::vector<uint32_t> ord(t.dims[m]);
            std::iota(ord.begin(), ord.end(), 0u);
            std::sort(ord.begin(), ord.end(), [&](uint32_t a, uint32_t b) {
                const double sa = s[m][a], sb = s[m][b];
                return (sa != sb) ? (sa > sb) : (a < b);
            });
            for (size_t i = 0; i < t.dims[m]; ++i) rank[m][ord[i]] = uint32_t(i);
        }
    }
    else if (how == "cadr")
    {
        for (int m = 0; m < N; ++m)
        {
            std::vector<uint32_t> deg(t.dims[m], 0);
            for (size_t e = 0; e < nnz; ++e) ++deg[t.c[m][e]];
            std::vector<uint32_t> ord(t.dims[m]);
            std::iota(ord.begin(), ord.end(), 0u);
            std::sort(ord.begin(), ord.end(), [&](uint32_t a, uint32_t b) {
                return deg[a] != deg[b] ? deg[a] > deg[b] : a < b;
            });
            for (size_t i = 0; i < t.dims[m]; ++i) rank[m][ord[i]] = uint32_t(i);
        }
    }
    else
    {
        return;  // none
    }
    relabel(t, rank);
    rank_out = rank;
}

// generic.cu:578-725
void dense_nd(const CooN& t, double threshold, const int inner[3], UnitsN& u)
{
    u = UnitsN{};
    const int N = t.N;
    const size_t nnz = t.nnz();
    u.cutoff = int(4096.0 * threshold);
    for (int s = 0; s < 3; ++s) u.inner[s] = inner[s];
    for (int m = 0; m < N; ++m)
        if (m != inner[0] && m != inner[1] && m != inner[2]) u.outer.push_back(m);
    const auto& c0 = t.c[inner[0]];
    const auto& c1 = t.c[inner[1]];
    const auto& c2 = t.c[inner[2]];
    std::vector<uint64_t> key(nnz);
    std::unordered_map<uint64_t, uint32_t> cnt;
    for (size_t e = 0; e < nnz; ++e)
    {
        const uint32_t a = c0[e], b = c1[e], c = c2[e];
        uint64_t o = 0;
        for (int m : u.outer) o = o * 1000003ull + t.c[m][e];
        const uint64_t tile =
            (uint64_t(a / 16) << 40) | (uint64_t(b / 16) << 20) | uint64_t(c / 16);
        key[e] = splitbit_hash(tile ^ (o * 0x9E3779B97F4A7C15ull));
        ++cnt[key[e]];
    }
    std::unordered_map<uint64_t, uint32_t> index;
    std::vector<uint32_t> nn;
    for (size_t e = 0; e < nnz; ++e)
    {
        if (cnt[key[e]] < uint32_t(u.cutoff)) continue;
        if (index.count(key[e])) continue;
        index[key[e]] = uint32_t(nn.size());
        nn.push_back(0);
        u.unit6.insert(u.unit6.end(), {c0[e] / 16, c1[e] / 16, c2[e] / 16, 0u, 0u,
                                       uint32_t((nn.size() - 1) * size_t(N - 3))});
        for (int m : u.outer) u.outer_coords.push_back(t.c[m][e]);
    }
    u.is_dense.assign(nnz, 0);
    if (nn.empty()) return;
    for (size_t e = 0; e < nnz; ++e)
    {
        auto it = index.find(key[e]);
        if (it != index.end()) ++nn[it->second];
    }
    std::vector<uint32_t> cur(nn.size());
    uint32_t off = 0;
    for (size_t k = 0; k < nn.size(); ++k)
    {
        u.unit6[6 * k + 3] = nn[k];
        u.unit6[6 * k + 4] = off;
        cur[k] = off;
        off += nn[k];
    }
    u.lid.resize(off);
    u.val.resize(off);
    for (size_t e = 0; e < nnz; ++e)
    {
        auto it = index.find(key[e]);
        if (it == index.end()) continue;
        const uint32_t k = it->second;
        u.lid[cur[k]] = (c0[e] % 16) * 256 + (c1[e] % 16) * 16 + (c2[e] % 16);
        u.val[cur[k]] = t.val[e];
        ++cur[k];
        u.is_dense[e] = 1;
    }
}

// generic.cu:1848-1958
void views_nd(const CooN& t, const std::vector<uint8_t>& is_dense, unsigned force_accumulate,
              ViewN& v)
{
    const int N = t.N;
    const size_t nnz = t.nnz();
    v = ViewN{};
    v.sc.resize(N);
    v.sv.resize(N);
    v.skip.resize(N);
    v.row.resize(N);
    v.start.resize(N);
    v.cnt.resize(N);
    v.single.resize(N);
    for (int n = 0; n < N; ++n)
    {
        const size_t dim = t.dims[n];
        std::vector<size_t> st(dim + 1, 0);
        for (size_t e = 0; e < nnz; ++e) ++st[size_t(t.c[n][e]) + 1];
        for (size_t i = 1; i <= dim; ++i) st[i] += st[i - 1];
        std::vector<size_t> cursor(st.begin(), st.end() - 1);
        std::vector<uint32_t> order(nnz);
        for (size_t e = 0; e < nnz; ++e) order[cursor[t.c[n][e]]++] = uint32_t(e);
        v.sc[n].resize(size_t(N - 1) * nnz);
        v.sv[n].resize(nnz);
        v.skip[n].assign(nnz, 0);
        for (size_t i = 0; i < nnz; ++i)
        {
            const uint32_t e = order[i];
            v.sv[n][i] = t.val[e];
            if (!is_dense.empty()) v.skip[n][i] = is_dense[e];
            int q = 0;
            for (int m = 0; m < N; ++m)
            {
                if (m == n) continue;
                v.sc[n][size_t(q) * nnz + i] = t.c[m][e];
                ++q;
            }
        }
        for (size_t r = 0; r < dim; ++r)
        {
            const size_t rs = st[r], re = st[r + 1];
            const size_t nseg = (re > rs) ? (re - rs + 1023) / 1024 : 0;
            for (size_t s = rs; s < re; s += 1024)
            {
                v.row[n].push_back(uint32_t(r));
                v.start[n].push_back(uint32_t(s));
                v.cnt[n].push_back(uint32_t(std::min<size_t>(1024, re - s)));
                v.single[n].push_back(nseg == 1 ? 1 : 0);
            }
        }
        if (force_accumulate & (1u << n))
            for (auto& s8 : v.single[n]) s8 = 0;
    }
}

// generic.cu:271-343
void mttkrp_seg_nd(const CooN& t, const ViewN& v, int n, bool use_skip,
                   const std::vector<std::vector<double>>& F, int R, double* FtV)
{
    const int N = t.N;
    const size_t nnz = t.nnz();
    // OpenMP over rows: a row's segments are consecutive and stay with one
    // thread in view order, so every output entry sees the serial sequence
    const size_t nseg = v.row[n].size();
    std::vector<size_t> grp;
    for (size_t s = 0; s < nseg; ++s)
        if (s == 0 || v.row[n][s] != v.row[n][s - 1]) grp.push_back(s);
    grp.push_back(nseg);
    const size_t ngrp = grp.size() - 1;
#pragma omp parallel
    {
    std::vector<double> acc(static_cast<size_t>(R));
#pragma omp for schedule(dynamic, 16)
    for (size_t gi = 0; gi < ngrp; ++gi)
    for (size_t s = grp[gi]; s < grp[gi + 1]; ++s)
    {
        std::fill(acc.begin(), acc.end(), 0.0);
        for (uint32_t e = v.start[n][s]; e < v.start[n][s] + v.cnt[n][s]; ++e)
        {
            if (use_skip && v.skip[n][e]) continue;
            for (int r = 0; r < R; ++r)
            {
                double prod = v.sv[n][e];
                int q = 0;
                for (int m = 0; m < N; ++m)
                {
                    if (m == n) continue;
                    prod *= F[m][size_t(v.sc[n][size_t(q) * nnz + e]) * R + r];
                    ++q;
                }
                acc[r] += prod;
            }
        }
        double* out = FtV + size_t(v.row[n][s]) * R;
        for (int r = 0; r < R; ++r)
        {
            if (v.single[n][s])
                out[r] = acc[r];
            else
                out[r] += acc[r];
        }
    }
    }
}

// generic.cu:429-561, exact FP64
void mttkrp_units_nd(const CooN& t, const UnitsN& u, int n,
                     const std::vector<std::vector<double>>& F, int R, double* FtV)
{
    int sl = -1;
    for (int x = 0; x < 3; ++x)
        if (u.inner[x] == n) sl = x;
    if (sl < 0) throw std::runtime_error("mttkrp_units_nd: inner modes only");
    // slots: sl = target, p = contracted, q = sliced (generic.cu:500-540)
    const int p = (sl + 1) % 3, q = (sl + 2) % 3;
    const int mp = u.inner[p], mq = u.inner[q];
    const int N = t.N;
    // OpenMP over units: each unit's 16 x R contribution is computed into its
    // own buffer slot in parallel, then the slots are added to FtV in unit
    // order, so every output entry sees the serial sequence.  Chunks of
    // units bound the buffer.
    constexpr size_t CHUNK = 4096;
    const size_t RU = 16 * static_cast<size_t>(R);
    std::vector<double> part(CHUNK * RU);
    for (size_t c0 = 0; c0 < u.n_units(); c0 += CHUNK)
    {
    const size_t c1 = std::min(u.n_units(), c0 + CHUNK);
#pragma omp parallel
    {
    std::vector<double> T(4096), w(static_cast<size_t>(R));
#pragma omp for schedule(dynamic, 8)
    for (size_t k = c0; k < c1; ++k)
    {
        const uint32_t* U = &u.unit6[6 * k];
        double* acc = &part[(k - c0) * RU];
        std::fill(T.begin(), T.end(), 0.0);
        for (uint32_t e = 0; e < U[3]; ++e) T[u.lid[U[4] + e]] += u.val[U[4] + e];
        std::fill(w.begin(), w.end(), 1.0);
        for (int oq = 0; oq < N - 3; ++oq)
        {
            const uint32_t c = u.outer_coords[U[5] + oq];
            for (int r = 0; r < R; ++r) w[r] *= F[u.outer[oq]][size_t(c) * R + r];
        }
        std::fill(acc, acc + RU, 0.0);
        const int base[3] = {int(U[0]) * 16, int(U[1]) * 16, int(U[2]) * 16};
        for (int lt = 0; lt < 16; ++lt)
            for (int lq = 0; lq < 16; ++lq)
            {
                if (base[q] + lq >= int(t.dims[mq])) continue;
                for (int r = 0; r < R; ++r)
                {
                    double g = 0.0;
                    for (int lp = 0; lp < 16; ++lp)
                    {
                        if (base[p] + lp >= int(t.dims[mp])) continue;
                        int loc[3];
                        loc[sl] = lt;
                        loc[p] = lp;
                        loc[q] = lq;
                        const double x = T[size_t(loc[0] * 256 + loc[1] * 16 + loc[2])];
                        if (x != 0.0) g += x * F[mp][size_t(base[p] + lp) * R + r];
                    }
                    acc[size_t(lt) * R + r] += g * F[mq][size_t(base[q] + lq) * R + r] * w[r];
                }
            }
    }
    }
    for (size_t k = c0; k < c1; ++k)
    {
        const uint32_t* U = &u.unit6[6 * k];
        const double* acc = &part[(k - c0) * RU];
        const int b0 = int(U[sl]) * 16;
        for (int lt = 0; lt < 16; ++lt)
        {
            const int row = b0 + lt;
            if (row >= int(t.dims[n])) continue;
            for (int r = 0; r < R; ++r) FtV[size_t(row) * R + r] += acc[size_t(lt) * R + r];
        }
    }
    }
}

// generic.cu:746-819
void chol_solve_nd(const double* FtF, const double* FtV, double* F, size_t dim, int R)
{
    std::vector<double> L(size_t(R) * R, 0.0);
    double tr = 0.0;
    for (int i = 0; i < R; ++i) tr += FtF[i * R + i];
    const double eps = 1e-12 * ((tr > 0.0) ? tr / double(R) : 1.0) + 1e-300;
    for (int i = 0; i < R; ++i)
        for (int j = 0; j <= i; ++j)
        {
            double s = FtF[i * R + j];
            if (i == j) s += eps;
            for (int k = 0; k < j; ++k) s -= L[i * R + k] * L[j * R + k];
            if (i == j)
                L[i * R + j] = (s > 0.0) ? std::sqrt(s) : std::sqrt(eps);
            else
                L[i * R + j] = s / L[j * R + j];
        }
    std::vector<double> y(static_cast<size_t>(R)), x(static_cast<size_t>(R));
    for (size_t row = 0; row < dim; ++row)
    {
        const double* b = FtV + row * R;
        for (int i = 0; i < R; ++i)
        {
            double s = b[i];
            for (int k = 0; k < i; ++k) s -= L[i * R + k] * y[k];
            y[i] = s / L[i * R + i];
        }
        for (int i = R - 1; i >= 0; --i)
        {
            double s = y[i];
            for (int k = i + 1; k < R; ++k) s -= L[k * R + i] * x[k];
            x[i] = s / L[i * R + i];
        }
        for (int i = 0; i < R; ++i) F[row * R + i] = x[i];
    }
}

// generic.cu:1639-2366
void als_nd(const CooN& t, const std::vector<std::vector<uint32_t>>& rank, const AlsNOpts& o,
            int iters, AlsNState& st)
{
    const int N = t.N;
    const int R = o.R;
    const size_t RR = size_t(R) * R;
    st = AlsNState{};
    st.F.resize(N);
    std::mt19937 gen(o.seed);
    std::uniform_real_distribution<double> dis(0.0, 1.0);
    for (int m = 0; m < N; ++m)
    {
        const size_t dim = t.dims[m];
        std::vector<double> u(dim * R);
        for (auto& x : u) x = dis(gen);
        st.F[m].assign(dim * R, 0.0);
        const bool has = m < int(rank.size()) && rank[m].size() == dim;
        for (size_t a = 0; a < dim; ++a)
        {
            const size_t nw = has ? rank[m][a] : a;
            for (int r = 0; r < R; ++r) st.F[m][nw * R + r] = u[a * R + r];
        }
    }
    st.lambda.assign(size_t(R), 1.0);
    UnitsN units;
    bool enabled = false;
    unsigned inner_mask = 0;
    for (int s = 0; s < 3; ++s) inner_mask |= 1u << o.inner[s];
    if (o.dense && N >= 4 && o.threshold > 0.0)
    {
        dense_nd(t, o.threshold, o.inner, units);
        enabled = units.n_units() > 0;
    }
    ViewN v;
    views_nd(t, enabled ? units.is_dense : std::vector<uint8_t>(), enabled ? inner_mask : 0u, v);
    std::vector<std::vector<double>> G(N, std::vector<double>(RR));
    for (int m = 0; m < N; ++m) gram(st.F[m].data(), t.dims[m], R, G[m].data());
    double X2 = 0.0;
    for (double x : t.val) X2 += x * x;
    const double Xn = std::sqrt(X2);
    size_t maxdim = 0;
    for (auto d : t.dims) maxdim = std::max(maxdim, d);
    std::vector<double> FtF(RR), FtV(maxdim * R), Ainv(RR);
    for (int it = 0; it < iters; ++it)
    {
        const auto t_it = std::chrono::steady_clock::now();
        for (int n = 0; n < N; ++n)
        {
            std::fill(FtF.begin(), FtF.end(), 1.0);
            for (int m = 0; m < N; ++m)
                if (m != n)
                    for (size_t x = 0; x < RR; ++x) FtF[x] *= G[m][x];
            const size_t dim = t.dims[n];
            std::fill(FtV.begin(), FtV.begin() + dim * R, 0.0);
            const bool inner = enabled && (inner_mask & (1u << n));
            if (inner) mttkrp_units_nd(t, units, n, st.F, R, FtV.data());
            mttkrp_seg_nd(t, v, n, inner, st.F, R, FtV.data());
            if (o.svd)
            {
                pinv_sym(FtF.data(), R, Ainv.data());
                for (size_t i = 0; i < dim; ++i)
                    for (int r = 0; r < R; ++r)
                    {
                        double acc = 0.0;
                        for (int s = 0; s < R; ++s) acc += Ainv[size_t(s) * R + r] * FtV[i * R + s];
                        st.F[n][i * R + r] = acc;
                    }
            }
            else
            {
                chol_solve_nd(FtF.data(), FtV.data(), st.F[n].data(), dim, R);
            }
            for (int r = 0; r < R; ++r)
            {
                double acc = 0.0;
                for (size_t i = 0; i < dim; ++i) acc += st.F[n][i * R + r] * st.F[n][i * R + r];
                double nr = std::sqrt(acc);
                if (!std::isfinite(nr) || nr < 1e-14) nr = 1.0;
                for (size_t i = 0; i < dim; ++i) st.F[n][i * R + r] /= nr;
                st.lambda[r] = nr;
            }
            gram(st.F[n].data(), dim, R, G[n].data());
        }
        double model2 = 0.0;
        for (size_t x = 0; x < RR; ++x)
        {
            double val = st.lambda[x / R] * st.lambda[x % R];
            for (int m = 0; m < N; ++m) val *= G[m][x];
            model2 += val;
        }
        double iprod = 0.0;
        const int last = N - 1;
        for (int r = 0; r < R; ++r)
        {
            double d = 0.0;
            for (size_t i = 0; i < t.dims[last]; ++i) d += st.F[last][i * R + r] * FtV[i * R + r];
            iprod += st.lambda[r] * d;
        }
        const double res = std::max(X2 - 2.0 * iprod + model2, 0.0);
        st.fits.push_back(Xn > 0.0 ? 1.0 - std::sqrt(res) / Xn : 0.0);
        st.iprod.push_back(iprod);
        st.model2.push_back(model2);
        st.ms.push_back(
            std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t_it)
                .count());
    }
}

// generic.cu:936-967
double residual_nd(const CooN& t, const std::vector<std::vector<double>>& F,
                   const std::vector<double>& lambda, int R)
{
    double res = 0.0;
    for (size_t e = 0; e < t.nnz(); ++e)
    {
        double xhat = 0.0;
        for (int r = 0; r < R; ++r)
        {
            double prod = lambda[r];
            for (int m = 0; m < t.N; ++m) prod *= F[m][size_t(t.c[m][e]) * R + r];
            xhat += prod;
        }
        const double d = t.val[e] - xhat;
        res += d * d;
    }
    return res;
}

// generic.cu:1389-1441
void selftest_tensor(CooN& t, std::vector<std::vector<double>>& F)
{
    const int dims[4] = {40, 24, 36, 3};
    const int R = 8;
    t = CooN{};
    t.N = 4;
    t.dims.assign(dims, dims + 4);
    t.c.assign(4, {});
    std::mt19937 gen(1234);
    std::uniform_real_distribution<double> uv(0.0, 1.0);
    auto push = [&](int i, int j, int k, int l, double v) {
        t.c[0].push_back(uint32_t(i));
        t.c[1].push_back(uint32_t(j));
        t.c[2].push_back(uint32_t(k));
        t.c[3].push_back(uint32_t(l));
        t.val.push_back(v);
    };
    const int tiles[2][3] = {{0, 0, 0}, {1, 0, 1}};
    for (int l = 0; l < dims[3]; ++l)
        for (int tt = 0; tt < 2; ++tt)
            for (int a = 0; a < 16; ++a)
                for (int b = 0; b < 16; ++b)
                    for (int c = 0; c < 16; ++c)
                        if (uv(gen) < 0.5)
                            push(tiles[tt][0] * 16 + a, tiles[tt][1] * 16 + b,
                                 tiles[tt][2] * 16 + c, l, 1.0 + uv(gen));
    for (int l = 0; l < dims[3]; ++l)
        for (int a = 32; a < dims[0]; ++a)
            for (int b = 16; b < dims[1]; ++b)
                for (int c = 32; c < dims[2]; ++c)
                    if (uv(gen) < 0.6) push(a, b, c, l, 1.0 + uv(gen));
    // the argument evaluation order of this call is the host compiler's (g++
    // here, as in the reference's nvcc host pass)
    for (int e = 0; e < 4000; ++e)
        push((int)(uv(gen) * dims[0]) % dims[0], (int)(uv(gen) * dims[1]) % dims[1],
             (int)(uv(gen) * dims[2]) % dims[2], (int)(uv(gen) * dims[3]) % dims[3],
             1.0 + uv(gen));
    F.assign(4, {});
    for (int m = 0; m < 4; ++m)
    {
        F[m].resize(size_t(dims[m]) * R);
        for (auto& x : F[m]) x = uv(gen);
    }
}

}  // namespace oracle
