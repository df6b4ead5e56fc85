// CPU oracle for the CP-ALS hot path — TEST INFRASTRUCTURE ONLY (see header).
#include "cptc_oracle.hpp"

#include <algorithm>
#include <cfloat>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <numeric>
#include <random>
#include <stdexcept>

#include <omp.h>

namespace oracle {

namespace {

double now_ms()
{
    return std::chrono::duration<double, std::milli>(
               std::chrono::steady_clock::now().time_since_epoch())
        .count();
}

// tensor.cu:24-37: digits only, no sign; *end = first non-digit.
int parse_int_digits(const char* s, const char** end)
{
    int v = 0;
    const char* p = s;
    while (*p >= '0' && *p <= '9')
    {
        v = v * 10 + (*p - '0');
        ++p;
    }
    *end = p;
    return v;
}

}  // namespace

// ---------------------------------------------------------------------------
// tensor.cu:39-271.  The whole file is held in one NUL-terminated buffer so
// that strtod, which the reference calls on its read buffer, sees the same
// bytes after the line (it skips '\r' and '\n' as whitespace).
// ---------------------------------------------------------------------------
bool load_tns3(const std::string& path, Coo3& out)
{
    FILE* f = std::fopen(path.c_str(), "rb");
    if (!f) return false;
    std::vector<char> buf;
    {
        std::fseek(f, 0, SEEK_END);
        const long sz = std::ftell(f);
        std::fseek(f, 0, SEEK_SET);
        buf.resize(size_t(sz) + 1);
        const size_t got = std::fread(buf.data(), 1, size_t(sz), f);
        buf.resize(got + 1);
        buf[got] = '\0';
    }
    std::fclose(f);
    out = Coo3{};
    size_t mx[3] = {0, 0, 0};
    const char* b = buf.data();
    const size_t n = buf.size() - 1;
    auto ws = [](char c) { return c == ' ' || c == '\t'; };
    auto process = [&](const char* s, size_t len) {
        if (len == 0 || s[0] == '#') return;
        const char* e = s + len;
        const char* p = s;
        const char* end = nullptr;
        int m[3];
        for (int f3 = 0; f3 < 3; ++f3)
        {
            while (p < e && ws(*p)) ++p;
            if (p >= e) return;
            m[f3] = parse_int_digits(p, &end);
            p = end;
        }
        while (p < e && ws(*p)) ++p;
        if (p >= e) return;
        char* endc = nullptr;
        const double v = std::strtod(p, &endc);
        if (endc == p) return;
        const int z[3] = {m[0] > 0 ? m[0] - 1 : 0, m[1] > 0 ? m[1] - 1 : 0,
                          m[2] > 0 ? m[2] - 1 : 0};
        out.m0.push_back(z[0]);
        out.m1.push_back(z[1]);
        out.m2.push_back(z[2]);
        out.val.push_back(v);
        for (int q = 0; q < 3; ++q) mx[q] = std::max(mx[q], size_t(z[q]));
    };
    size_t ls = 0;
    for (size_t i = 0; i < n; ++i)
        if (b[i] == '\n')
        {
            process(b + ls, i - ls);
            ls = i + 1;
        }
    if (ls < n) process(b + ls, n - ls);
    for (int q = 0; q < 3; ++q) out.dims[q] = mx[q] + 1;
    return true;
}

// ---------------------------------------------------------------------------
// cadr.cu:23-66 / 69-81
// ---------------------------------------------------------------------------
void cadr3(const Coo3& t, std::vector<int32_t> perm[3])
{
    const std::vector<int32_t>* cs[3] = {&t.m0, &t.m1, &t.m2};
    for (int m = 0; m < 3; ++m)
    {
        std::vector<size_t> deg(t.dims[m], 0);
        for (int32_t c : *cs[m]) deg[size_t(c)]++;
        std::vector<int> sorted(deg.size());
        std::iota(sorted.begin(), sorted.end(), 0);
        std::sort(sorted.begin(), sorted.end(), [&](int a, int b) { return deg[a] > deg[b]; });
        perm[m].assign(deg.size(), 0);
        for (int nw = 0; nw < int(sorted.size()); ++nw) perm[m][sorted[nw]] = nw;
    }
}

void apply_cadr3(Coo3& t, const std::vector<int32_t> perm[3])
{
    for (size_t e = 0; e < t.nnz(); ++e)
    {
        t.m0[e] = perm[0][t.m0[e]];
        t.m1[e] = perm[1][t.m1[e]];
        t.m2[e] = perm[2][t.m2[e]];
    }
}

// ---------------------------------------------------------------------------
// common.cu:66-123
// ---------------------------------------------------------------------------
void init_factors3(const size_t dims[3], int R, unsigned seed, std::vector<double> F[3])
{
    std::mt19937 gen(seed);
    std::uniform_real_distribution<double> dis(0.0, 1.0);
    for (int m = 0; m < 3; ++m)
    {
        F[m].resize(dims[m] * size_t(R));
        for (auto& x : F[m]) x = dis(gen);
    }
}

// ---------------------------------------------------------------------------
// partition.cu:581-1493
// ---------------------------------------------------------------------------
static int g_num_cus = 256;

void partition3(const Coo3& t, double threshold, Partition3& p)
{
    p = Partition3{};
    for (int m = 0; m < 3; ++m) p.nblk[m] = (t.dims[m] + 15) / 16;
    const size_t nnz = t.nnz();
    if (threshold > 0.0)
    {
        int c = int(4096.0 * threshold);
        p.cutoff = std::min(std::max(c, 1), 4096);
    }
    if (nnz == 0) return;
    std::vector<uint64_t> key(nnz);
    for (size_t e = 0; e < nnz; ++e)
        key[e] = (uint64_t(t.m0[e] / 16) * p.nblk[1] + uint64_t(t.m1[e] / 16)) * p.nblk[2] +
                 uint64_t(t.m2[e] / 16);
    std::vector<uint32_t> order(nnz);
    std::iota(order.begin(), order.end(), 0u);
    std::stable_sort(order.begin(), order.end(),
                     [&](uint32_t a, uint32_t b) { return key[a] < key[b]; });
    // runs of equal block_id
    std::vector<size_t> rs;  // run starts
    std::vector<int> rc;     // run counts
    for (size_t q = 0; q < nnz; ++q)
    {
        if (q == 0 || key[order[q]] != key[order[q - 1]])
        {
            rs.push_back(q);
            rc.push_back(0);
        }
        rc.back()++;
    }
    if (threshold <= 0.0)
    {
        // partition.cu:1030-1098 (rates scaled by the CU count as the reference does)
        const double sm_scale = double(g_num_cus) / 24.0;
        const double rate_wmma = 1.20 / sm_scale;
        const double rate_cuda = 0.688 / sm_scale;
        const double frac_dense = rate_cuda / (rate_wmma + rate_cuda);
        const size_t target = size_t(double(nnz) * frac_dense);
        std::vector<int> cs(rc);
        std::sort(cs.begin(), cs.end(), std::greater<int>());
        size_t acc = 0;
        int cut = 1;
        for (int c : cs)
        {
            acc += size_t(c);
            if (acc >= target)
            {
                cut = c;
                break;
            }
        }
        p.cutoff = cut;
    }
    for (size_t r = 0; r < rs.size(); ++r)
    {
        const bool dense = rc[r] >= p.cutoff;
        const uint64_t bid = key[order[rs[r]]];
        if (dense)
        {
            Tile tl;
            tl.b[2] = int32_t(bid % p.nblk[2]);
            const uint64_t tmp = bid / p.nblk[2];
            tl.b[1] = int32_t(tmp % p.nblk[1]);
            tl.b[0] = int32_t(tmp / p.nblk[1]);
            tl.nnz = rc[r];
            tl.off = p.pool_lid.size();
            p.tiles.push_back(tl);
        }
        for (int q = 0; q < rc[r]; ++q)
        {
            const uint32_t e = order[rs[r] + size_t(q)];
            const int i = t.m0[e], j = t.m1[e], l = t.m2[e];
            if (dense)
            {
                p.pool_lid.push_back(((i % 16) * 16 + (j % 16)) * 16 + (l % 16));
                p.pool_val.push_back(t.val[e]);
            }
            else
            {
                p.sp_i.push_back(uint32_t(i));
                p.sp_j.push_back(uint32_t(j));
                p.sp_k.push_back(uint32_t(l));
                p.sp_val.push_back(t.val[e]);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// partition.cu:1691-1810, 1865-2329
// ---------------------------------------------------------------------------
void views3(const std::vector<uint32_t>& i, const std::vector<uint32_t>& j,
            const std::vector<uint32_t>& k, const std::vector<double>& v, const size_t dims[3],
            View3& out)
{
    out = View3{};
    const size_t nnz = v.size();
    out.nnz = nnz;
    if (nnz == 0) return;
    if (dims[0] >= 32768 || dims[1] >= 32768 || dims[2] >= 32768)
        throw std::runtime_error("views3: dims >= 32768 do not fit the 15-bit packed layout");
    std::vector<uint64_t> packed(nnz);
    for (size_t e = 0; e < nnz; ++e)
        packed[e] = (uint64_t(i[e]) << 30) | (uint64_t(j[e]) << 15) | uint64_t(k[e]);
    for (int mode = 0; mode < 3; ++mode)
    {
        std::vector<uint64_t> key(nnz);
        for (size_t e = 0; e < nnz; ++e)
        {
            const uint64_t a = i[e], b = j[e], c = k[e];
            key[e] = mode == 0 ? (a << 30) | (c << 15) | b
                   : mode == 1 ? (b << 30) | (c << 15) | a
                               : (c << 30) | (b << 15) | a;
        }
        std::vector<uint32_t> ord(nnz);
        std::iota(ord.begin(), ord.end(), 0u);
        std::stable_sort(ord.begin(), ord.end(),
                         [&](uint32_t x, uint32_t y) { return key[x] < key[y]; });
        out.coords[mode].resize(nnz);
        out.vals[mode].resize(nnz);
        for (size_t q = 0; q < nnz; ++q)
        {
            out.coords[mode][q] = packed[ord[q]];
            out.vals[mode][q] = v[ord[q]];
        }
        size_t q = 0;
        while (q < nnz)
        {
            const uint32_t tgt = uint32_t(key[ord[q]] >> 30);
            size_t e = q;
            while (e < nnz && uint32_t(key[ord[e]] >> 30) == tgt) ++e;
            const size_t cnt = e - q;
            for (size_t c = 0; c < cnt; c += 1024)
            {
                out.blk_row[mode].push_back(tgt);
                out.blk_start[mode].push_back(uint32_t(q + c));
                out.blk_cnt[mode].push_back(uint32_t(std::min<size_t>(1024, cnt - c)));
            }
            q = e;
        }
    }
}

void dense_views3(const Partition3& p, const size_t dims[3], View3& out)
{
    std::vector<uint32_t> i, j, k;
    std::vector<double> v;
    for (const Tile& t : p.tiles)
        for (int e = 0; e < t.nnz; ++e)
        {
            const int lid = p.pool_lid[t.off + size_t(e)];
            i.push_back(uint32_t(t.b[0] * 16 + (lid >> 8)));
            j.push_back(uint32_t(t.b[1] * 16 + ((lid >> 4) & 15)));
            k.push_back(uint32_t(t.b[2] * 16 + (lid & 15)));
            v.push_back(p.pool_val[t.off + size_t(e)]);
        }
    views3(i, j, k, v, dims, out);
}

// ---------------------------------------------------------------------------
// sparse.cu:35-64 (decode), 614-711 (segment sum)
// ---------------------------------------------------------------------------
void mttkrp3_view(const View3& v, int mode, const double* A, const double* B, const double* C,
                  int R, double* FtV)
{
    const size_t nseg = v.blk_row[mode].size();
    if (nseg == 0) return;
    const double* F1 = mode == 0 ? B : A;
    const double* F2 = mode == 2 ? B : C;
    // segments of one row are consecutive: group them
    std::vector<size_t> g;
    for (size_t s = 0; s < nseg; ++s)
        if (s == 0 || v.blk_row[mode][s] != v.blk_row[mode][s - 1]) g.push_back(s);
    g.push_back(nseg);
    const uint64_t* co = v.coords[mode].data();
    const double* va = v.vals[mode].data();
    #pragma omp parallel
    {
        std::vector<double> acc(static_cast<size_t>(R));
        #pragma omp for schedule(dynamic, 16)
        for (int64_t gi = 0; gi < int64_t(g.size()) - 1; ++gi)
        {
            for (size_t s = g[gi]; s < g[gi + 1]; ++s)
            {
                std::fill(acc.begin(), acc.end(), 0.0);
                const uint32_t st = v.blk_start[mode][s], cn = v.blk_cnt[mode][s];
                for (uint32_t e = st; e < st + cn; ++e)
                {
                    const uint64_t pc = co[e];
                    const uint32_t ci = uint32_t((pc >> 30) & 0x7FFF);
                    const uint32_t cj = uint32_t((pc >> 15) & 0x7FFF);
                    const uint32_t ck = uint32_t(pc & 0x7FFF);
                    const uint32_t o0 = mode == 0 ? cj : ci;
                    const uint32_t o1 = mode == 2 ? cj : ck;
                    const double* f1 = F1 + size_t(o0) * R;
                    const double* f2 = F2 + size_t(o1) * R;
                    const double x = va[e];
                    for (int r = 0; r < R; ++r) acc[r] += x * f1[r] * f2[r];
                }
                double* out = FtV + size_t(v.blk_row[mode][s]) * R;
                for (int r = 0; r < R; ++r) out[r] += acc[r];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// dense.cu:89-1077, exact FP64
// ---------------------------------------------------------------------------
void mttkrp3_tiles(const Partition3& p, int mode, const double* A, const double* B,
                   const double* C, int R, const size_t dims[3], double* FtV)
{
    const int nt = int(p.tiles.size());
    if (nt == 0) return;
    // rows touched by different tiles collide: accumulate per tile, then add
    // serially in tile order (deterministic)
    std::vector<std::vector<double>> part(static_cast<size_t>(nt));
    #pragma omp parallel
    {
        std::vector<double> T(4096);
        #pragma omp for schedule(dynamic, 4)
        for (int ti = 0; ti < nt; ++ti)
        {
            const Tile& t = p.tiles[ti];
            std::fill(T.begin(), T.end(), 0.0);
            for (int e = 0; e < t.nnz; ++e)
            {
                double x = p.pool_val[t.off + size_t(e)];
                x = std::min(std::max(x, -double(FLT_MAX)), double(FLT_MAX));
                T[size_t(p.pool_lid[t.off + size_t(e)])] = x;
            }
            const int b0 = t.b[0] * 16, b1 = t.b[1] * 16, b2 = t.b[2] * 16;
            std::vector<double>& o = part[ti];
            o.assign(16 * size_t(R), 0.0);
            for (int li = 0; li < 16; ++li)
                for (int lj = 0; lj < 16; ++lj)
                    for (int lk = 0; lk < 16; ++lk)
                    {
                        const double x = T[size_t((li * 16 + lj) * 16 + lk)];
                        if (x == 0.0) continue;
                        const int gi = b0 + li, gj = b1 + lj, gk = b2 + lk;
                        if (size_t(gi) >= dims[0] || size_t(gj) >= dims[1] || size_t(gk) >= dims[2])
                            continue;
                        const double* a = A + size_t(gi) * R;
                        const double* b = B + size_t(gj) * R;
                        const double* c = C + size_t(gk) * R;
                        double* out = &o[size_t(mode == 0 ? li : mode == 1 ? lj : lk) * R];
                        for (int r = 0; r < R; ++r)
                            out[r] += mode == 0 ? x * b[r] * c[r]
                                    : mode == 1 ? x * a[r] * c[r]
                                                : x * a[r] * b[r];
                    }
        }
    }
    for (int ti = 0; ti < nt; ++ti)
    {
        const Tile& t = p.tiles[ti];
        const int base = t.b[mode] * 16;
        for (int l = 0; l < 16; ++l)
        {
            if (size_t(base + l) >= dims[mode]) continue;
            for (int r = 0; r < R; ++r) FtV[size_t(base + l) * R + r] += part[ti][size_t(l) * R + r];
        }
    }
}

void gram(const double* F, size_t rows, int R, double* G)
{
    #pragma omp parallel for schedule(dynamic, 1)
    for (int r = 0; r < R; ++r)
        for (int s = r; s < R; ++s)
        {
            double acc = 0.0;
            for (size_t i = 0; i < rows; ++i) acc += F[i * R + r] * F[i * R + s];
            G[size_t(r) * R + s] = acc;
            G[size_t(s) * R + r] = acc;
        }
}

// ---------------------------------------------------------------------------
// solver.cu:900-1002.  Cyclic Jacobi eigen-decomposition (Golub & Van Loan,
// "Matrix Computations", 4th ed., Alg. 8.5.3); for a symmetric matrix the
// truncated SVD pseudoinverse V diag(1/sigma) U^T equals
// sum_i v_i v_i^T / lambda_i over |lambda_i| > R * ulp(max |lambda|).
// ---------------------------------------------------------------------------
int pinv_sym(const double* Ain, int R, double* Ainv)
{
    const size_t n = size_t(R);
    std::vector<double> a(Ain, Ain + n * n), v(n * n, 0.0);
    for (size_t q = 0; q < n; ++q) v[q * n + q] = 1.0;
    double fro = 0.0;
    for (double x : a) fro += x * x;
    fro = std::sqrt(fro);
    // gesvdj's settings (solver.cu:837-838): at most 15 sweeps, tolerance
    // 1e-14 on the off-diagonal norm relative to the Frobenius norm
    int sweep = 0;
    for (; sweep < 15; ++sweep)
    {
        double off = 0.0;
        for (size_t p = 0; p < n; ++p)
            for (size_t q = p + 1; q < n; ++q) off += a[p * n + q] * a[p * n + q];
        if (std::sqrt(2.0 * off) <= 1e-14 * fro || fro == 0.0) break;
        for (size_t p = 0; p + 1 < n; ++p)
            for (size_t q = p + 1; q < n; ++q)
            {
                const double apq = a[p * n + q];
                if (apq == 0.0) continue;
                const double theta = (a[q * n + q] - a[p * n + p]) / (2.0 * apq);
                const double t = (theta >= 0 ? 1.0 : -1.0) /
                                 (std::fabs(theta) + std::sqrt(theta * theta + 1.0));
                const double c = 1.0 / std::sqrt(t * t + 1.0), s = t * c;
                for (size_t r = 0; r < n; ++r)
                {
                    const double arp = a[r * n + p], arq = a[r * n + q];
                    a[r * n + p] = c * arp - s * arq;
                    a[r * n + q] = s * arp + c * arq;
                }
                for (size_t r = 0; r < n; ++r)
                {
                    const double apr = a[p * n + r], aqr = a[q * n + r];
                    a[p * n + r] = c * apr - s * aqr;
                    a[q * n + r] = s * apr + c * aqr;
                }
                for (size_t r = 0; r < n; ++r)
                {
                    const double vrp = v[r * n + p], vrq = v[r * n + q];
                    v[r * n + p] = c * vrp - s * vrq;
                    v[r * n + q] = s * vrp + c * vrq;
                }
            }
    }
    double smax = 0.0;
    for (size_t q = 0; q < n; ++q) smax = std::max(smax, std::fabs(a[q * n + q]));
    const double tol = double(R) * (std::nextafter(smax, smax + 1.0) - smax);
    std::fill(Ainv, Ainv + n * n, 0.0);
    for (size_t q = 0; q < n; ++q)
    {
        const double lam = a[q * n + q];
        if (!(std::fabs(lam) > tol)) continue;
        const double inv = 1.0 / lam;
        for (size_t r = 0; r < n; ++r)
            for (size_t c = 0; c < n; ++c) Ainv[r * n + c] += v[r * n + q] * inv * v[c * n + q];
    }
    return sweep;
}

// ---------------------------------------------------------------------------
// als.cu:362-821
// ---------------------------------------------------------------------------
namespace {

void mttkrp_all(const Als3Input& in, const Als3State& st, int mode, double* FtV)
{
    const double* A = st.F[0].data();
    const double* B = st.F[1].data();
    const double* C = st.F[2].data();
    if (in.tiles) mttkrp3_tiles(*in.tiles, mode, A, B, C, st.R, st.dims, FtV);
    if (in.residual) mttkrp3_view(*in.residual, mode, A, B, C, st.R, FtV);
    if (in.dense_view) mttkrp3_view(*in.dense_view, mode, A, B, C, st.R, FtV);
}

// update_mode: solve -> divide by lambda -> column norms -> normalise/absorb
// (als.cu:480-517, 308-360)
void update_mode(Als3State& st, int mode, const double* FtF, const double* FtV)
{
    const int R = st.R;
    const size_t dim = st.dims[mode];
    std::vector<double> Ainv(size_t(R) * R);
    pinv_sym(FtF, R, Ainv.data());
    double* F = st.F[mode].data();
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < int64_t(dim); ++i)
    {
        const double* y = FtV + size_t(i) * R;
        double* f = F + size_t(i) * R;
        for (int r = 0; r < R; ++r)
        {
            // column-major GEMM F(R x dim) = Ainv(R x R) * FtV(R x dim)
            double acc = 0.0;
            for (int s = 0; s < R; ++s) acc += Ainv[size_t(s) * R + r] * y[s];
            f[r] = acc / st.lambda[r];
        }
    }
    std::vector<double> nrm(size_t(R), 0.0);
    for (int r = 0; r < R; ++r)
    {
        double acc = 0.0;
        for (size_t i = 0; i < dim; ++i) acc += F[i * R + r] * F[i * R + r];
        nrm[r] = std::sqrt(acc);
    }
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < int64_t(dim); ++i)
        for (int r = 0; r < R; ++r)
        {
            double& x = F[size_t(i) * R + r];
            x = nrm[r] < 1e-14 ? 0.0 : x / nrm[r];
        }
    for (int r = 0; r < R; ++r) st.lambda[r] = nrm[r] < 1e-14 ? 0.0 : st.lambda[r] * nrm[r];
}

}  // namespace

void als3_iterate(const Als3Input& in, Als3State& st, int iters, double* fits, double* ms,
                  double* mttkrp_ms)
{
    const int R = st.R;
    const size_t RR = size_t(R) * R;
    const size_t maxdim = std::max({st.dims[0], st.dims[1], st.dims[2]});
    if (st.lambda.size() != size_t(R)) st.lambda.assign(size_t(R), 1.0);
    std::vector<double> G[3], FtF(RR), FtV(maxdim * R);
    for (auto& g : G) g.resize(RR);
    const double X2 = in.x_sq;
    const double Xn = std::sqrt(X2);
    for (int it = 0; it < iters; ++it)
    {
        const double t0 = now_ms();
        double tm = 0.0;
        for (int mode = 0; mode < 3; ++mode)
        {
            const int p = mode == 0 ? 1 : 0, q = mode == 2 ? 1 : 2;
            gram(st.F[p].data(), st.dims[p], R, G[p].data());
            gram(st.F[q].data(), st.dims[q], R, G[q].data());
            for (size_t x = 0; x < RR; ++x) FtF[x] = G[p][x] * G[q][x];
            const size_t dim = st.dims[mode];
            std::fill(FtV.begin(), FtV.begin() + dim * R, 0.0);
            const double m0 = now_ms();
            mttkrp_all(in, st, mode, FtV.data());
            tm += now_ms() - m0;
            update_mode(st, mode, FtF.data(), FtV.data());
            gram(st.F[mode].data(), dim, R, G[mode].data());
        }
        // Gram fit (als.cu:659-715): FtV still holds mode C's MTTKRP
        double iprod = 0.0;
        for (int r = 0; r < R; ++r)
        {
            double d = 0.0;
            for (size_t i = 0; i < st.dims[2]; ++i) d += st.F[2][i * R + r] * FtV[i * R + r];
            iprod += st.lambda[r] * d;
        }
        double model2 = 0.0;
        for (int r = 0; r < R; ++r)
            for (int s = 0; s < R; ++s)
            {
                const size_t x = size_t(r) * R + s;
                model2 += st.lambda[r] * st.lambda[s] * G[0][x] * G[1][x] * G[2][x];
            }
        const double res = std::max(X2 - 2.0 * iprod + model2, 0.0);
        const double fit = Xn > 0.0 ? 1.0 - std::sqrt(res) / Xn : 0.0;
        if (fits) fits[it] = fit;
        if (ms) ms[it] = now_ms() - t0;
        if (mttkrp_ms) mttkrp_ms[it] = tm;
    }
}

// common.cu:251-342 (p0/p1 split accumulation), 345-439, 442-505, 517-650
void residual3(const Als3Input& in, const Als3State& st, bool with_lambda, double* res_sq,
               double* x_sq)
{
    const int R = st.R;
    const double* A = st.F[0].data();
    const double* B = st.F[1].data();
    const double* C = st.F[2].data();
    const double* lam = st.lambda.data();
    double res = 0.0, xx = 0.0;
    auto one = [&](uint32_t i, uint32_t j, uint32_t k, double v) {
        const double* pa = A + size_t(i) * R;
        const double* pb = B + size_t(j) * R;
        const double* pc = C + size_t(k) * R;
        double p0 = 0.0, p1 = 0.0;
        int r = 0;
        for (; r + 1 < R; r += 2)
        {
            double x0 = pa[r] * pb[r] * pc[r];
            double x1 = pa[r + 1] * pb[r + 1] * pc[r + 1];
            if (with_lambda)
            {
                x0 *= lam[r];
                x1 *= lam[r + 1];
            }
            p0 += x0;
            p1 += x1;
        }
        for (; r < R; ++r)
        {
            double x = pa[r] * pb[r] * pc[r];
            if (with_lambda) x *= lam[r];
            p0 += x;
        }
        const double d = v - (p0 + p1);
        res += d * d;
        xx += v * v;
    };
    for (const View3* vw : {in.residual, in.dense_view})
    {
        if (!vw || vw->nnz == 0) continue;
        for (size_t e = 0; e < vw->nnz; ++e)
        {
            const uint64_t pc = vw->coords[0][e];
            one(uint32_t((pc >> 30) & 0x7FFF), uint32_t((pc >> 15) & 0x7FFF),
                uint32_t(pc & 0x7FFF), vw->vals[0][e]);
        }
    }
    if (in.tiles)
        for (const Tile& t : in.tiles->tiles)
            for (int e = 0; e < t.nnz; ++e)
            {
                const int lid = in.tiles->pool_lid[t.off + size_t(e)];
                one(uint32_t(t.b[0] * 16 + (lid >> 8)), uint32_t(t.b[1] * 16 + ((lid >> 4) & 15)),
                    uint32_t(t.b[2] * 16 + (lid & 15)), in.tiles->pool_val[t.off + size_t(e)]);
            }
    *res_sq = res;
    *x_sq = xx;
}

void set_num_cus(int n) { g_num_cus = n > 0 ? n : 256; }

// ---------------------------------------------------------------------------
// sgd.cu:51-288 (CP-SGD kernels), sequential restatement
// ---------------------------------------------------------------------------
std::vector<uint32_t> sgd3_sample(uint64_t seed, uint32_t batch, uint64_t nnz)
{
    // sgd.cu:195-215
    std::vector<uint32_t> idx(batch);
    for (uint32_t b = 0; b < batch; ++b)
    {
        uint64_t x = seed + uint64_t(b) * 0x9E3779B97F4A7C15ull;
        x ^= x >> 30;
        x *= 0xBF58476D1CE4E5B9ull;
        x ^= x >> 27;
        x *= 0x94D049BB133111EBull;
        x ^= x >> 31;
        idx[b] = uint32_t(x % nnz);
    }
    return idx;
}

namespace {
double sgd3_xhat(const double* a, const double* b, const double* c, const double* lambda, int R)
{
    double x = 0.0;
    for (int r = 0; r < R; ++r) x += lambda[r] * a[r] * b[r] * c[r];
    return x;
}
}  // namespace

void sgd3_step(const std::vector<uint64_t>& coords, const std::vector<double>& vals,
               const std::vector<uint32_t>& idx, double* A, double* B, double* C,
               const double* lambda, int R, double gamma)
{
    // sgd.cu:51-130: read the three rows, xhat, e, then the three steps from
    // the values read
    const size_t nr = static_cast<size_t>(R);
    std::vector<double> a(nr), b(nr), c(nr);
    for (uint32_t e : idx)
    {
        const uint64_t pc = coords[e];
        double* pa = A + size_t((pc >> 30) & 0x7FFF) * R;
        double* pb = B + size_t((pc >> 15) & 0x7FFF) * R;
        double* pcc = C + size_t(pc & 0x7FFF) * R;
        std::copy(pa, pa + R, a.begin());
        std::copy(pb, pb + R, b.begin());
        std::copy(pcc, pcc + R, c.begin());
        const double err = vals[e] - sgd3_xhat(a.data(), b.data(), c.data(), lambda, R);
        for (int r = 0; r < R; ++r)
        {
            pa[r] += gamma * err * b[r] * c[r];
            pb[r] += gamma * err * a[r] * c[r];
            pcc[r] += gamma * err * a[r] * b[r];
        }
    }
}

void sgd3_normalize(double* F, size_t rows, int R, double* lambda)
{
    // sgd.cu:219-288
    for (int r = 0; r < R; ++r)
    {
        double acc = 0.0;
        for (size_t i = 0; i < rows; ++i) acc += F[i * R + r] * F[i * R + r];
        const double n = std::sqrt(acc);
        for (size_t i = 0; i < rows; ++i) F[i * R + r] = n < 1e-14 ? 0.0 : F[i * R + r] / n;
        lambda[r] = n < 1e-14 ? 0.0 : n;
    }
}

double sgd3_loss(const std::vector<uint64_t>& coords, const std::vector<double>& vals,
                 const std::vector<uint32_t>& idx, const double* A, const double* B,
                 const double* C, const double* lambda, int R)
{
    // sgd.cu:133-192
    double s = 0.0;
    for (uint32_t e : idx)
    {
        const uint64_t pc = coords[e];
        const double x = sgd3_xhat(A + size_t((pc >> 30) & 0x7FFF) * R,
                                   B + size_t((pc >> 15) & 0x7FFF) * R,
                                   C + size_t(pc & 0x7FFF) * R, lambda, R);
        s += (vals[e] - x) * (vals[e] - x);
    }
    return s;
}

}  // namespace oracle
