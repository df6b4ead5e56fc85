// `.tns` COO text ingest and export.
//
// Two parsers with the reference's two sets of semantics:
//   * order 3 (tensor.cu:24-271): fields bounded by the line, index m ->
//     (m > 0 ? m - 1 : 0), dims = max(0-based) + 1;
//   * N-order (generic.cu:971-1155): order from the first numeric line,
//     dims = max(1-based) or 1, lines longer than 4 MiB rejected.
// In both, strtod reads the value from the file bytes themselves, so (as in
// the reference) it skips '\r' / '\n' when a line ends right after its
// indices.
// The file is memory-mapped (read-only, with zero pages after its end, so
// every scan and strtod stops at a NUL) and parsed in two OpenMP passes over
// newline-aligned chunks: count the lines of each chunk, then parse each
// chunk straight into the output arrays at its prefix offset (lines that do
// not parse leave gaps, closed afterwards).  Output order = file order.
#include <charconv>
#include <cstdio>
#include <system_error>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include <fcntl.h>
#include <omp.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "cptc_hip.h"
#include "hip_util.hpp"

namespace {

// Read-only mapping of a file followed by at least one zero page: bytes
// [0, size) are the file, byte `size` and beyond (to the end of the span)
// read as 0.
struct Mapped
{
    const char* p = nullptr;
    size_t size = 0;
    size_t span = 0;
    ~Mapped()
    {
        if (p) munmap(const_cast<char*>(p), span);
    }
};

bool map_file(const char* path, Mapped& m)
{
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return false;
    struct stat st;
    if (fstat(fd, &st) != 0 || !S_ISREG(st.st_mode))
    {
        close(fd);
        return false;
    }
    const size_t pg = size_t(sysconf(_SC_PAGESIZE));
    const size_t sz = size_t(st.st_size);
    const size_t span = (sz / pg + 2) * pg;
    void* base = mmap(nullptr, span, PROT_READ, MAP_PRIVATE | MAP_ANONYMOUS, -1, 0);
    if (base == MAP_FAILED)
    {
        close(fd);
        return false;
    }
    if (sz > 0 &&
        mmap(base, sz, PROT_READ, MAP_PRIVATE | MAP_FIXED, fd, 0) == MAP_FAILED)
    {
        munmap(base, span);
        close(fd);
        return false;
    }
    close(fd);
    m.p = static_cast<const char*>(base);
    m.size = sz;
    m.span = span;
    return true;
}

inline int digits(const char* s, const char** end)
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

// The value field as strtod(p, &end) reads it (end = nullptr: no number).
// Plain decimals starting at p ([-]digits or [-].digits, optional fraction
// and exponent) go through std::from_chars, which rounds correctly like
// strtod (the same double) at a quarter of the cost; such a number ends
// before the line end `e`.  Anything else (a '+' sign, hex, inf / nan,
// whitespace or a newline before the number, out-of-range results) takes
// strtod itself.
inline const char* parse_value(const char* p, const char* e, double* v)
{
    const char* q = (*p == '-') ? p + 1 : p;
    if ((*q >= '0' && *q <= '9') || (*q == '.' && q[1] >= '0' && q[1] <= '9'))
    {
        const auto r = std::from_chars(p, e, *v);
        if (r.ec == std::errc() && r.ptr < e + 1 && *r.ptr != 'x' && *r.ptr != 'X')
            return r.ptr;
    }
    char* end = nullptr;
    *v = std::strtod(p, &end);
    return end == p ? nullptr : end;
}

// Where one chunk's parsed elements go: mode m's index of element e at
// idx[m][e], the value at val[e]; n = elements written so far.
struct Sink
{
    uint32_t* idx[CPTC_MAX_MODES] = {};
    double* val = nullptr;
    size_t n = 0;
    uint64_t mx[CPTC_MAX_MODES] = {};
};

// Newline-aligned chunk boundaries over [0, n).
std::vector<size_t> chunk_bounds(const char* b, size_t n, int parts)
{
    std::vector<size_t> cut(size_t(parts) + 1, n);
    cut[0] = 0;
    for (int t = 1; t < parts; ++t)
    {
        size_t p = n * size_t(t) / size_t(parts);
        if (p < cut[t - 1]) p = cut[t - 1];
        while (p < n && b[p - 1] != '\n') ++p;
        cut[t] = p;
    }
    return cut;
}

// tensor.cu:100-197
void parse3_line(const char* s, size_t len, Sink& c)
{
    if (len == 0 || s[0] == '#') return;
    const char* e = s + len;
    const char* p = s;
    const char* end = nullptr;
    int m[3];
    for (int f = 0; f < 3; ++f)
    {
        while (p < e && (*p == ' ' || *p == '\t')) ++p;
        if (p >= e) return;
        m[f] = digits(p, &end);
        p = end;
    }
    while (p < e && (*p == ' ' || *p == '\t')) ++p;
    if (p >= e) return;
    double v = 0.0;
    if (!parse_value(p, e, &v)) return;
    for (int f = 0; f < 3; ++f)
    {
        const uint32_t z = m[f] > 0 ? uint32_t(m[f] - 1) : 0u;
        c.idx[f][c.n] = z;
        if (z > c.mx[f]) c.mx[f] = z;
    }
    c.val[c.n++] = v;
}

// generic.cu:1067-1096
void parseN_line(const char* s, size_t len, int nmodes, Sink& c)
{
    if (len == 0 || s[0] == '#') return;
    const char* p = s;
    const char* end = nullptr;
    int m[CPTC_MAX_MODES];
    for (int f = 0; f < nmodes; ++f)
    {
        while (*p == ' ' || *p == '\t') ++p;
        if (!(*p >= '0' && *p <= '9')) return;
        m[f] = digits(p, &end);
        p = end;
    }
    while (*p == ' ' || *p == '\t') ++p;
    double v = 0.0;
    if (!parse_value(p, s + len, &v)) return;
    for (int f = 0; f < nmodes; ++f)
    {
        c.idx[f][c.n] = m[f] > 0 ? uint32_t(m[f] - 1) : 0u;
        if (uint64_t(m[f]) > c.mx[f]) c.mx[f] = uint64_t(m[f]);
    }
    c.val[c.n++] = v;
}

// Two passes over newline-aligned chunks of the mapping: line counts (and
// the longest line) per chunk, then each chunk parses into `out` at the
// prefix sum of the counts; gaps left by lines that did not parse are
// closed in chunk order.  Fills out->nnz, idx, val and the per-mode maxima.
template <class LineFn>
int parse_file(const Mapped& f, int nmodes, size_t max_line, const char* path, cptc_coo* out,
               uint64_t* mx, LineFn fn)
{
    const char* b = f.p;
    const size_t n = f.size;
    const int parts = std::max(1, std::min(omp_get_max_threads(), int(n / (1 << 20)) + 1));
    const std::vector<size_t> cut = chunk_bounds(b, n, parts);
    std::vector<size_t> lines(size_t(parts), 0), longest(size_t(parts), 0);
    #pragma omp parallel for schedule(static, 1) num_threads(parts)
    for (int t = 0; t < parts; ++t)
    {
        size_t cnt = 0, lmax = 0, ls = cut[t];
        const char* q = b + cut[t];
        const char* e = b + cut[t + 1];
        while (q < e)
        {
            const char* nl = static_cast<const char*>(std::memchr(q, '\n', size_t(e - q)));
            const char* le = nl ? nl : e;
            lmax = std::max(lmax, size_t(le - (b + ls)));
            ++cnt;
            q = le + 1;
            ls = size_t(q - b);
        }
        lines[t] = cnt;
        longest[t] = lmax;
    }
    size_t cap = 0, lmax = 0;
    std::vector<size_t> base(size_t(parts) + 1, 0);
    for (int t = 0; t < parts; ++t)
    {
        base[t + 1] = base[t] + lines[t];
        lmax = std::max(lmax, longest[t]);
    }
    cap = base[parts];
    CPTC_REQUIRE(lmax < max_line, CPTC_ERR_IO, "line longer than read buffer (%zu bytes) in %s",
                 max_line, path);
    std::memset(out, 0, sizeof(*out));
    out->nmodes = nmodes;
    out->idx = static_cast<uint32_t*>(std::malloc(sizeof(uint32_t) * nmodes * (cap ? cap : 1)));
    out->val = static_cast<double*>(std::malloc(sizeof(double) * (cap ? cap : 1)));
    CPTC_REQUIRE(out->idx && out->val, CPTC_ERR_IO, "tns: out of host memory for %zu lines", cap);
    std::vector<Sink> sinks(static_cast<size_t>(parts));
    #pragma omp parallel for schedule(static, 1) num_threads(parts)
    for (int t = 0; t < parts; ++t)
    {
        Sink& sk = sinks[t];
        for (int m = 0; m < nmodes; ++m) sk.idx[m] = out->idx + size_t(m) * cap + base[t];
        sk.val = out->val + base[t];
        size_t ls = cut[t];
        const char* q = b + cut[t];
        const char* e = b + cut[t + 1];
        while (q < e)
        {
            const char* nl = static_cast<const char*>(std::memchr(q, '\n', size_t(e - q)));
            const char* le = nl ? nl : e;
            fn(b + ls, size_t(le - (b + ls)), sk);
            q = le + 1;
            ls = size_t(q - b);
        }
    }
    // close the gaps (chunk order), then the mode stride becomes nnz
    size_t nnz = 0;
    for (int t = 0; t < parts; ++t)
    {
        const Sink& sk = sinks[t];
        if (nnz != base[t] && sk.n)
        {
            for (int m = 0; m < nmodes; ++m)
                std::memmove(out->idx + size_t(m) * cap + nnz, sk.idx[m], sk.n * sizeof(uint32_t));
            std::memmove(out->val + nnz, sk.val, sk.n * sizeof(double));
        }
        nnz += sk.n;
        for (int m = 0; m < nmodes; ++m) mx[m] = std::max(mx[m], sk.mx[m]);
    }
    if (nnz != cap)
        for (int m = 1; m < nmodes; ++m)
            std::memmove(out->idx + size_t(m) * nnz, out->idx + size_t(m) * cap,
                         nnz * sizeof(uint32_t));
    out->nnz = nnz;
    return CPTC_OK;
}

}  // namespace

extern "C" int cptc_tns_load3(const char* path, cptc_coo* out)
{
    CPTC_REQUIRE(path && out, CPTC_ERR_ARG, "cptc_tns_load3: null argument");
    Mapped f;
    CPTC_REQUIRE(map_file(path, f), CPTC_ERR_IO, "cannot open file: %s", path);
    uint64_t mx[CPTC_MAX_MODES] = {};
    CPTC_TRY(parse_file(f, 3, ~size_t(0), path, out, mx,
                        [](const char* s, size_t len, Sink& c) { parse3_line(s, len, c); }));
    for (int m = 0; m < 3; ++m) out->dims[m] = mx[m] + 1;
    return CPTC_OK;
}

// generic.cu:983-1021
extern "C" int cptc_tns_probe_nmodes(const char* path)
{
    FILE* f = path ? std::fopen(path, "rb") : nullptr;
    if (!f) return -1;
    std::vector<char> line(1 << 16);
    int nmodes = -1;
    while (std::fgets(line.data(), int(line.size()), f))
    {
        const char* b = line.data();
        if (b[0] == '#' || b[0] == '\n' || b[0] == '\r') continue;
        const char* p = b;
        while (*p == ' ' || *p == '\t') ++p;
        if (!(*p >= '0' && *p <= '9')) continue;
        int fields = 0;
        const char* q = p;
        while (*q && *q != '\n' && *q != '\r')
        {
            while (*q == ' ' || *q == '\t') ++q;
            if (*q == '\n' || *q == '\r' || !*q) break;
            ++fields;
            while (*q && *q != ' ' && *q != '\t') ++q;
        }
        nmodes = fields - 1;
        break;
    }
    std::fclose(f);
    return nmodes;
}

extern "C" int cptc_tns_load_generic(const char* path, cptc_coo* out)
{
    CPTC_REQUIRE(path && out, CPTC_ERR_ARG, "cptc_tns_load_generic: null argument");
    const int nmodes = cptc_tns_probe_nmodes(path);
    CPTC_REQUIRE(nmodes >= 2, CPTC_ERR_IO, "invalid tensor order %d in %s", nmodes, path);
    CPTC_REQUIRE(nmodes <= CPTC_MAX_MODES, CPTC_ERR_UNSUPPORTED, "tensor order %d > %d", nmodes,
                 CPTC_MAX_MODES);
    Mapped f;
    CPTC_REQUIRE(map_file(path, f), CPTC_ERR_IO, "cannot open file: %s", path);
    // generic.cu:1132-1138: a line longer than the 4 MiB read buffer aborts
    uint64_t mx[CPTC_MAX_MODES] = {};
    CPTC_TRY(parse_file(
        f, nmodes, size_t(1) << 22, path, out, mx,
        [nmodes](const char* s, size_t len, Sink& c) { parseN_line(s, len, nmodes, c); }));
    for (int m = 0; m < nmodes; ++m) out->dims[m] = mx[m] > 0 ? mx[m] : 1;
    return CPTC_OK;
}

extern "C" int cptc_tns_write(const char* path, const cptc_coo* c)
{
    CPTC_REQUIRE(path && c && c->nmodes >= 1 && c->nmodes <= CPTC_MAX_MODES, CPTC_ERR_ARG,
                 "cptc_tns_write: bad arguments");
    FILE* f = std::fopen(path, "wb");
    CPTC_REQUIRE(f, CPTC_ERR_IO, "cannot create %s", path);
    const size_t nnz = c->nnz;
    const int nm = c->nmodes;
    constexpr size_t BLK = 1 << 16;
    const size_t nblk = (nnz + BLK - 1) / BLK;
    int rc = CPTC_OK;
    // format blocks in parallel, write them in order
    for (size_t b0 = 0; b0 < nblk && rc == CPTC_OK; b0 += 64)
    {
        const size_t b1 = std::min(nblk, b0 + 64);
        std::vector<std::string> out(b1 - b0);
        #pragma omp parallel for schedule(dynamic, 1)
        for (int64_t b = int64_t(b0); b < int64_t(b1); ++b)
        {
            std::string& s = out[size_t(b) - b0];
            s.reserve(BLK * 48);
            char tmp[64];
            const size_t lo = size_t(b) * BLK, hi = std::min(nnz, lo + BLK);
            for (size_t e = lo; e < hi; ++e)
            {
                for (int m = 0; m < nm; ++m)
                {
                    auto r = std::to_chars(tmp, tmp + sizeof tmp,
                                           uint64_t(c->idx[size_t(m) * nnz + e]) + 1);
                    s.append(tmp, r.ptr);
                    s.push_back(' ');
                }
                auto r = std::to_chars(tmp, tmp + sizeof tmp, c->val[e]);
                s.append(tmp, r.ptr);
                s.push_back('\n');
            }
        }
        for (auto& s : out)
            if (std::fwrite(s.data(), 1, s.size(), f) != s.size()) rc = CPTC_ERR_IO;
    }
    if (std::fclose(f) != 0) rc = CPTC_ERR_IO;
    CPTC_REQUIRE(rc == CPTC_OK, rc, "write failed: %s", path);
    return CPTC_OK;
}
