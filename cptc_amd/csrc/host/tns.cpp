// `.tns` COO text ingest and export.
//
// Two parsers with the reference's two sets of semantics:
//   * order 3 (tensor.cu:24-271): fields bounded by the line, index m ->
//     (m > 0 ? m - 1 : 0), dims = max(0-based) + 1;
//   * N-order (generic.cu:971-1155): order from the first numeric line,
//     dims = max(1-based) or 1, lines longer than 4 MiB rejected.
// In both, strtod reads the value from the file buffer itself, so (as in the
// reference) it skips '\r' / '\n' when a line ends right after its indices.
// The file is read whole and parsed by OpenMP threads over newline-aligned
// chunks; the chunk results are concatenated in file order.
#include <charconv>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include <omp.h>

#include "cptc_hip.h"
#include "hip_util.hpp"

namespace {

bool read_file(const char* path, std::vector<char>& buf)
{
    FILE* f = std::fopen(path, "rb");
    if (!f) return false;
    std::fseek(f, 0, SEEK_END);
    const long sz = std::ftell(f);
    std::fseek(f, 0, SEEK_SET);
    buf.resize(size_t(sz > 0 ? sz : 0) + 1);
    const size_t got = sz > 0 ? std::fread(buf.data(), 1, size_t(sz), f) : 0;
    std::fclose(f);
    buf.resize(got + 1);
    buf[got] = '\0';
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

struct Chunk
{
    std::vector<uint32_t> idx[CPTC_MAX_MODES];
    std::vector<double> val;
    uint64_t mx[CPTC_MAX_MODES] = {};
    bool too_long = false;
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
void parse3_line(const char* s, size_t len, Chunk& c)
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
    char* endc = nullptr;
    const double v = std::strtod(p, &endc);
    if (endc == p) return;
    for (int f = 0; f < 3; ++f)
    {
        const uint32_t z = m[f] > 0 ? uint32_t(m[f] - 1) : 0u;
        c.idx[f].push_back(z);
        if (z > c.mx[f]) c.mx[f] = z;
    }
    c.val.push_back(v);
}

// generic.cu:1067-1096
void parseN_line(const char* s, size_t len, int nmodes, Chunk& c)
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
    char* endc = nullptr;
    const double v = std::strtod(p, &endc);
    if (endc == p) return;
    for (int f = 0; f < nmodes; ++f)
    {
        c.idx[f].push_back(m[f] > 0 ? uint32_t(m[f] - 1) : 0u);
        if (uint64_t(m[f]) > c.mx[f]) c.mx[f] = uint64_t(m[f]);
    }
    c.val.push_back(v);
}

template <class LineFn>
void parse_chunks(const std::vector<char>& buf, std::vector<Chunk>& chunks, LineFn fn)
{
    const char* b = buf.data();
    const size_t n = buf.size() - 1;
    const int parts = std::max(1, std::min(omp_get_max_threads(), int(n / (1 << 20)) + 1));
    chunks.assign(size_t(parts), Chunk{});
    const std::vector<size_t> cut = chunk_bounds(b, n, parts);
    #pragma omp parallel for schedule(static, 1) num_threads(parts)
    for (int t = 0; t < parts; ++t)
    {
        size_t ls = cut[t];
        for (size_t i = cut[t]; i < cut[t + 1]; ++i)
            if (b[i] == '\n')
            {
                fn(b + ls, i - ls, chunks[t]);
                ls = i + 1;
            }
        if (ls < cut[t + 1]) fn(b + ls, cut[t + 1] - ls, chunks[t]);
    }
}

int assemble(std::vector<Chunk>& chunks, int nmodes, cptc_coo* out)
{
    size_t nnz = 0;
    for (auto& c : chunks) nnz += c.val.size();
    std::memset(out, 0, sizeof(*out));
    out->nmodes = nmodes;
    out->nnz = nnz;
    out->idx = static_cast<uint32_t*>(std::malloc(sizeof(uint32_t) * nmodes * (nnz ? nnz : 1)));
    out->val = static_cast<double*>(std::malloc(sizeof(double) * (nnz ? nnz : 1)));
    CPTC_REQUIRE(out->idx && out->val, CPTC_ERR_IO, "tns: out of host memory for %zu elements", nnz);
    std::vector<size_t> base(chunks.size() + 1, 0);
    for (size_t t = 0; t < chunks.size(); ++t) base[t + 1] = base[t] + chunks[t].val.size();
    #pragma omp parallel for schedule(static, 1)
    for (int64_t t = 0; t < int64_t(chunks.size()); ++t)
    {
        Chunk& c = chunks[t];
        for (int m = 0; m < nmodes; ++m)
            if (!c.idx[m].empty())
                std::memcpy(out->idx + size_t(m) * nnz + base[t], c.idx[m].data(),
                            c.idx[m].size() * sizeof(uint32_t));
        if (!c.val.empty())
            std::memcpy(out->val + base[t], c.val.data(), c.val.size() * sizeof(double));
    }
    return CPTC_OK;
}

}  // namespace

extern "C" int cptc_tns_load3(const char* path, cptc_coo* out)
{
    CPTC_REQUIRE(path && out, CPTC_ERR_ARG, "cptc_tns_load3: null argument");
    std::vector<char> buf;
    CPTC_REQUIRE(read_file(path, buf), CPTC_ERR_IO, "cannot open file: %s", path);
    std::vector<Chunk> chunks;
    parse_chunks(buf, chunks, [](const char* s, size_t len, Chunk& c) { parse3_line(s, len, c); });
    CPTC_TRY(assemble(chunks, 3, out));
    for (int m = 0; m < 3; ++m)
    {
        uint64_t mx = 0;
        for (auto& c : chunks) mx = std::max(mx, c.mx[m]);
        out->dims[m] = mx + 1;
    }
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
    std::vector<char> buf;
    CPTC_REQUIRE(read_file(path, buf), CPTC_ERR_IO, "cannot open file: %s", path);
    // generic.cu:1132-1138: a line longer than the 4 MiB read buffer aborts
    {
        size_t ls = 0;
        const size_t n = buf.size() - 1;
        for (size_t i = 0; i <= n; ++i)
            if (i == n || buf[i] == '\n')
            {
                CPTC_REQUIRE(i - ls < (size_t(1) << 22), CPTC_ERR_IO,
                             "line longer than read buffer (4194304 bytes) in %s", path);
                ls = i + 1;
            }
    }
    std::vector<Chunk> chunks;
    parse_chunks(buf, chunks,
                 [nmodes](const char* s, size_t len, Chunk& c) { parseN_line(s, len, nmodes, c); });
    CPTC_TRY(assemble(chunks, nmodes, out));
    for (int m = 0; m < nmodes; ++m)
    {
        uint64_t mx = 0;
        for (auto& c : chunks) mx = std::max(mx, c.mx[m]);
        out->dims[m] = mx > 0 ? mx : 1;
    }
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
