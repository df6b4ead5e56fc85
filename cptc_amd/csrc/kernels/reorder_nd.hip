// Device reordering of the generic N-order path: the reference's HITS, CADR
// and auto relabelling (generic.cu:1176-1376), bit-exact with its host code.
//
// HITS (generic.cu:1290-1341): T rounds of
//   ns_m[c_m(e)] += prod_{q != m, q ascending} s_q[c_q(e)]
// over the elements e = 0, stride, 2 stride, ... (stride = nnz / budget when
// nnz > budget), every mode from the same s, then s_m = ns_m / max(ns_m).
// The reference adds each row's terms one after another in element order, so
// the sums here keep that order: a stable sort of the sample by c_m gives
// each row its elements in element order, the products are formed in
// parallel (the same multiplication order), and one wave per (mode, row)
// adds them in sequence (lane 0, fed through LDS by the whole wave).  Ranks
// sort by
// score descending, ties by index ascending: a stable descending radix sort
// of the scores over indices in ascending order.
// CADR (generic.cu:1342-1357): degree descending, index ascending (same
// stable sort over integer degrees).
// auto (generic.cu:1201-1288): a sampled fill probe of 16^3 tiles x outer
// tuples before and after HITS (the latter maps relabelled coordinates
// through the ranks once more, as the reference does); integer counts, the
// ratio formed on the host.
#include "dev_util.hpp"

#include <rocprim/device/device_radix_sort.hpp>

#include <algorithm>
#include <cstdio>
#include <string>
#include <vector>

#include "../host/layout_nd.hpp"

namespace cptc {

using namespace dev;

namespace {

constexpr int MAXM = CPTC_MAX_MODES;
constexpr uint64_t GOLDEN = 0x9E3779B97F4A7C15ull;

struct Scores
{
    const double* s[MAXM];
};
struct ModeCoords
{
    const uint32_t* c[MAXM];
};

__device__ inline uint64_t splitbit_hash(uint64_t x)
{
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

__global__ void iota_kernel(uint32_t* __restrict__ a, uint64_t n)
{
    const uint64_t stride = uint64_t(gridDim.x) * blockDim.x;
    for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
        a[i] = uint32_t(i);
}

__global__ void fill_kernel(double* __restrict__ a, uint64_t n, double v)
{
    const uint64_t stride = uint64_t(gridDim.x) * blockDim.x;
    for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
        a[i] = v;
}

// deg[x] += #{e : c[e] = x}: per-block LDS counts (dim <= DEG_LDS_MAX), then
// one global add per bin and block; larger dims count in global memory,
// where the many bins keep contention low.
constexpr uint64_t DEG_LDS_MAX = 16384;

__global__ void degree_lds_kernel(const uint32_t* __restrict__ c, uint64_t nnz, uint32_t dim,
                                  uint32_t* __restrict__ deg)
{
    extern __shared__ uint32_t h[];
    for (uint32_t x = threadIdx.x; x < dim; x += blockDim.x) h[x] = 0;
    __syncthreads();
    const uint64_t step = uint64_t(gridDim.x) * blockDim.x;
    for (uint64_t e = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; e < nnz; e += step)
        atomicAdd(&h[c[e]], 1u);
    __syncthreads();
    for (uint32_t x = threadIdx.x; x < dim; x += blockDim.x)
        if (h[x]) atomicAdd(&deg[x], h[x]);
}

__global__ void degree_global_kernel(const uint32_t* __restrict__ c, uint64_t nnz,
                                     uint32_t* __restrict__ deg)
{
    const uint64_t step = uint64_t(gridDim.x) * blockDim.x;
    for (uint64_t e = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; e < nnz; e += step)
        atomicAdd(&deg[c[e]], 1u);
}

// off[x] = first position of a key >= x in the sorted keys (x = 0..dim)
__global__ void row_offsets_kernel(const uint32_t* __restrict__ skey, uint64_t S, uint64_t dim,
                                   uint64_t* __restrict__ off)
{
    const uint64_t step = uint64_t(gridDim.x) * blockDim.x;
    for (uint64_t x = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; x <= dim; x += step)
    {
        uint64_t lo = 0, hi = S;
        while (lo < hi)
        {
            const uint64_t mid = (lo + hi) / 2;
            if (uint64_t(skey[mid]) < x)
                lo = mid + 1;
            else
                hi = mid;
        }
        off[x] = lo;
    }
}

__global__ void scatter_rank_kernel(const uint32_t* __restrict__ ord, uint64_t n,
                                    uint32_t* __restrict__ rank)
{
    const uint64_t stride = uint64_t(gridDim.x) * blockDim.x;
    for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
        rank[ord[i]] = uint32_t(i);
}

// sample keys of mode m: key[k] = c_m(k * stride), val[k] = k
__global__ void sample_keys_kernel(const uint32_t* __restrict__ c, uint64_t stride, uint64_t S,
                                   uint32_t* __restrict__ key, uint32_t* __restrict__ val)
{
    const uint64_t step = uint64_t(gridDim.x) * blockDim.x;
    for (uint64_t k = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; k < S; k += step)
    {
        key[k] = c[k * stride];
        val[k] = uint32_t(k);
    }
}

// co[q][j] = c_q(el[j] * stride) for every q != m (q ascending; nq = N - 1 rows)
__global__ void gather_others_kernel(ModeCoords mc, int N, int m, const uint32_t* __restrict__ el,
                                     uint64_t stride, uint64_t S, uint32_t* __restrict__ co)
{
    const uint64_t step = uint64_t(gridDim.x) * blockDim.x;
    for (uint64_t j = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; j < S; j += step)
    {
        const uint64_t e = uint64_t(el[j]) * stride;
        int r = 0;
        for (int q = 0; q < N; ++q)
            if (q != m) co[uint64_t(r++) * S + j] = mc.c[q][e];
    }
}

// p[j] = prod_{q != m, q ascending} s_q[co[q][j]], starting from 1.0
__global__ void hits_products_kernel(Scores sc, int N, int m, const uint32_t* __restrict__ co,
                                     uint64_t S, double* __restrict__ p)
{
    const uint64_t step = uint64_t(gridDim.x) * blockDim.x;
    for (uint64_t j = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; j < S; j += step)
    {
        double x = 1.0;
        int r = 0;
        for (int q = 0; q < N; ++q)
            if (q != m) x *= sc.s[q][co[uint64_t(r++) * S + j]];
        p[j] = x;
    }
}

// ns_m[x] = ((0 + p_m[off_m[x]]) + p_m[off_m[x] + 1]) + ... for every mode:
// one wave per (mode, row).  The wave stages windows of SUM_WIN terms in LDS
// (coalesced loads, the next window prefetched into registers) and lane 0
// adds them in order; a full window is unrolled so its LDS reads run ahead
// of the add chain.
constexpr int SUM_WIN = 256;

struct RowSums
{
    const double* p[MAXM];
    const uint64_t* off[MAXM];
    double* ns[MAXM];
    uint64_t first[MAXM + 1];   // first task of each mode: sum of the dims before it
    int N;
};

__device__ __forceinline__ void wave_sync()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__global__ __launch_bounds__(64) void row_sequential_sum_kernel(RowSums rs)
{
    __shared__ double buf[SUM_WIN];
    const int lane = threadIdx.x;
    const uint64_t ntask = rs.first[rs.N];
    for (uint64_t t = blockIdx.x; t < ntask; t += gridDim.x)
    {
        int m = 0;
        while (m + 1 < rs.N && t >= rs.first[m + 1]) ++m;
        const uint64_t x = t - rs.first[m];
        const double* __restrict__ p = rs.p[m];
        const uint64_t b = rs.off[m][x], e = rs.off[m][x + 1];
        double acc = 0.0;
        double nxt[SUM_WIN / 64];
        auto load = [&](uint64_t c0) {
#pragma unroll
            for (int k = 0; k < SUM_WIN / 64; ++k)
            {
                const uint64_t i = c0 + uint64_t(lane + 64 * k);
                nxt[k] = (i < e) ? p[i] : 0.0;
            }
        };
        load(b);
        for (uint64_t c0 = b; c0 < e; c0 += SUM_WIN)
        {
            wave_sync();
#pragma unroll
            for (int k = 0; k < SUM_WIN / 64; ++k) buf[lane + 64 * k] = nxt[k];
            wave_sync();
            if (c0 + SUM_WIN < e) load(c0 + SUM_WIN);
            if (lane == 0)
            {
                if (e - c0 >= uint64_t(SUM_WIN))
                {
#pragma unroll
                    for (int i = 0; i < SUM_WIN; ++i) acc += buf[i];
                }
                else
                {
                    const int cnt = int(e - c0);
                    for (int i = 0; i < cnt; ++i) acc += buf[i];
                }
            }
        }
        if (lane == 0) rs.ns[m][x] = acc;
        wave_sync();
    }
}

// *mx = max(v[0..n)) (0 for n = 0; values are >= 0)
__global__ __launch_bounds__(1024) void max_kernel(const double* __restrict__ v, uint64_t n,
                                                   double* __restrict__ mx)
{
    __shared__ double red[1024];
    double m = 0.0;
    for (uint64_t i = threadIdx.x; i < n; i += 1024) m = fmax(m, v[i]);
    red[threadIdx.x] = m;
    __syncthreads();
    for (int w = 512; w > 0; w >>= 1)
    {
        if (int(threadIdx.x) < w) red[threadIdx.x] = fmax(red[threadIdx.x], red[threadIdx.x + w]);
        __syncthreads();
    }
    if (threadIdx.x == 0) *mx = red[0];
}

// s[x] = ns[x] / mx when mx > 0, else ns[x]
__global__ void normalize_scores_kernel(const double* __restrict__ ns, uint64_t n,
                                        const double* __restrict__ mx, double* __restrict__ s)
{
    const double d = *mx;
    const uint64_t step = uint64_t(gridDim.x) * blockDim.x;
    for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += step)
        s[i] = (d > 0.0) ? ns[i] / d : ns[i];
}

__global__ void relabel_kernel(uint32_t* __restrict__ c, uint64_t nnz,
                               const uint32_t* __restrict__ rank)
{
    const uint64_t step = uint64_t(gridDim.x) * blockDim.x;
    for (uint64_t e = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; e < nnz; e += step)
        c[e] = rank[c[e]];
}

// twice[a] = rank[rank[a]]
__global__ void compose_kernel(const uint32_t* __restrict__ rank, uint64_t n,
                               uint32_t* __restrict__ twice)
{
    const uint64_t step = uint64_t(gridDim.x) * blockDim.x;
    for (uint64_t a = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; a < n; a += step)
        twice[a] = rank[rank[a]];
}

// probe keys (generic.cu:1208-1237): tile = ((a/16) nbj + b/16) nbk + c/16 over
// modes 0, 1, 2; o folds the outer modes; coordinates mapped through `map`
// (per mode, may be null)
__global__ void probe_keys_kernel(ModeCoords mc, ModeCoords map, int N, uint64_t st, uint64_t S,
                                  uint64_t nbj, uint64_t nbk, uint64_t* __restrict__ key)
{
    const uint64_t step = uint64_t(gridDim.x) * blockDim.x;
    for (uint64_t k = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; k < S; k += step)
    {
        const uint64_t e = k * st;
        auto co = [&](int m) -> uint64_t {
            const uint32_t x = mc.c[m][e];
            return map.c[m] ? map.c[m][x] : x;
        };
        const uint64_t a = co(0), b = co(1), c = co(2);
        const uint64_t tile = ((a / 16) * nbj + b / 16) * nbk + c / 16;
        uint64_t o = 0;
        for (int m = 3; m < N; ++m) o = o * 1000003ull + co(m);
        key[k] = splitbit_hash(tile ^ (o * GOLDEN));
    }
}

unsigned grid1(uint64_t n) { return grid_for(n, 256, 16384); }

template <class K, class V>
int sort_pairs_desc(const K* kin, K* kout, const V* vin, V* vout, size_t n, int end_bit,
                    hipStream_t s)
{
    size_t bytes = 0;
    CPTC_HIP(rocprim::radix_sort_pairs_desc(nullptr, bytes, kin, kout, vin, vout, n, 0,
                                            unsigned(end_bit), s));
    Tmp<char> tmp;
    CPTC_TRY(tmp.alloc(bytes ? bytes : 1));
    CPTC_HIP(rocprim::radix_sort_pairs_desc(tmp.p, bytes, kin, kout, vin, vout, n, 0,
                                            unsigned(end_bit), s));
    return CPTC_OK;
}

// rank[ord[i]] = i with ord = indices sorted by key descending, ties by index
// ascending (stable sort of an ascending iota)
template <class K>
int rank_desc(const K* d_key, uint64_t n, int end_bit, uint32_t* d_rank, hipStream_t s)
{
    Tmp<K> kout;
    Tmp<uint32_t> iota, ord;
    CPTC_TRY(kout.alloc(n));
    CPTC_TRY(iota.alloc(n));
    CPTC_TRY(ord.alloc(n));
    hipLaunchKernelGGL(iota_kernel, dim3(grid1(n)), dim3(256), 0, s, iota.p, n);
    CPTC_LAUNCHED();
    CPTC_TRY(sort_pairs_desc(d_key, kout.p, iota.p, ord.p, n, end_bit, s));
    hipLaunchKernelGGL(scatter_rank_kernel, dim3(grid1(n)), dim3(256), 0, s, ord.p, n, d_rank);
    CPTC_LAUNCHED();
    return CPTC_OK;
}

struct DevRanks
{
    std::vector<uint32_t*> r;
    ~DevRanks()
    {
        for (auto& p : r) dfree(p);
    }
};

int cadr_device(int N, const uint64_t* dims, const uint32_t* d_coords, uint64_t nnz,
                DevRanks& rk, hipStream_t s)
{
    rk.r.assign(N, nullptr);
    for (int m = 0; m < N; ++m)
    {
        Tmp<uint32_t> deg;
        CPTC_TRY(deg.alloc(dims[m]));
        CPTC_HIP(hipMemsetAsync(deg.p, 0, dims[m] * sizeof(uint32_t), s));
        const uint32_t* c = d_coords + uint64_t(m) * nnz;
        if (dims[m] <= DEG_LDS_MAX)
        {
            static cptc::DeviceOnce attr;
            CPTC_HIP(attr.lds_limit({reinterpret_cast<const void*>(degree_lds_kernel)},
                                    int(DEG_LDS_MAX * sizeof(uint32_t))));
            // one block per CU: each flushes at most dims[m] counts
            hipLaunchKernelGGL(degree_lds_kernel, dim3(std::min(grid1(nnz), 256u)), dim3(256),
                               dims[m] * sizeof(uint32_t), s, c, nnz, uint32_t(dims[m]), deg.p);
        }
        else
        {
            hipLaunchKernelGGL(degree_global_kernel, dim3(grid1(nnz)), dim3(256), 0, s, c, nnz,
                               deg.p);
        }
        CPTC_LAUNCHED();
        CPTC_TRY(dalloc(&rk.r[m], dims[m]));
        CPTC_TRY(rank_desc(deg.p, dims[m], 32, rk.r[m], s));
    }
    return CPTC_OK;
}

int hits_device(int N, const uint64_t* dims, const uint32_t* d_coords, uint64_t nnz, int rounds,
                uint64_t budget, DevRanks& rk, hipStream_t s)
{
    const uint64_t stride = (nnz > budget && budget > 0) ? (nnz / budget) : 1;
    const uint64_t S = (nnz + stride - 1) / stride;
    ModeCoords mc{};
    for (int m = 0; m < N; ++m) mc.c[m] = d_coords + uint64_t(m) * nnz;
    // per mode: row offsets of the sample and the other coordinates in row order
    std::vector<Tmp<uint64_t>> off(N);
    std::vector<Tmp<uint32_t>> co(N);
    {
        Tmp<uint32_t> key, val, skey, el;
        CPTC_TRY(key.alloc(S));
        CPTC_TRY(val.alloc(S));
        CPTC_TRY(skey.alloc(S));
        CPTC_TRY(el.alloc(S));
        for (int m = 0; m < N; ++m)
        {
            hipLaunchKernelGGL(sample_keys_kernel, dim3(grid1(S)), dim3(256), 0, s, mc.c[m],
                               stride, S, key.p, val.p);
            CPTC_LAUNCHED();
            CPTC_TRY(sort_pairs(key.p, skey.p, val.p, el.p, S,
                                bit_width(dims[m] > 0 ? dims[m] - 1 : 0), s));
            CPTC_TRY(off[m].alloc(dims[m] + 1));
            hipLaunchKernelGGL(row_offsets_kernel, dim3(grid1(dims[m] + 1)), dim3(256), 0, s,
                               skey.p, S, dims[m], off[m].p);
            CPTC_LAUNCHED();
            CPTC_TRY(co[m].alloc(uint64_t(N - 1) * S));
            hipLaunchKernelGGL(gather_others_kernel, dim3(grid1(S)), dim3(256), 0, s, mc, N, m,
                               el.p, stride, S, co[m].p);
            CPTC_LAUNCHED();
        }
    }
    std::vector<Tmp<double>> sc(N), ns(N), p(N);
    Tmp<double> mx;
    CPTC_TRY(mx.alloc(N));
    RowSums rs{};
    rs.N = N;
    for (int m = 0; m < N; ++m)
    {
        CPTC_TRY(p[m].alloc(S));
        rs.first[m + 1] = rs.first[m] + dims[m];
    }
    for (int m = 0; m < N; ++m)
    {
        CPTC_TRY(sc[m].alloc(dims[m]));
        CPTC_TRY(ns[m].alloc(dims[m]));
        hipLaunchKernelGGL(fill_kernel, dim3(grid1(dims[m])), dim3(256), 0, s, sc[m].p, dims[m],
                           1.0);
        CPTC_LAUNCHED();
    }
    for (int it = 0; it < rounds; ++it)
    {
        Scores cur{};
        for (int m = 0; m < N; ++m) cur.s[m] = sc[m].p;
        for (int m = 0; m < N; ++m)
        {
            hipLaunchKernelGGL(hits_products_kernel, dim3(grid1(S)), dim3(256), 0, s, cur, N, m,
                               co[m].p, S, p[m].p);
            CPTC_LAUNCHED();
            rs.p[m] = p[m].p;
            rs.off[m] = off[m].p;
            rs.ns[m] = ns[m].p;
        }
        const unsigned tasks = unsigned(std::min<uint64_t>(rs.first[N], 1u << 20));
        hipLaunchKernelGGL(row_sequential_sum_kernel, dim3(tasks), dim3(64), 0, s, rs);
        CPTC_LAUNCHED();
        for (int m = 0; m < N; ++m)
        {
            hipLaunchKernelGGL(max_kernel, dim3(1), dim3(1024), 0, s, ns[m].p, dims[m], mx.p + m);
            CPTC_LAUNCHED();
            hipLaunchKernelGGL(normalize_scores_kernel, dim3(grid1(dims[m])), dim3(256), 0, s,
                               ns[m].p, dims[m], mx.p + m, sc[m].p);
            CPTC_LAUNCHED();
        }
    }
    rk.r.assign(N, nullptr);
    for (int m = 0; m < N; ++m)
    {
        CPTC_TRY(dalloc(&rk.r[m], dims[m]));
        CPTC_TRY(rank_desc(sc[m].p, dims[m], 64, rk.r[m], s));
    }
    CPTC_HIP(hipStreamSynchronize(s));
    return CPTC_OK;
}

// fill of the sampled 16^3 tiles x outer tuples with >= 122 elements
int probe_fill_device(int N, const uint64_t* dims, const uint32_t* d_coords, uint64_t nnz,
                      const DevRanks* map, double* fill, hipStream_t s)
{
    const uint64_t budget = 2000000;
    const uint64_t st = (nnz > budget) ? (nnz / budget) : 1;
    const uint64_t S = (nnz + st - 1) / st;
    ModeCoords mc{}, mp{};
    for (int m = 0; m < N; ++m)
    {
        mc.c[m] = d_coords + uint64_t(m) * nnz;
        mp.c[m] = map ? map->r[m] : nullptr;
    }
    Tmp<uint64_t> key, skey, ukey;
    Tmp<uint32_t> cnt, nruns_d;
    CPTC_TRY(key.alloc(S));
    CPTC_TRY(skey.alloc(S));
    CPTC_TRY(ukey.alloc(S));
    CPTC_TRY(cnt.alloc(S));
    CPTC_TRY(nruns_d.alloc(1));
    hipLaunchKernelGGL(probe_keys_kernel, dim3(grid1(S)), dim3(256), 0, s, mc, mp, N, st, S,
                       (dims[1] + 15) / 16, (dims[2] + 15) / 16, key.p);
    CPTC_LAUNCHED();
    {
        size_t bytes = 0;
        CPTC_HIP(rocprim::radix_sort_keys(nullptr, bytes, key.p, skey.p, S, 0, 64, s));
        Tmp<char> tmp;
        CPTC_TRY(tmp.alloc(bytes ? bytes : 1));
        CPTC_HIP(rocprim::radix_sort_keys(tmp.p, bytes, key.p, skey.p, S, 0, 64, s));
    }
    CPTC_TRY(run_length(skey.p, S, ukey.p, cnt.p, nruns_d.p, s));
    uint32_t nruns = 0;
    CPTC_TRY(d2h_one(&nruns, nruns_d.p, s));
    std::vector<uint32_t> h(nruns);
    CPTC_HIP(hipMemcpyAsync(h.data(), cnt.p, nruns * sizeof(uint32_t), hipMemcpyDeviceToHost, s));
    CPTC_HIP(hipStreamSynchronize(s));
    long long tiles = 0, in = 0;
    for (uint32_t c : h)
    {
        const long long n = (long long)c * (long long)st;
        if (n >= 122)
        {
            ++tiles;
            in += n;
        }
    }
    *fill = tiles ? double(in) / (double(tiles) * 4096.0) : 0.0;
    return CPTC_OK;
}

int download_ranks(int N, const uint64_t* dims, const DevRanks& rk,
                   std::vector<std::vector<uint32_t>>& rank, hipStream_t s)
{
    rank.assign(N, {});
    for (int m = 0; m < N; ++m)
    {
        rank[m].resize(dims[m]);
        CPTC_HIP(hipMemcpyAsync(rank[m].data(), rk.r[m], dims[m] * sizeof(uint32_t),
                                hipMemcpyDeviceToHost, s));
    }
    CPTC_HIP(hipStreamSynchronize(s));
    return CPTC_OK;
}

int relabel_all(int N, uint32_t* d_coords, uint64_t nnz, const DevRanks& rk, hipStream_t s)
{
    for (int m = 0; m < N; ++m)
    {
        hipLaunchKernelGGL(relabel_kernel, dim3(grid1(nnz)), dim3(256), 0, s,
                           d_coords + uint64_t(m) * nnz, nnz, rk.r[m]);
        CPTC_LAUNCHED();
    }
    return CPTC_OK;
}

}  // namespace

int reorder_nd_device(int N, const uint64_t* dims, uint32_t* d_coords, uint64_t nnz,
                      std::string how, int rounds, uint64_t budget,
                      std::vector<std::vector<uint32_t>>& rank, std::string& used, bool verbose,
                      hipStream_t s)
{
    rank.clear();
    used = "none";
    if (rounds < 1) rounds = 1;
    if (budget == 0) budget = 8000000;
    CPTC_REQUIRE(N >= 1 && N <= MAXM && nnz <= 0xFFFFFFFFull, CPTC_ERR_ARG,
                 "reorder: %d modes, %llu nnz", N, (unsigned long long)nnz);
    if (how != "hits" && how != "cadr" && how != "none" && how != "auto")
    {
        if (verbose)
            std::printf("[GEN] unknown GEN_REORDER=%s -> falling back to cadr\n", how.c_str());
        how = "cadr";
    }
    if (how == "none" || nnz == 0) return CPTC_OK;
    DevRanks rk;
    if (how == "cadr")
    {
        CPTC_TRY(cadr_device(N, dims, d_coords, nnz, rk, s));
        used = "cadr";
    }
    else if (how == "hits")
    {
        CPTC_TRY(hits_device(N, dims, d_coords, nnz, rounds, budget, rk, s));
        used = "hits";
    }
    else
    {
        // auto (generic.cu:1201-1288)
        if (N < 3)
        {
            if (verbose) std::printf("[GEN] reorder=auto -> none (order %d < 3)\n", N);
            return CPTC_OK;
        }
        double f_raw = 0.0;
        CPTC_TRY(probe_fill_device(N, dims, d_coords, nnz, nullptr, &f_raw, s));
        if (f_raw < 0.02)
        {
            if (verbose)
                std::printf("[GEN] reorder=auto -> none (raw probe fill %g < 0.02)\n", f_raw);
            return CPTC_OK;
        }
        CPTC_TRY(hits_device(N, dims, d_coords, nnz, rounds, budget, rk, s));
        // the reference probes coordinates it has already relabelled through
        // the ranks once more: rank[rank[c]]
        DevRanks twice;
        twice.r.assign(N, nullptr);
        for (int m = 0; m < N; ++m)
        {
            CPTC_TRY(dalloc(&twice.r[m], dims[m]));
            hipLaunchKernelGGL(compose_kernel, dim3(grid1(dims[m])), dim3(256), 0, s, rk.r[m],
                               dims[m], twice.r[m]);
            CPTC_LAUNCHED();
        }
        double f_hits = 0.0;
        CPTC_TRY(probe_fill_device(N, dims, d_coords, nnz, &twice, &f_hits, s));
        if (f_hits < 0.11)
        {
            if (verbose)
                std::printf("[GEN] reorder=auto -> none (probe fill %g -> %g < 0.11)\n", f_raw,
                            f_hits);
            return CPTC_OK;
        }
        if (verbose)
            std::printf("[GEN] reorder=auto -> hits (probe fill %g -> %g >= 0.11)\n", f_raw,
                        f_hits);
        used = "hits";
    }
    CPTC_TRY(relabel_all(N, d_coords, nnz, rk, s));
    CPTC_TRY(download_ranks(N, dims, rk, rank, s));
    return CPTC_OK;
}

}  // namespace cptc
