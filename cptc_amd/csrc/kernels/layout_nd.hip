// Device layout of the generic N-order path.
//
// Dense units (generic.cu:578-725).  The reference counts a 64-bit hash key
// per element in a host hash map and numbers the keys whose count reaches
// the cutoff by first occurrence.  Here the keys are sorted stably with the
// element index as payload (rocPRIM radix sort), so each key is one run whose
// payload lists its elements in element order; a run is a unit when its
// count reaches the cutoff, and sorting the units' first elements gives the
// first-occurrence numbering.  Hash collisions merge groups exactly as in the
// reference, because both group by the hash value.
//
// Views (generic.cu:1848-1958).  A stable radix sort by coordinate n is the
// counting sort of the reference; segments are cut on the host from the row
// run lengths.  The kernel's own views ("work views") drop the dense
// elements and sort each row over the other modes with successive stable
// sorts (least significant level first).
#include "dev_util.hpp"

#include <rocprim/device/device_select.hpp>

#include <algorithm>
#include <vector>

#include "../host/layout_nd.hpp"

namespace cptc {

namespace {

using dev::bit_width;
using dev::d2h_one;
using dev::dalloc;
using dev::dfree;
using dev::exclusive_sum;
using dev::run_length;
using dev::sort_pairs;
using dev::Tmp;

struct ModeSet
{
    int inner[3];
    int outer[CPTC_MAX_MODES];
    int nouter;
};

__device__ inline uint64_t splitbit(uint64_t x)
{
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

__global__ void unit_keys_kernel(const uint32_t* __restrict__ co, uint64_t nnz, ModeSet ms,
                                 uint64_t* __restrict__ key, uint32_t* __restrict__ idx)
{
    const uint64_t stride = uint64_t(gridDim.x) * blockDim.x;
    for (uint64_t e = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; e < nnz; e += stride)
    {
        const uint64_t a = co[uint64_t(ms.inner[0]) * nnz + e];
        const uint64_t b = co[uint64_t(ms.inner[1]) * nnz + e];
        const uint64_t c = co[uint64_t(ms.inner[2]) * nnz + e];
        uint64_t o = 0;
#pragma unroll
        for (int k = 0; k < CPTC_MAX_MODES; ++k)
            if (k < ms.nouter) o = o * 1000003ull + co[uint64_t(ms.outer[k]) * nnz + e];
        const uint64_t tile = ((a / 16) << 40) | ((b / 16) << 20) | (c / 16);
        key[e] = splitbit(tile ^ (o * 0x9E3779B97F4A7C15ull));
        idx[e] = uint32_t(e);
    }
}

// first[r] = the run's first element when it is a unit, else 0xFFFFFFFF
// (never an element index: nnz <= 0x7FFFFFFF).
__global__ void unit_runs_kernel(const uint32_t* __restrict__ counts,
                                 const uint32_t* __restrict__ roff,
                                 const uint32_t* __restrict__ sidx, uint32_t nruns, int cutoff,
                                 uint32_t* __restrict__ first, uint32_t* __restrict__ rid,
                                 uint32_t* __restrict__ isunit)
{
    const uint32_t stride = gridDim.x * blockDim.x;
    for (uint32_t r = blockIdx.x * blockDim.x + threadIdx.x; r < nruns; r += stride)
    {
        const bool u = int64_t(counts[r]) >= int64_t(cutoff);
        first[r] = u ? sidx[roff[r]] : 0xFFFFFFFFu;
        rid[r] = r;
        isunit[r] = u ? 1u : 0u;
    }
}

__global__ void unit_counts_kernel(const uint32_t* __restrict__ urun,
                                   const uint32_t* __restrict__ counts, uint32_t nunits,
                                   uint32_t* __restrict__ ucnt)
{
    const uint32_t stride = gridDim.x * blockDim.x;
    for (uint32_t k = blockIdx.x * blockDim.x + threadIdx.x; k < nunits; k += stride)
        ucnt[k] = counts[urun[k]];
}

__global__ void unit_meta_kernel(const uint32_t* __restrict__ ufirst,
                                 const uint32_t* __restrict__ ucnt,
                                 const uint32_t* __restrict__ ustart, uint32_t nunits,
                                 const uint32_t* __restrict__ co, uint64_t nnz, ModeSet ms,
                                 uint32_t* __restrict__ unit6, uint32_t* __restrict__ outer_coords)
{
    const uint32_t stride = gridDim.x * blockDim.x;
    for (uint32_t k = blockIdx.x * blockDim.x + threadIdx.x; k < nunits; k += stride)
    {
        const uint64_t e = ufirst[k];
        unit6[6 * size_t(k) + 0] = co[uint64_t(ms.inner[0]) * nnz + e] / 16;
        unit6[6 * size_t(k) + 1] = co[uint64_t(ms.inner[1]) * nnz + e] / 16;
        unit6[6 * size_t(k) + 2] = co[uint64_t(ms.inner[2]) * nnz + e] / 16;
        unit6[6 * size_t(k) + 3] = ucnt[k];
        unit6[6 * size_t(k) + 4] = ustart[k];
        unit6[6 * size_t(k) + 5] = k * uint32_t(ms.nouter);
#pragma unroll
        for (int q = 0; q < CPTC_MAX_MODES; ++q)
            if (q < ms.nouter)
                outer_coords[size_t(k) * ms.nouter + q] = co[uint64_t(ms.outer[q]) * nnz + e];
    }
}

// One workgroup per unit: its run of the sorted payload, in element order.
__global__ void unit_pool_kernel(const uint32_t* __restrict__ urun,
                                 const uint32_t* __restrict__ roff,
                                 const uint32_t* __restrict__ ucnt,
                                 const uint32_t* __restrict__ ustart,
                                 const uint32_t* __restrict__ sidx,
                                 const uint32_t* __restrict__ co, const double* __restrict__ vals,
                                 uint64_t nnz, ModeSet ms, uint32_t* __restrict__ lid,
                                 double* __restrict__ pval, uint8_t* __restrict__ isd)
{
    const uint32_t k = blockIdx.x;
    const uint32_t base = roff[urun[k]], n = ucnt[k], st = ustart[k];
    for (uint32_t j = threadIdx.x; j < n; j += blockDim.x)
    {
        const uint64_t e = sidx[base + j];
        const uint32_t a = co[uint64_t(ms.inner[0]) * nnz + e] % 16;
        const uint32_t b = co[uint64_t(ms.inner[1]) * nnz + e] % 16;
        const uint32_t c = co[uint64_t(ms.inner[2]) * nnz + e] % 16;
        lid[st + j] = a * 256 + b * 16 + c;
        pval[st + j] = vals[e];
        isd[e] = 1;
    }
}

__global__ void iota_kernel(uint32_t* __restrict__ x, uint64_t n)
{
    const uint64_t stride = uint64_t(gridDim.x) * blockDim.x;
    for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
        x[i] = uint32_t(i);
}

__global__ void view_gather_kernel(const uint32_t* __restrict__ order,
                                   const uint32_t* __restrict__ co, const double* __restrict__ vals,
                                   const uint8_t* __restrict__ isd, uint64_t nnz, int N, int n,
                                   uint32_t* __restrict__ sc, double* __restrict__ sv,
                                   uint8_t* __restrict__ skip)
{
    const uint64_t stride = uint64_t(gridDim.x) * blockDim.x;
    for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < nnz; i += stride)
    {
        const uint64_t e = order[i];
        sv[i] = vals[e];
        if (skip) skip[i] = isd[e];
        int q = 0;
        for (int m = 0; m < N; ++m)
        {
            if (m == n) continue;
            sc[uint64_t(q) * nnz + i] = co[uint64_t(m) * nnz + e];
            ++q;
        }
    }
}

__global__ void keep_flags_kernel(const uint8_t* __restrict__ isd, uint64_t n,
                                  uint8_t* __restrict__ keep)
{
    const uint64_t stride = uint64_t(gridDim.x) * blockDim.x;
    for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
        keep[i] = isd[i] ? 0 : 1;
}

__global__ void gather_keys_kernel(const uint32_t* __restrict__ col,
                                   const uint32_t* __restrict__ perm, uint64_t n,
                                   uint32_t* __restrict__ key)
{
    const uint64_t stride = uint64_t(gridDim.x) * blockDim.x;
    for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
        key[i] = col[perm[i]];
}

struct Levels
{
    int m[CPTC_MAX_MODES];
};

__global__ void work_gather_kernel(const uint32_t* __restrict__ order,
                                   const uint32_t* __restrict__ co,
                                   const double* __restrict__ vals, uint64_t nnz, uint64_t M,
                                   int nlev, Levels lv, uint32_t* __restrict__ sc,
                                   double* __restrict__ sv)
{
    const uint64_t stride = uint64_t(gridDim.x) * blockDim.x;
    for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < M; i += stride)
    {
        const uint64_t e = order[i];
        sv[i] = vals[e];
#pragma unroll
        for (int q = 0; q < CPTC_MAX_MODES; ++q)
            if (q < nlev) sc[uint64_t(q) * M + i] = co[uint64_t(lv.m[q]) * nnz + e];
    }
}

template <class T>
int upload(T** d, const std::vector<T>& h, hipStream_t s)
{
    CPTC_TRY(dalloc(d, h.size()));
    if (!h.empty())
        CPTC_HIP(hipMemcpyAsync(*d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice, s));
    return CPTC_OK;
}

}  // namespace

void free_units(DevUnitsN& u)
{
    dfree(u.d_unit6);
    dfree(u.d_outer_coords);
    dfree(u.d_lid);
    dfree(u.d_val);
    dfree(u.d_is_dense);
    u.nunits = u.dense_nnz = 0;
}

void free_view(DevViewN& v)
{
    dfree(v.d_sc);
    dfree(v.d_vals);
    dfree(v.d_skip);
    dfree(v.d_row);
    dfree(v.d_start);
    dfree(v.d_cnt);
    dfree(v.d_single);
    if (v.d_key) (void)hipFree(v.d_key);
    v.d_key = nullptr;
    v.key_bytes = 0;
    v.level_bits.clear();
    v.nnz = v.nseg = 0;
    v.level_modes.clear();
}

// generic.cu:578-725
int units_nd_device(int N, const uint64_t* dims, const uint32_t* d_coords, const double* d_vals,
                    uint64_t nnz, double threshold, const int inner[3], DevUnitsN& out,
                    hipStream_t s)
{
    (void)dims;
    free_units(out);
    out.cutoff = int(4096.0 * threshold);
    ModeSet ms{};
    out.outer.clear();
    for (int q = 0; q < 3; ++q) out.inner[q] = ms.inner[q] = inner[q];
    for (int m = 0; m < N; ++m)
        if (m != inner[0] && m != inner[1] && m != inner[2])
        {
            ms.outer[ms.nouter++] = m;
            out.outer.push_back(m);
        }
    CPTC_TRY(dalloc(&out.d_is_dense, nnz));
    if (nnz == 0) return CPTC_OK;
    CPTC_REQUIRE(nnz <= 0x7FFFFFFFull, CPTC_ERR_UNSUPPORTED, "units: nnz %llu > 0x7FFFFFFF",
                 (unsigned long long)nnz);
    CPTC_HIP(hipMemsetAsync(out.d_is_dense, 0, nnz, s));
    const unsigned g = grid_for(nnz, 256, 8192);

    Tmp<uint64_t> kin, kout;
    Tmp<uint32_t> iin, sidx;
    CPTC_TRY(kin.alloc(nnz));
    CPTC_TRY(kout.alloc(nnz));
    CPTC_TRY(iin.alloc(nnz));
    CPTC_TRY(sidx.alloc(nnz));
    hipLaunchKernelGGL(unit_keys_kernel, dim3(g), dim3(256), 0, s, d_coords, nnz, ms, kin.p, iin.p);
    CPTC_LAUNCHED();
    CPTC_TRY(sort_pairs(kin.p, kout.p, iin.p, sidx.p, nnz, 64, s));
    kin.reset();

    Tmp<uint64_t> ukeys;
    Tmp<uint32_t> counts, nruns_d;
    CPTC_TRY(ukeys.alloc(nnz));
    CPTC_TRY(counts.alloc(nnz));
    CPTC_TRY(nruns_d.alloc(1));
    CPTC_TRY(run_length(kout.p, nnz, ukeys.p, counts.p, nruns_d.p, s));
    uint32_t nruns = 0;
    CPTC_TRY(d2h_one(&nruns, nruns_d.p, s));

    Tmp<uint32_t> roff, first, rid, isunit, ufirst, urun;
    CPTC_TRY(roff.alloc(nruns));
    CPTC_TRY(first.alloc(nruns));
    CPTC_TRY(rid.alloc(nruns));
    CPTC_TRY(isunit.alloc(nruns));
    CPTC_TRY(ufirst.alloc(nruns));
    CPTC_TRY(urun.alloc(nruns));
    CPTC_TRY(exclusive_sum(counts.p, roff.p, nruns, s));
    const unsigned gr = grid_for(nruns, 256, 8192);
    hipLaunchKernelGGL(unit_runs_kernel, dim3(gr), dim3(256), 0, s, counts.p, roff.p, sidx.p,
                       nruns, out.cutoff, first.p, rid.p, isunit.p);
    CPTC_LAUNCHED();
    // number of units = sum of flags (last inclusive prefix)
    {
        Tmp<uint32_t> pre;
        CPTC_TRY(pre.alloc(nruns));
        CPTC_TRY(dev::inclusive_sum(isunit.p, pre.p, nruns, s));
        uint32_t nu = 0;
        CPTC_TRY(d2h_one(&nu, pre.p + (nruns - 1), s));
        out.nunits = nu;
    }
    if (out.nunits == 0) return CPTC_OK;
    // first-occurrence numbering: sort the units' first elements (the
    // non-units carry 0xFFFFFFFF and sort last)
    CPTC_TRY(sort_pairs(first.p, ufirst.p, rid.p, urun.p, nruns, 32, s));
    const uint32_t nu = uint32_t(out.nunits);
    Tmp<uint32_t> ucnt, ustart;
    CPTC_TRY(ucnt.alloc(nu));
    CPTC_TRY(ustart.alloc(nu));
    const unsigned gu = grid_for(nu, 256, 8192);
    hipLaunchKernelGGL(unit_counts_kernel, dim3(gu), dim3(256), 0, s, urun.p, counts.p, nu, ucnt.p);
    CPTC_LAUNCHED();
    CPTC_TRY(exclusive_sum(ucnt.p, ustart.p, nu, s));
    uint32_t last_start = 0, last_cnt = 0;
    CPTC_TRY(d2h_one(&last_start, ustart.p + (nu - 1), s));
    CPTC_TRY(d2h_one(&last_cnt, ucnt.p + (nu - 1), s));
    out.dense_nnz = uint64_t(last_start) + last_cnt;

    CPTC_TRY(dalloc(&out.d_unit6, size_t(nu) * 6));
    CPTC_TRY(dalloc(&out.d_outer_coords, size_t(nu) * ms.nouter));
    CPTC_TRY(dalloc(&out.d_lid, out.dense_nnz));
    CPTC_TRY(dalloc(&out.d_val, out.dense_nnz));
    hipLaunchKernelGGL(unit_meta_kernel, dim3(gu), dim3(256), 0, s, ufirst.p, ucnt.p, ustart.p, nu,
                       d_coords, nnz, ms, out.d_unit6, out.d_outer_coords);
    CPTC_LAUNCHED();
    hipLaunchKernelGGL(unit_pool_kernel, dim3(nu), dim3(256), 0, s, urun.p, roff.p, ucnt.p,
                       ustart.p, sidx.p, d_coords, d_vals, nnz, ms, out.d_lid, out.d_val,
                       out.d_is_dense);
    CPTC_LAUNCHED();
    CPTC_HIP(hipStreamSynchronize(s));
    return CPTC_OK;
}

int build_segments(const uint32_t* d_sorted_rows, uint64_t nnz, bool force_accumulate,
                   DevViewN& out, hipStream_t s);

// generic.cu:1848-1958
int view_nd_device(int N, const uint64_t* dims, int n, const uint32_t* d_coords,
                   const double* d_vals, const uint8_t* d_is_dense, bool force_accumulate,
                   uint64_t nnz, DevViewN& out, hipStream_t s)
{
    free_view(out);
    out.nnz = nnz;
    for (int m = 0; m < N; ++m)
        if (m != n) out.level_modes.push_back(m);
    if (nnz == 0) return CPTC_OK;
    CPTC_REQUIRE(nnz <= 0x7FFFFFFFull, CPTC_ERR_UNSUPPORTED, "views: nnz %llu > 0x7FFFFFFF",
                 (unsigned long long)nnz);
    const unsigned g = grid_for(nnz, 256, 8192);
    Tmp<uint32_t> skey, iin, order;
    CPTC_TRY(skey.alloc(nnz));
    CPTC_TRY(iin.alloc(nnz));
    CPTC_TRY(order.alloc(nnz));
    hipLaunchKernelGGL(iota_kernel, dim3(g), dim3(256), 0, s, iin.p, nnz);
    CPTC_LAUNCHED();
    const uint64_t dim = dims[n];
    CPTC_TRY(sort_pairs(d_coords + uint64_t(n) * nnz, skey.p, iin.p, order.p, nnz,
                        bit_width(dim > 0 ? dim - 1 : 0), s));
    iin.reset();
    CPTC_TRY(dalloc(&out.d_sc, size_t(N - 1) * nnz));
    CPTC_TRY(dalloc(&out.d_vals, nnz));
    if (d_is_dense) CPTC_TRY(dalloc(&out.d_skip, nnz));
    hipLaunchKernelGGL(view_gather_kernel, dim3(g), dim3(256), 0, s, order.p, d_coords, d_vals,
                       d_is_dense, nnz, N, n, out.d_sc, out.d_vals, out.d_skip);
    CPTC_LAUNCHED();
    CPTC_TRY(build_segments(skey.p, nnz, force_accumulate, out, s));
    CPTC_HIP(hipStreamSynchronize(s));
    return CPTC_OK;
}

// Row run lengths of the sorted target coordinates -> <= 1024-element
// segments in ascending row order (host), uploaded into `out`.
int build_segments(const uint32_t* d_sorted_rows, uint64_t nnz, bool force_accumulate,
                   DevViewN& out, hipStream_t s)
{
    Tmp<uint32_t> urow, counts, nruns_d;
    CPTC_TRY(urow.alloc(nnz));
    CPTC_TRY(counts.alloc(nnz));
    CPTC_TRY(nruns_d.alloc(1));
    CPTC_TRY(run_length(d_sorted_rows, nnz, urow.p, counts.p, nruns_d.p, s));
    uint32_t nruns = 0;
    CPTC_TRY(d2h_one(&nruns, nruns_d.p, s));
    std::vector<uint32_t> hrow(nruns), hcnt(nruns);
    CPTC_HIP(hipMemcpyAsync(hrow.data(), urow.p, nruns * sizeof(uint32_t), hipMemcpyDeviceToHost, s));
    CPTC_HIP(hipMemcpyAsync(hcnt.data(), counts.p, nruns * sizeof(uint32_t), hipMemcpyDeviceToHost, s));
    CPTC_HIP(hipStreamSynchronize(s));
    std::vector<uint32_t> row, start, cnt;
    std::vector<uint8_t> single;
    uint64_t off = 0;
    for (uint32_t r = 0; r < nruns; ++r)
    {
        const uint64_t rs = off, re = off + hcnt[r];
        const uint8_t one = (!force_accumulate && hcnt[r] <= CPTC_SEG) ? 1 : 0;
        for (uint64_t x = rs; x < re; x += CPTC_SEG)
        {
            row.push_back(hrow[r]);
            start.push_back(uint32_t(x));
            cnt.push_back(uint32_t(std::min<uint64_t>(CPTC_SEG, re - x)));
            single.push_back(one);
        }
        off = re;
    }
    out.nseg = row.size();
    CPTC_TRY(upload(&out.d_row, row, s));
    CPTC_TRY(upload(&out.d_start, start, s));
    CPTC_TRY(upload(&out.d_cnt, cnt, s));
    CPTC_TRY(upload(&out.d_single, single, s));
    return CPTC_OK;
}

int work_view_nd_device(int N, const uint64_t* dims, int n, const uint32_t* d_coords,
                        const double* d_vals, const uint8_t* d_is_dense, bool force_accumulate,
                        uint64_t nnz, DevViewN& out, hipStream_t s)
{
    free_view(out);
    // levels: the other modes by dimension, smallest first (ties: mode order)
    out.level_modes.clear();
    for (int m = 0; m < N; ++m)
        if (m != n) out.level_modes.push_back(m);
    std::stable_sort(out.level_modes.begin(), out.level_modes.end(),
                     [&](int a, int b) { return dims[a] < dims[b]; });
    if (nnz == 0) return CPTC_OK;
    CPTC_REQUIRE(nnz <= 0x7FFFFFFFull, CPTC_ERR_UNSUPPORTED, "views: nnz %llu > 0x7FFFFFFF",
                 (unsigned long long)nnz);
    const unsigned g = grid_for(nnz, 256, 8192);
    Tmp<uint32_t> perm, perm2, key, key2;
    CPTC_TRY(perm.alloc(nnz));
    CPTC_TRY(perm2.alloc(nnz));
    CPTC_TRY(key.alloc(nnz));
    CPTC_TRY(key2.alloc(nnz));
    uint64_t M = nnz;
    hipLaunchKernelGGL(iota_kernel, dim3(g), dim3(256), 0, s, perm2.p, nnz);
    CPTC_LAUNCHED();
    if (d_is_dense)
    {
        Tmp<uint8_t> keep;
        Tmp<uint64_t> cnt_d;
        CPTC_TRY(keep.alloc(nnz));
        CPTC_TRY(cnt_d.alloc(1));
        hipLaunchKernelGGL(keep_flags_kernel, dim3(g), dim3(256), 0, s, d_is_dense, nnz, keep.p);
        CPTC_LAUNCHED();
        size_t bytes = 0;
        CPTC_HIP(rocprim::select(nullptr, bytes, perm2.p, keep.p, perm.p, cnt_d.p, nnz, s));
        Tmp<char> tmp;
        CPTC_TRY(tmp.alloc(bytes ? bytes : 1));
        CPTC_HIP(rocprim::select(tmp.p, bytes, perm2.p, keep.p, perm.p, cnt_d.p, nnz, s));
        CPTC_TRY(d2h_one(&M, cnt_d.p, s));
    }
    else
    {
        std::swap(perm.p, perm2.p);
    }
    out.nnz = M;
    if (M == 0) return CPTC_OK;
    const unsigned gm = grid_for(M, 256, 8192);
    // least significant level first, the target coordinate last
    std::vector<int> passes(out.level_modes.rbegin(), out.level_modes.rend());
    passes.push_back(n);
    for (int m : passes)
    {
        hipLaunchKernelGGL(gather_keys_kernel, dim3(gm), dim3(256), 0, s,
                           d_coords + uint64_t(m) * nnz, perm.p, M, key.p);
        CPTC_LAUNCHED();
        CPTC_TRY(sort_pairs(key.p, key2.p, perm.p, perm2.p, M,
                            bit_width(dims[m] > 0 ? dims[m] - 1 : 0), s));
        std::swap(perm.p, perm2.p);
    }
    // perm = final order, key2 = its sorted target rows
    Levels lv{};
    const int nlev = N - 1;
    for (int q = 0; q < nlev; ++q) lv.m[q] = out.level_modes[q];
    CPTC_TRY(dalloc(&out.d_sc, size_t(nlev) * M));
    CPTC_TRY(dalloc(&out.d_vals, M));
    hipLaunchKernelGGL(work_gather_kernel, dim3(gm), dim3(256), 0, s, perm.p, d_coords, d_vals,
                       nnz, M, nlev, lv, out.d_sc, out.d_vals);
    CPTC_LAUNCHED();
    // packed level keys for the MTTKRP kernel (when the widths fit 64 bits)
    for (int q = 0; q < nlev; ++q)
    {
        const uint64_t d = dims[out.level_modes[q]];
        out.level_bits.push_back(std::max(1, bit_width(d > 0 ? d - 1 : 0)));
    }
    out.key_bytes = cptc_level_key_bytes(nlev, out.level_bits.data());
    if (out.key_bytes > 0)
    {
        CPTC_HIP(hipMalloc(&out.d_key, size_t(M) * size_t(out.key_bytes)));
        CPTC_TRY(cptc_pack_level_keys(nlev, out.d_sc, M, out.level_bits.data(), out.d_key,
                                      out.key_bytes, s));
    }
    CPTC_TRY(build_segments(key2.p, M, force_accumulate, out, s));
    CPTC_HIP(hipStreamSynchronize(s));
    return CPTC_OK;
}

}  // namespace cptc
