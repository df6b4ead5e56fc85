// Device-side layout of an order-3 tensor: CADR degrees and relabel, the
// hybrid 16^3 partition and the row-sorted per-mode views.
//
// Bit-exactness contract (with the reference's partition.cu / cadr.cu):
//   * partition: elements stably sorted by block_id; runs of equal block_id;
//     a run with count >= cutoff is a dense tile (ascending block_id, pool in
//     run order), the others form the residual in the same order;
//   * views: per mode a stable sort on (target, o1, o0) with 15-bit fields,
//     rows cut into <= 1024-element segments in ascending row order;
//   * CADR: relabel order = std::sort(iota, deg[a] > deg[b]) with libstdc++,
//     run on the host over the device-computed degrees.
// rocPRIM's LSD radix sort is stable, which is the property the contract
// needs; it sorts on exactly the key bits in use.
#include "dev_util.hpp"

#include <algorithm>
#include <numeric>
#include <vector>

#include "../host/layout.hpp"

namespace cptc {

namespace {

using dev::bit_width;
using dev::d2h_one;
using dev::dalloc;
using dev::dfree;
using dev::exclusive_sum;
using dev::inclusive_sum;
using dev::sort_pairs;
using dev::Tmp;

// ---------------------------------------------------------------- kernels --

__global__ void histogram_lds_kernel(const int32_t* __restrict__ m, size_t nnz, int dim,
                                     unsigned* __restrict__ deg)
{
    extern __shared__ unsigned h[];
    for (int x = threadIdx.x; x < dim; x += blockDim.x) h[x] = 0;
    __syncthreads();
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    for (size_t e = size_t(blockIdx.x) * blockDim.x + threadIdx.x; e < nnz; e += stride)
        atomicAdd(&h[m[e]], 1u);
    __syncthreads();
    for (int x = threadIdx.x; x < dim; x += blockDim.x)
        if (h[x]) atomicAdd(&deg[x], h[x]);
}

__global__ void histogram_global_kernel(const int32_t* __restrict__ m, size_t nnz,
                                        unsigned* __restrict__ deg)
{
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    for (size_t e = size_t(blockIdx.x) * blockDim.x + threadIdx.x; e < nnz; e += stride)
        atomicAdd(&deg[m[e]], 1u);
}

__global__ void relabel_kernel(int32_t* __restrict__ m, size_t nnz, const int32_t* __restrict__ perm)
{
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    for (size_t e = size_t(blockIdx.x) * blockDim.x + threadIdx.x; e < nnz; e += stride)
        m[e] = perm[m[e]];
}

__global__ void block_keys_kernel(const int32_t* __restrict__ m0, const int32_t* __restrict__ m1,
                                  const int32_t* __restrict__ m2, size_t nnz, uint64_t nbj,
                                  uint64_t nbk, uint64_t* __restrict__ key,
                                  uint32_t* __restrict__ idx)
{
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    for (size_t e = size_t(blockIdx.x) * blockDim.x + threadIdx.x; e < nnz; e += stride)
    {
        const uint64_t bi = uint64_t(m0[e]) / TILE, bj = uint64_t(m1[e]) / TILE,
                       bk = uint64_t(m2[e]) / TILE;
        key[e] = (bi * nbj + bj) * nbk + bk;
        idx[e] = uint32_t(e);
    }
}

__global__ void run_classify_kernel(const uint32_t* __restrict__ counts, size_t nruns, int cutoff,
                                    uint64_t* __restrict__ dcnt, uint64_t* __restrict__ scnt,
                                    uint32_t* __restrict__ isd)
{
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    for (size_t r = size_t(blockIdx.x) * blockDim.x + threadIdx.x; r < nruns; r += stride)
    {
        const bool d = int64_t(counts[r]) >= int64_t(cutoff);
        dcnt[r] = d ? counts[r] : 0;
        scnt[r] = d ? 0 : counts[r];
        isd[r] = d ? 1u : 0u;
    }
}

__global__ void tiles_kernel(const uint64_t* __restrict__ ukeys, const uint32_t* __restrict__ counts,
                             const uint32_t* __restrict__ isd, const uint32_t* __restrict__ tidx,
                             const uint64_t* __restrict__ doff, size_t nruns, uint64_t nbj,
                             uint64_t nbk, int32_t* __restrict__ tiles4,
                             uint64_t* __restrict__ pool_off)
{
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    for (size_t r = size_t(blockIdx.x) * blockDim.x + threadIdx.x; r < nruns; r += stride)
    {
        if (!isd[r]) continue;
        const uint64_t b = ukeys[r];
        const uint32_t t = tidx[r];
        const uint64_t bk = b % nbk, tmp = b / nbk;
        tiles4[4 * size_t(t) + 0] = int32_t(tmp / nbj);
        tiles4[4 * size_t(t) + 1] = int32_t(tmp % nbj);
        tiles4[4 * size_t(t) + 2] = int32_t(bk);
        tiles4[4 * size_t(t) + 3] = int32_t(counts[r]);
        pool_off[t] = doff[r];
    }
}

__global__ void head_flags_kernel(const uint64_t* __restrict__ skey, size_t n,
                                  uint32_t* __restrict__ head)
{
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    for (size_t p = size_t(blockIdx.x) * blockDim.x + threadIdx.x; p < n; p += stride)
        head[p] = (p == 0 || skey[p] != skey[p - 1]) ? 1u : 0u;
}

__global__ void scatter_kernel(const uint32_t* __restrict__ sidx, const uint32_t* __restrict__ runid,
                               const uint64_t* __restrict__ rstart, const uint32_t* __restrict__ isd,
                               const uint64_t* __restrict__ doff, const uint64_t* __restrict__ soff,
                               size_t nnz, const int32_t* __restrict__ m0,
                               const int32_t* __restrict__ m1, const int32_t* __restrict__ m2,
                               const double* __restrict__ val, int32_t* __restrict__ pool_lid,
                               double* __restrict__ pool_val, uint32_t* __restrict__ si,
                               uint32_t* __restrict__ sj, uint32_t* __restrict__ sk,
                               double* __restrict__ sv)
{
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    for (size_t p = size_t(blockIdx.x) * blockDim.x + threadIdx.x; p < nnz; p += stride)
    {
        const uint32_t r = runid[p] - 1u;
        const uint64_t k = p - rstart[r];
        const uint32_t e = sidx[p];
        const int i = m0[e], j = m1[e], l = m2[e];
        if (isd[r])
        {
            const uint64_t d = doff[r] + k;
            pool_lid[d] = ((i % TILE) * TILE + (j % TILE)) * TILE + (l % TILE);
            pool_val[d] = val[e];
        }
        else
        {
            const uint64_t d = soff[r] + k;
            si[d] = uint32_t(i);
            sj[d] = uint32_t(j);
            sk[d] = uint32_t(l);
            sv[d] = val[e];
        }
    }
}

__global__ void add_u64_kernel(const uint64_t* __restrict__ a, const uint64_t* __restrict__ b,
                               uint64_t* __restrict__ c, size_t n)
{
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    for (size_t x = size_t(blockIdx.x) * blockDim.x + threadIdx.x; x < n; x += stride)
        c[x] = a[x] + b[x];
}

__global__ void pack_kernel(const uint32_t* __restrict__ i, const uint32_t* __restrict__ j,
                            const uint32_t* __restrict__ k, size_t n, uint64_t* __restrict__ out)
{
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    for (size_t e = size_t(blockIdx.x) * blockDim.x + threadIdx.x; e < n; e += stride)
        out[e] = (uint64_t(i[e]) << 30) | (uint64_t(j[e]) << 15) | uint64_t(k[e]);
}

// key = (target << 30) | (o1 << 15) | o0: mode 0 (i, k, j), 1 (j, k, i), 2 (k, j, i)
__global__ void view_keys_kernel(const uint64_t* __restrict__ packed, size_t n, int mode,
                                 uint64_t* __restrict__ key, uint32_t* __restrict__ idx)
{
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    for (size_t e = size_t(blockIdx.x) * blockDim.x + threadIdx.x; e < n; e += stride)
    {
        const uint64_t pc = packed[e];
        const uint64_t a = (pc >> 30) & 0x7FFF, b = (pc >> 15) & 0x7FFF, c = pc & 0x7FFF;
        key[e] = mode == 0 ? (a << 30) | (c << 15) | b
               : mode == 1 ? (b << 30) | (c << 15) | a
                           : (c << 30) | (b << 15) | a;
        idx[e] = uint32_t(e);
    }
}

__global__ void gather_kernel(const uint32_t* __restrict__ perm, const uint64_t* __restrict__ packed,
                              const double* __restrict__ val, size_t n,
                              uint64_t* __restrict__ oc, double* __restrict__ ov)
{
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    for (size_t p = size_t(blockIdx.x) * blockDim.x + threadIdx.x; p < n; p += stride)
    {
        const uint32_t e = perm[p];
        oc[p] = packed[e];
        ov[p] = val[e];
    }
}

__global__ void decode_tiles_kernel(const int32_t* __restrict__ tiles4,
                                    const uint64_t* __restrict__ off, const int32_t* __restrict__ lid,
                                    const double* __restrict__ pval, uint32_t* __restrict__ oi,
                                    uint32_t* __restrict__ oj, uint32_t* __restrict__ ok,
                                    double* __restrict__ ov)
{
    const size_t t = blockIdx.x;
    const int b0 = tiles4[4 * t] * TILE, b1 = tiles4[4 * t + 1] * TILE,
              b2 = tiles4[4 * t + 2] * TILE;
    const uint64_t lo = off[t], hi = off[t + 1];
    for (uint64_t e = lo + threadIdx.x; e < hi; e += blockDim.x)
    {
        const int l = lid[e];
        oi[e] = uint32_t(b0 + (l >> 8));
        oj[e] = uint32_t(b1 + ((l >> 4) & 15));
        ok[e] = uint32_t(b2 + (l & 15));
        ov[e] = pval[e];
    }
}

// Degrees of one mode into d_deg (dim entries).
int degrees(const int32_t* d_m, size_t nnz, uint64_t dim, unsigned* d_deg, hipStream_t s)
{
    CPTC_HIP(hipMemsetAsync(d_deg, 0, dim * sizeof(unsigned), s));
    if (nnz == 0) return CPTC_OK;
    const unsigned grid = grid_for(nnz, 256, 2048);
    if (dim * sizeof(unsigned) <= 128 * 1024)
    {
        static cptc::DeviceOnce attr;
        CPTC_HIP(attr.lds_limit({reinterpret_cast<const void*>(histogram_lds_kernel)},
                                128 * 1024));
        hipLaunchKernelGGL(histogram_lds_kernel, dim3(grid), dim3(256), dim * sizeof(unsigned), s,
                           d_m, nnz, int(dim), d_deg);
    }
    else
    {
        hipLaunchKernelGGL(histogram_global_kernel, dim3(grid), dim3(256), 0, s, d_m, nnz, d_deg);
    }
    CPTC_LAUNCHED();
    return CPTC_OK;
}

// Blocked-view sort key: (target >> lg_tb, o1 >> lg_kb) of the packed
// (i<<30 | j<<15 | k) coordinate, target / o1 by mode as the views.
__global__ void blk_keys_kernel(const uint64_t* __restrict__ coords, size_t n, int mode,
                                int lg_tb, int lg_kb, uint32_t* __restrict__ key,
                                uint32_t* __restrict__ idx)
{
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    const int kbits = 15 - lg_kb;
    for (size_t e = size_t(blockIdx.x) * blockDim.x + threadIdx.x; e < n; e += stride)
    {
        const uint64_t pc = coords[e];
        const uint32_t i = uint32_t(pc >> 30) & 0x7FFFu, j = uint32_t(pc >> 15) & 0x7FFFu,
                       k = uint32_t(pc) & 0x7FFFu;
        const uint32_t t = mode == 0 ? i : (mode == 1 ? j : k);
        const uint32_t o1 = mode == 2 ? j : k;
        key[e] = ((t >> lg_tb) << kbits) | (o1 >> lg_kb);
        idx[e] = uint32_t(e);
    }
}

__global__ void blk_gather_kernel(const uint32_t* __restrict__ idx,
                                  const uint64_t* __restrict__ cin, const double* __restrict__ vin,
                                  size_t n, uint64_t* __restrict__ cout, double* __restrict__ vout)
{
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    for (size_t e = size_t(blockIdx.x) * blockDim.x + threadIdx.x; e < n; e += stride)
    {
        const uint32_t s = idx[e];
        cout[e] = cin[s];
        vout[e] = vin[s];
    }
}

}  // namespace

// ------------------------------------------------------------- lifecycle --

void free_coo(DevCoo3& c)
{
    for (auto& p : c.d_m) dfree(p);
    dfree(c.d_val);
    c.nnz = 0;
}

void free_partition(DevPartition3& p)
{
    dfree(p.d_tiles4);
    dfree(p.d_pool_off);
    dfree(p.d_pool_lid);
    dfree(p.d_pool_val);
    for (auto& q : p.d_sp) dfree(q);
    dfree(p.d_sp_val);
    p.ntiles = 0;
    p.dense_nnz = p.sparse_nnz = 0;
    p.h_tiles4.clear();
    p.h_pool_off.clear();
}

void free_blk(DevBlk3& b)
{
    for (int m = 0; m < 3; ++m)
    {
        dfree(b.d_coords[m]);
        dfree(b.d_vals[m]);
        for (uint32_t** p : {&b.d_span_start[m], &b.d_span_cnt[m], &b.d_span_kb[m],
                             &b.d_chunk_span0[m], &b.d_chunk_nspan[m], &b.d_chunk_tb[m]})
            dfree(*p);
        b.nspan[m] = b.nchunk[m] = 0;
    }
    b.nnz = 0;
    b.ready = false;
}

void free_views(DevViews3& v)
{
    for (int m = 0; m < 3; ++m)
    {
        dfree(v.d_coords[m]);
        dfree(v.d_vals[m]);
        dfree(v.d_blk_row[m]);
        dfree(v.d_blk_start[m]);
        dfree(v.d_blk_cnt[m]);
        v.nseg[m] = 0;
    }
    v.nnz = 0;
    v.ready = false;
}

int upload_coo3(const uint32_t* idx, const double* val, size_t nnz, const uint64_t dims[3],
                DevCoo3& out, hipStream_t s)
{
    free_coo(out);
    for (int m = 0; m < 3; ++m) out.dims[m] = dims[m];
    out.nnz = nnz;
    if (nnz == 0) return CPTC_OK;
    for (int m = 0; m < 3; ++m)
    {
        CPTC_TRY(dalloc(&out.d_m[m], nnz));
        CPTC_HIP(hipMemcpyAsync(out.d_m[m], idx + size_t(m) * nnz, nnz * sizeof(int32_t),
                                hipMemcpyHostToDevice, s));
    }
    CPTC_TRY(dalloc(&out.d_val, nnz));
    CPTC_HIP(hipMemcpyAsync(out.d_val, val, nnz * sizeof(double), hipMemcpyHostToDevice, s));
    CPTC_HIP(hipStreamSynchronize(s));
    return CPTC_OK;
}

// cadr.cu:23-81
int cadr3_device(DevCoo3& c, std::vector<int32_t> perm[3], int32_t* d_perm[3], int relabel,
                 hipStream_t s)
{
    for (int m = 0; m < 3; ++m)
    {
        const uint64_t dim = c.dims[m];
        Tmp<unsigned> deg;
        CPTC_TRY(deg.alloc(dim));
        CPTC_TRY(degrees(c.d_m[m], c.nnz, dim, deg.p, s));
        std::vector<unsigned> h(dim);
        CPTC_HIP(hipMemcpyAsync(h.data(), deg.p, dim * sizeof(unsigned), hipMemcpyDeviceToHost, s));
        CPTC_HIP(hipStreamSynchronize(s));
        std::vector<int> sorted(dim);
        std::iota(sorted.begin(), sorted.end(), 0);
        std::sort(sorted.begin(), sorted.end(), [&](int a, int b) { return h[a] > h[b]; });
        perm[m].assign(dim, 0);
        for (int nw = 0; nw < int(dim); ++nw) perm[m][sorted[nw]] = nw;
        CPTC_TRY(dalloc(&d_perm[m], dim));
        CPTC_HIP(hipMemcpyAsync(d_perm[m], perm[m].data(), dim * sizeof(int32_t),
                                hipMemcpyHostToDevice, s));
        if (relabel && c.nnz)
        {
            hipLaunchKernelGGL(relabel_kernel, dim3(grid_for(c.nnz, 256, 8192)), dim3(256), 0, s,
                               c.d_m[m], c.nnz, d_perm[m]);
            CPTC_LAUNCHED();
        }
    }
    CPTC_HIP(hipStreamSynchronize(s));
    return CPTC_OK;
}

// partition.cu:581-1493
int partition3_device(const DevCoo3& c, double threshold, int num_cus, DevPartition3& out,
                      hipStream_t s)
{
    free_partition(out);
    for (int m = 0; m < 3; ++m) out.nblk[m] = (c.dims[m] + TILE - 1) / TILE;
    if (threshold > 0.0)
    {
        int cut = int(4096.0 * threshold);
        out.cutoff = std::min(std::max(cut, 1), 4096);
    }
    const size_t nnz = c.nnz;
    if (nnz == 0)
    {
        out.h_pool_off.assign(1, 0);
        CPTC_TRY(dalloc(&out.d_pool_off, 1));
        CPTC_HIP(hipMemsetAsync(out.d_pool_off, 0, sizeof(uint64_t), s));
        return CPTC_OK;
    }
    CPTC_REQUIRE(nnz <= size_t(UINT32_MAX), CPTC_ERR_UNSUPPORTED,
                 "partition: nnz %zu exceeds uint32 range", nnz);
    const unsigned g = grid_for(nnz, 256, 8192);
    Tmp<uint64_t> kin, kout;
    Tmp<uint32_t> iin, iout;
    CPTC_TRY(kin.alloc(nnz));
    CPTC_TRY(kout.alloc(nnz));
    CPTC_TRY(iin.alloc(nnz));
    CPTC_TRY(iout.alloc(nnz));
    hipLaunchKernelGGL(block_keys_kernel, dim3(g), dim3(256), 0, s, c.d_m[0], c.d_m[1], c.d_m[2],
                       nnz, uint64_t(out.nblk[1]), uint64_t(out.nblk[2]), kin.p, iin.p);
    CPTC_LAUNCHED();
    const uint64_t maxkey = out.nblk[0] * out.nblk[1] * out.nblk[2] - 1;
    CPTC_TRY(sort_pairs(kin.p, kout.p, iin.p, iout.p, nnz, bit_width(maxkey), s));
    // runs of equal block_id
    Tmp<uint64_t> ukeys;
    Tmp<uint32_t> counts, nruns_d;
    CPTC_TRY(ukeys.alloc(nnz));
    CPTC_TRY(counts.alloc(nnz));
    CPTC_TRY(nruns_d.alloc(1));
    {
        size_t bytes = 0;
        CPTC_HIP(rocprim::run_length_encode(nullptr, bytes, kout.p, nnz, ukeys.p, counts.p,
                                            nruns_d.p, s));
        Tmp<char> tmp;
        CPTC_TRY(tmp.alloc(bytes ? bytes : 1));
        CPTC_HIP(rocprim::run_length_encode(tmp.p, bytes, kout.p, nnz, ukeys.p, counts.p,
                                            nruns_d.p, s));
    }
    uint32_t nruns = 0;
    CPTC_TRY(d2h_one(&nruns, nruns_d.p, s));
    if (threshold <= 0.0)
    {
        // partition.cu:1030-1098
        std::vector<uint32_t> hc(nruns);
        CPTC_HIP(hipMemcpyAsync(hc.data(), counts.p, nruns * sizeof(uint32_t),
                                hipMemcpyDeviceToHost, s));
        CPTC_HIP(hipStreamSynchronize(s));
        const double sm_scale = double(num_cus > 0 ? num_cus : 24) / 24.0;
        const double rate_wmma = 1.20 / sm_scale;
        const double rate_cuda = 0.688 / sm_scale;
        const double frac_dense = rate_cuda / (rate_wmma + rate_cuda);
        const size_t target = size_t(double(nnz) * frac_dense);
        std::vector<int> cs(hc.begin(), hc.end());
        std::sort(cs.begin(), cs.end(), std::greater<int>());
        size_t acc = 0;
        int cut = 1;
        for (int x : cs)
        {
            acc += size_t(x);
            if (acc >= target)
            {
                cut = x;
                break;
            }
        }
        out.cutoff = cut;
    }
    Tmp<uint64_t> dcnt, scnt, doff, soff, rstart, r64;
    Tmp<uint32_t> isd, tidx;
    CPTC_TRY(dcnt.alloc(nruns));
    CPTC_TRY(scnt.alloc(nruns));
    CPTC_TRY(doff.alloc(nruns));
    CPTC_TRY(soff.alloc(nruns));
    CPTC_TRY(rstart.alloc(nruns));
    CPTC_TRY(r64.alloc(nruns));
    CPTC_TRY(isd.alloc(nruns));
    CPTC_TRY(tidx.alloc(nruns));
    const unsigned gr = grid_for(nruns, 256, 8192);
    hipLaunchKernelGGL(run_classify_kernel, dim3(gr), dim3(256), 0, s, counts.p, size_t(nruns),
                       out.cutoff, dcnt.p, scnt.p, isd.p);
    CPTC_LAUNCHED();
    CPTC_TRY(exclusive_sum(dcnt.p, doff.p, nruns, s));
    CPTC_TRY(exclusive_sum(scnt.p, soff.p, nruns, s));
    CPTC_TRY(exclusive_sum(isd.p, tidx.p, nruns, s));
    // run starts = exclusive sum of all counts = dense + sparse offsets
    hipLaunchKernelGGL(add_u64_kernel, dim3(gr), dim3(256), 0, s, doff.p, soff.p, rstart.p,
                       size_t(nruns));
    CPTC_LAUNCHED();
    uint64_t last_d = 0, last_s = 0, last_doff = 0, last_soff = 0;
    uint32_t last_t = 0, last_isd = 0;
    CPTC_TRY(d2h_one(&last_d, dcnt.p + (nruns - 1), s));
    CPTC_TRY(d2h_one(&last_s, scnt.p + (nruns - 1), s));
    CPTC_TRY(d2h_one(&last_doff, doff.p + (nruns - 1), s));
    CPTC_TRY(d2h_one(&last_soff, soff.p + (nruns - 1), s));
    CPTC_TRY(d2h_one(&last_t, tidx.p + (nruns - 1), s));
    CPTC_TRY(d2h_one(&last_isd, isd.p + (nruns - 1), s));
    out.dense_nnz = size_t(last_doff + last_d);
    out.sparse_nnz = size_t(last_soff + last_s);
    out.ntiles = int64_t(last_t) + int64_t(last_isd);
    CPTC_TRY(dalloc(&out.d_tiles4, size_t(out.ntiles) * 4));
    CPTC_TRY(dalloc(&out.d_pool_off, size_t(out.ntiles) + 1));
    CPTC_TRY(dalloc(&out.d_pool_lid, out.dense_nnz));
    CPTC_TRY(dalloc(&out.d_pool_val, out.dense_nnz));
    for (int m = 0; m < 3; ++m) CPTC_TRY(dalloc(&out.d_sp[m], out.sparse_nnz));
    CPTC_TRY(dalloc(&out.d_sp_val, out.sparse_nnz));
    if (out.ntiles > 0)
    {
        hipLaunchKernelGGL(tiles_kernel, dim3(gr), dim3(256), 0, s, ukeys.p, counts.p, isd.p,
                           tidx.p, doff.p, size_t(nruns), uint64_t(out.nblk[1]),
                           uint64_t(out.nblk[2]), out.d_tiles4, out.d_pool_off);
        CPTC_LAUNCHED();
    }
    const uint64_t dn = out.dense_nnz;
    CPTC_HIP(hipMemcpyAsync(out.d_pool_off + out.ntiles, &dn, sizeof(uint64_t),
                            hipMemcpyHostToDevice, s));
    // per-position run id (1-based) from head flags
    Tmp<uint32_t> head, runid;
    CPTC_TRY(head.alloc(nnz));
    CPTC_TRY(runid.alloc(nnz));
    hipLaunchKernelGGL(head_flags_kernel, dim3(g), dim3(256), 0, s, kout.p, nnz, head.p);
    CPTC_LAUNCHED();
    CPTC_TRY(inclusive_sum(head.p, runid.p, nnz, s));
    hipLaunchKernelGGL(scatter_kernel, dim3(g), dim3(256), 0, s, iout.p, runid.p, rstart.p, isd.p,
                       doff.p, soff.p, nnz, c.d_m[0], c.d_m[1], c.d_m[2], c.d_val, out.d_pool_lid,
                       out.d_pool_val, out.d_sp[0], out.d_sp[1], out.d_sp[2], out.d_sp_val);
    CPTC_LAUNCHED();
    out.h_tiles4.resize(size_t(out.ntiles) * 4);
    out.h_pool_off.resize(size_t(out.ntiles) + 1);
    if (out.ntiles > 0)
        CPTC_HIP(hipMemcpyAsync(out.h_tiles4.data(), out.d_tiles4,
                                out.h_tiles4.size() * sizeof(int32_t), hipMemcpyDeviceToHost, s));
    CPTC_HIP(hipMemcpyAsync(out.h_pool_off.data(), out.d_pool_off,
                            out.h_pool_off.size() * sizeof(uint64_t), hipMemcpyDeviceToHost, s));
    CPTC_HIP(hipStreamSynchronize(s));
    return CPTC_OK;
}

// partition.cu:1865-2329
int views3_device(const uint32_t* d_i, const uint32_t* d_j, const uint32_t* d_k,
                  const double* d_val, size_t nnz, const uint64_t dims[3], DevViews3& out,
                  hipStream_t s)
{
    free_views(out);
    out.nnz = nnz;
    if (nnz == 0) return CPTC_OK;
    CPTC_REQUIRE(dims[0] < 32768 && dims[1] < 32768 && dims[2] < 32768, CPTC_ERR_UNSUPPORTED,
                 "views: dims %llu x %llu x %llu exceed the 15-bit packed layout (< 32768)",
                 (unsigned long long)dims[0], (unsigned long long)dims[1],
                 (unsigned long long)dims[2]);
    CPTC_REQUIRE(nnz <= size_t(UINT32_MAX), CPTC_ERR_UNSUPPORTED, "views: nnz %zu too large", nnz);
    const unsigned g = grid_for(nnz, 256, 8192);
    Tmp<uint64_t> packed, kin, kout;
    Tmp<uint32_t> iin, iout;
    CPTC_TRY(packed.alloc(nnz));
    CPTC_TRY(kin.alloc(nnz));
    CPTC_TRY(kout.alloc(nnz));
    CPTC_TRY(iin.alloc(nnz));
    CPTC_TRY(iout.alloc(nnz));
    hipLaunchKernelGGL(pack_kernel, dim3(g), dim3(256), 0, s, d_i, d_j, d_k, nnz, packed.p);
    CPTC_LAUNCHED();
    const uint32_t* tgt[3] = {d_i, d_j, d_k};
    for (int mode = 0; mode < 3; ++mode)
    {
        hipLaunchKernelGGL(view_keys_kernel, dim3(g), dim3(256), 0, s, packed.p, nnz, mode, kin.p,
                           iin.p);
        CPTC_LAUNCHED();
        CPTC_TRY(sort_pairs(kin.p, kout.p, iin.p, iout.p, nnz, 45, s));
        CPTC_TRY(dalloc(&out.d_coords[mode], nnz));
        CPTC_TRY(dalloc(&out.d_vals[mode], nnz));
        hipLaunchKernelGGL(gather_kernel, dim3(g), dim3(256), 0, s, iout.p, packed.p, d_val, nnz,
                           out.d_coords[mode], out.d_vals[mode]);
        CPTC_LAUNCHED();
        // row segments: counts per target row, rows ascending
        const uint64_t dim = dims[mode];
        Tmp<unsigned> deg;
        CPTC_TRY(deg.alloc(dim));
        CPTC_TRY(degrees(reinterpret_cast<const int32_t*>(tgt[mode]), nnz, dim, deg.p, s));
        std::vector<unsigned> h(dim);
        CPTC_HIP(hipMemcpyAsync(h.data(), deg.p, dim * sizeof(unsigned), hipMemcpyDeviceToHost, s));
        CPTC_HIP(hipStreamSynchronize(s));
        std::vector<uint32_t> br, bs, bc;
        uint64_t cum = 0;
        for (uint64_t r = 0; r < dim; ++r)
        {
            const uint64_t cnt = h[r];
            for (uint64_t c0 = 0; c0 < cnt; c0 += CPTC_SEG)
            {
                br.push_back(uint32_t(r));
                bs.push_back(uint32_t(cum + c0));
                bc.push_back(uint32_t(std::min<uint64_t>(CPTC_SEG, cnt - c0)));
            }
            cum += cnt;
        }
        out.nseg[mode] = br.size();
        CPTC_TRY(dalloc(&out.d_blk_row[mode], br.size()));
        CPTC_TRY(dalloc(&out.d_blk_start[mode], bs.size()));
        CPTC_TRY(dalloc(&out.d_blk_cnt[mode], bc.size()));
        CPTC_HIP(hipMemcpyAsync(out.d_blk_row[mode], br.data(), br.size() * 4,
                                hipMemcpyHostToDevice, s));
        CPTC_HIP(hipMemcpyAsync(out.d_blk_start[mode], bs.data(), bs.size() * 4,
                                hipMemcpyHostToDevice, s));
        CPTC_HIP(hipMemcpyAsync(out.d_blk_cnt[mode], bc.data(), bc.size() * 4,
                                hipMemcpyHostToDevice, s));
        CPTC_HIP(hipStreamSynchronize(s));
    }
    out.ready = true;
    return CPTC_OK;
}

int blk_views3_device(const DevViews3& v, const uint64_t dims[3], int lg_tb, int lg_kb,
                      uint32_t chunk, uint32_t stage_min, DevBlk3& out, hipStream_t s)
{
    free_blk(out);
    CPTC_REQUIRE(v.ready && lg_tb >= 0 && lg_tb <= 15 && lg_kb >= 0 && lg_kb <= 15 && chunk >= 1,
                 CPTC_ERR_ARG, "blocked views: bad arguments");
    out.lg_tb = lg_tb;
    out.lg_kb = lg_kb;
    out.nnz = v.nnz;
    const size_t n = v.nnz;
    if (n == 0)
    {
        out.ready = true;
        return CPTC_OK;
    }
    const int kbits = 15 - lg_kb;
    const int end_bit = (15 - lg_tb) + kbits;
    const unsigned g = grid_for(n, 256, 8192);
    Tmp<uint32_t> kin, kout, iin, iout, ukeys, counts, nruns;
    CPTC_TRY(kin.alloc(n));
    CPTC_TRY(kout.alloc(n));
    CPTC_TRY(iin.alloc(n));
    CPTC_TRY(iout.alloc(n));
    CPTC_TRY(ukeys.alloc(n));
    CPTC_TRY(counts.alloc(n));
    CPTC_TRY(nruns.alloc(1));
    for (int mode = 0; mode < 3; ++mode)
    {
        hipLaunchKernelGGL(blk_keys_kernel, dim3(g), dim3(256), 0, s, v.d_coords[mode], n, mode,
                           lg_tb, lg_kb, kin.p, iin.p);
        CPTC_LAUNCHED();
        CPTC_TRY(sort_pairs(kin.p, kout.p, iin.p, iout.p, n, end_bit, s));
        CPTC_TRY(dalloc(&out.d_coords[mode], n));
        CPTC_TRY(dalloc(&out.d_vals[mode], n));
        hipLaunchKernelGGL(blk_gather_kernel, dim3(g), dim3(256), 0, s, iout.p,
                           v.d_coords[mode], v.d_vals[mode], n, out.d_coords[mode],
                           out.d_vals[mode]);
        CPTC_LAUNCHED();
        CPTC_TRY(dev::run_length(kout.p, n, ukeys.p, counts.p, nruns.p, s));
        uint32_t nr = 0;
        CPTC_TRY(d2h_one(&nr, nruns.p, s));
        std::vector<uint32_t> hk(nr), hc(nr);
        CPTC_HIP(hipMemcpyAsync(hk.data(), ukeys.p, nr * sizeof(uint32_t), hipMemcpyDeviceToHost, s));
        CPTC_HIP(hipMemcpyAsync(hc.data(), counts.p, nr * sizeof(uint32_t), hipMemcpyDeviceToHost, s));
        CPTC_HIP(hipStreamSynchronize(s));
        // spans: a staged block pair (split into pieces of <= chunk elements),
        // or consecutive unstaged block pairs of one row block (<= chunk)
        std::vector<uint32_t> ss, sc, sk, stb;
        uint64_t start = 0;
        for (uint32_t r = 0; r < nr; ++r)
        {
            const uint32_t tb = hk[r] >> kbits, kb = hk[r] & ((1u << kbits) - 1);
            const uint32_t cnt = hc[r];
            if (cnt >= stage_min)
            {
                for (uint32_t c0 = 0; c0 < cnt; c0 += chunk)
                {
                    ss.push_back(uint32_t(start + c0));
                    sc.push_back(std::min(chunk, cnt - c0));
                    sk.push_back(kb | 0x80000000u);
                    stb.push_back(tb);
                }
            }
            else if (!ss.empty() && stb.back() == tb && (sk.back() >> 31) == 0 &&
                     uint64_t(sc.back()) + cnt <= chunk)
                sc.back() += cnt;
            else
            {
                ss.push_back(uint32_t(start));
                sc.push_back(cnt);
                sk.push_back(kb);
                stb.push_back(tb);
            }
            start += cnt;
        }
        // chunks: consecutive spans of one row block, <= chunk elements (or one span)
        std::vector<uint32_t> c0v, cnv, ctv;
        uint64_t tot = 0;
        for (uint32_t x = 0; x < uint32_t(ss.size()); ++x)
        {
            if (!c0v.empty() && ctv.back() == stb[x] && tot + sc[x] <= chunk)
            {
                cnv.back()++;
                tot += sc[x];
                continue;
            }
            c0v.push_back(x);
            cnv.push_back(1);
            ctv.push_back(stb[x]);
            tot = sc[x];
        }
        {
            // chunks dispatched in the order of their first run-level block
            // (then target block): the workgroups resident at one time stage
            // and gather the rows of a few run-level blocks, which then stay
            // in L2 (config 3: 2.30 -> 2.20 ms per launch against target-block
            // order; by chunk size, longest first: 2.51-2.62)
            std::vector<uint32_t> ci(c0v.size());
            for (size_t x = 0; x < c0v.size(); ++x) ci[x] = uint32_t(x);
            std::stable_sort(ci.begin(), ci.end(), [&](uint32_t a, uint32_t b) {
                const uint32_t ka = sk[c0v[a]] & 0x7FFFFFFFu, kb = sk[c0v[b]] & 0x7FFFFFFFu;
                return ka < kb;
            });
            std::vector<uint32_t> a0(c0v.size()), an(c0v.size()), at(c0v.size());
            for (size_t x = 0; x < ci.size(); ++x)
            {
                a0[x] = c0v[ci[x]];
                an[x] = cnv[ci[x]];
                at[x] = ctv[ci[x]];
            }
            c0v.swap(a0);
            cnv.swap(an);
            ctv.swap(at);
        }
        out.nspan[mode] = ss.size();
        out.nchunk[mode] = c0v.size();
        auto up = [&](uint32_t** dst, const std::vector<uint32_t>& src) -> int {
            CPTC_TRY(dalloc(dst, src.size()));
            CPTC_HIP(hipMemcpyAsync(*dst, src.data(), src.size() * sizeof(uint32_t),
                                    hipMemcpyHostToDevice, s));
            return CPTC_OK;
        };
        CPTC_TRY(up(&out.d_span_start[mode], ss));
        CPTC_TRY(up(&out.d_span_cnt[mode], sc));
        CPTC_TRY(up(&out.d_span_kb[mode], sk));
        CPTC_TRY(up(&out.d_chunk_span0[mode], c0v));
        CPTC_TRY(up(&out.d_chunk_nspan[mode], cnv));
        CPTC_TRY(up(&out.d_chunk_tb[mode], ctv));
        CPTC_HIP(hipStreamSynchronize(s));
    }
    (void)dims;
    out.ready = true;
    return CPTC_OK;
}

// partition.cu:2335-2517
int dense_views3_device(const DevPartition3& p, const uint64_t dims[3], DevViews3& out,
                        hipStream_t s)
{
    free_views(out);
    if (p.ntiles == 0 || p.dense_nnz == 0) return CPTC_OK;
    Tmp<uint32_t> i, j, k;
    Tmp<double> v;
    CPTC_TRY(i.alloc(p.dense_nnz));
    CPTC_TRY(j.alloc(p.dense_nnz));
    CPTC_TRY(k.alloc(p.dense_nnz));
    CPTC_TRY(v.alloc(p.dense_nnz));
    hipLaunchKernelGGL(decode_tiles_kernel, dim3(unsigned(p.ntiles)), dim3(256), 0, s, p.d_tiles4,
                       p.d_pool_off, p.d_pool_lid, p.d_pool_val, i.p, j.p, k.p, v.p);
    CPTC_LAUNCHED();
    return views3_device(i.p, j.p, k.p, v.p, p.dense_nnz, dims, out, s);
}

}  // namespace cptc

extern "C" int cptc_cadr3(int32_t* m0, int32_t* m1, int32_t* m2, size_t nnz,
                          const uint64_t dims[3], int32_t* perm0, int32_t* perm1, int32_t* perm2,
                          int relabel)
{
    CPTC_REQUIRE(dims && perm0 && perm1 && perm2 && (nnz == 0 || (m0 && m1 && m2)), CPTC_ERR_ARG,
                 "cptc_cadr3: null argument");
    {
        const int32_t* hm[3] = {m0, m1, m2};
        for (int m = 0; m < 3; ++m)
            for (size_t e = 0; e < nnz; ++e)
                CPTC_REQUIRE(hm[m][e] >= 0 && uint64_t(hm[m][e]) < dims[m], CPTC_ERR_ARG,
                             "cptc_cadr3: mode %d index %d outside [0, %llu)", m, hm[m][e],
                             (unsigned long long)dims[m]);
    }
    hipStream_t s = nullptr;
    CPTC_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    cptc::DevCoo3 c;
    for (int m = 0; m < 3; ++m) c.dims[m] = dims[m];
    c.nnz = nnz;
    int32_t* host[3] = {m0, m1, m2};
    int32_t* out[3] = {perm0, perm1, perm2};
    int32_t* d_perm[3] = {nullptr, nullptr, nullptr};
    std::vector<int32_t> perm[3];
    int rc = CPTC_OK;
    for (int m = 0; m < 3 && rc == CPTC_OK && nnz; ++m)
    {
        rc = cptc::dalloc(&c.d_m[m], nnz);
        if (rc == CPTC_OK &&
            hipMemcpyAsync(c.d_m[m], host[m], nnz * 4, hipMemcpyHostToDevice, s) != hipSuccess)
            rc = CPTC_ERR_HIP;
    }
    if (rc == CPTC_OK) rc = cptc::cadr3_device(c, perm, d_perm, relabel, s);
    for (int m = 0; m < 3 && rc == CPTC_OK; ++m)
    {
        std::memcpy(out[m], perm[m].data(), perm[m].size() * sizeof(int32_t));
        if (relabel && nnz &&
            hipMemcpyAsync(host[m], c.d_m[m], nnz * 4, hipMemcpyDeviceToHost, s) != hipSuccess)
            rc = CPTC_ERR_HIP;
    }
    if (rc == CPTC_OK && hipStreamSynchronize(s) != hipSuccess) rc = CPTC_ERR_HIP;
    for (auto& p : d_perm) cptc::dfree(p);
    cptc::free_coo(c);
    (void)hipStreamDestroy(s);
    return rc;
}
