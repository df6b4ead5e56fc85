// The C++ interface of include/{tensor,cadr,partition,sparse,dense,solver,
// als,common,compute_fit,generic}.hpp: the reference's function names and
// argument meanings over this library's device layout and kernels.  As in
// the reference, device and argument errors print a message and exit the
// process (the C ABI underneath returns status codes instead).
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <iostream>
#include <random>
#include <string>
#include <vector>

#include "als.hpp"
#include "cadr.hpp"
#include "common.hpp"
#include "compute_fit.hpp"
#include "cptc_hip.h"
#include "dense.hpp"
#include "generic.hpp"
#include "host_util.hpp"
#include "layout.hpp"
#include "partition.hpp"
#include "sgd.hpp"
#include "solver.hpp"
#include "sparse.hpp"

namespace {

[[noreturn]] void die(const char* where, int rc)
{
    std::cerr << "[cpTC] " << where << " failed (" << rc << "): " << cptc_last_error()
              << std::endl;
    std::exit(EXIT_FAILURE);
}

#define API_TRY(where, expr)                 \
    do                                       \
    {                                        \
        const int rc_ = (expr);              \
        if (rc_ != CPTC_OK) die(where, rc_); \
    } while (0)

template <class T>
T* dalloc(size_t n)
{
    T* p = nullptr;
    if (n) CHECK_HIP(hipMalloc(reinterpret_cast<void**>(&p), n * sizeof(T)));
    return p;
}

template <class T>
void dfree(T*& p)
{
    if (p) (void)hipFree(p);
    p = nullptr;
}

int num_cus()
{
    int dev = 0;
    CHECK_HIP(hipGetDevice(&dev));
    hipDeviceProp_t prop{};
    CHECK_HIP(hipGetDeviceProperties(&prop, dev));
    return prop.multiProcessorCount;
}

// HybridCOOTensor <-> the library's layout structs (shallow, non-owning)
cptc::DevPartition3 part_of(const HybridCOOTensor& h)
{
    cptc::DevPartition3 p;
    p.cutoff = h.dense_cutoff;
    for (int m = 0; m < 3; ++m) p.nblk[m] = h.num_blocks[m];
    p.ntiles = h.num_dense_tiles;
    p.d_tiles4 = h.d_tiles4;
    p.d_pool_off = h.d_pool_off;
    p.dense_nnz = h.dense_nnz;
    p.d_pool_lid = h.d_dense_coords_pool;
    p.d_pool_val = h.d_dense_values_pool;
    p.sparse_nnz = h.sparse_nnz;
    p.d_sp[0] = h.d_sp_i;
    p.d_sp[1] = h.d_sp_j;
    p.d_sp[2] = h.d_sp_k;
    p.d_sp_val = h.d_sp_val;
    p.h_tiles4.reserve(h.dense_tiles.size() * 4);
    p.h_pool_off.assign(1, 0);
    for (const DenseTile16& t : h.dense_tiles)
    {
        p.h_tiles4.insert(p.h_tiles4.end(), {t.block_idx[0], t.block_idx[1], t.block_idx[2], t.nnz});
        p.h_pool_off.push_back(p.h_pool_off.back() + uint64_t(t.nnz));
    }
    return p;
}

cptc::DevViews3 views_of(const HybridCOOTensor& h)
{
    cptc::DevViews3 v;
    v.nnz = h.sparse_nnz;
    v.ready = h.mttkrp_ready && h.sparse_nnz > 0;
    for (int m = 0; m < 3; ++m)
    {
        v.d_coords[m] = h.d_sp2_coords[m];
        v.d_vals[m] = h.d_sp2_val[m];
        v.nseg[m] = h.mttkrp_blocks[m];
        v.d_blk_row[m] = h.d_blk_row[m];
        v.d_blk_start[m] = h.d_blk_start[m];
        v.d_blk_cnt[m] = h.d_blk_cnt[m];
    }
    return v;
}

void take_views(HybridCOOTensor& h, cptc::DevViews3& v)
{
    for (int m = 0; m < 3; ++m)
    {
        h.d_sp2_coords[m] = v.d_coords[m];
        h.d_sp2_val[m] = v.d_vals[m];
        h.d_blk_row[m] = v.d_blk_row[m];
        h.d_blk_start[m] = v.d_blk_start[m];
        h.d_blk_cnt[m] = v.d_blk_cnt[m];
        h.mttkrp_blocks[m] = v.nseg[m];
    }
    h.mttkrp_ready = true;
    v = cptc::DevViews3{};   // ownership moved
}

const float* tiles_f32(const HybridCOOTensor& h, hipStream_t s)
{
    if (h.num_dense_tiles <= 0) return nullptr;
    if (!h.d_tile_f32)
    {
        h.d_tile_f32 = dalloc<float>(size_t(h.num_dense_tiles) * 4096);
        API_TRY("dense tile packing",
                cptc_dense_tiles_pack3(h.d_dense_coords_pool, h.d_dense_values_pool, h.d_pool_off,
                                       size_t(h.num_dense_tiles), h.d_tile_f32, s));
    }
    return h.d_tile_f32;
}

}  // namespace

// ------------------------------------------------------------- tensor.hpp --

void load_tns_file(const std::string& filename, COOTensor& tensor)
{
    cptc_coo c{};
    API_TRY("load_tns_file", cptc_tns_load3(filename.c_str(), &c));
    free_coo_tensor(tensor);
    tensor.nnz = c.nnz;
    for (int m = 0; m < 3; ++m) tensor.dims[m] = c.dims[m];
    const size_t n = c.nnz;
    tensor.h_m0.assign(c.idx, c.idx + n);
    tensor.h_m1.assign(c.idx + n, c.idx + 2 * n);
    tensor.h_m2.assign(c.idx + 2 * n, c.idx + 3 * n);
    tensor.h_val.assign(c.val, c.val + n);
    cptc_coo_free(&c);
    tensor.d_m0 = dalloc<int>(n);
    tensor.d_m1 = dalloc<int>(n);
    tensor.d_m2 = dalloc<int>(n);
    tensor.d_val = dalloc<double>(n);
    if (n)
    {
        CHECK_HIP(hipMemcpy(tensor.d_m0, tensor.h_m0.data(), n * sizeof(int), hipMemcpyHostToDevice));
        CHECK_HIP(hipMemcpy(tensor.d_m1, tensor.h_m1.data(), n * sizeof(int), hipMemcpyHostToDevice));
        CHECK_HIP(hipMemcpy(tensor.d_m2, tensor.h_m2.data(), n * sizeof(int), hipMemcpyHostToDevice));
        CHECK_HIP(hipMemcpy(tensor.d_val, tensor.h_val.data(), n * sizeof(double),
                            hipMemcpyHostToDevice));
    }
}

void free_coo_tensor(COOTensor& tensor)
{
    dfree(tensor.d_m0);
    dfree(tensor.d_m1);
    dfree(tensor.d_m2);
    dfree(tensor.d_val);
    tensor = COOTensor{};
}

// --------------------------------------------------------------- cadr.hpp --

TensorPermutation compute_cadr_reordering(const COOTensor& tensor)
{
    std::cout << "[CADR] Computing degree-based mode reordering mapping..." << std::endl;
    TensorPermutation perm;
    perm.perm0.resize(tensor.dims[0]);
    perm.perm1.resize(tensor.dims[1]);
    perm.perm2.resize(tensor.dims[2]);
    const uint64_t dims[3] = {tensor.dims[0], tensor.dims[1], tensor.dims[2]};
    // relabel = 0: the coordinate arrays are only read
    API_TRY("compute_cadr_reordering",
            cptc_cadr3(const_cast<int*>(tensor.h_m0.data()), const_cast<int*>(tensor.h_m1.data()),
                       const_cast<int*>(tensor.h_m2.data()), tensor.nnz, dims, perm.perm0.data(),
                       perm.perm1.data(), perm.perm2.data(), 0));
    perm.d_perm0 = dalloc<int>(tensor.dims[0]);
    perm.d_perm1 = dalloc<int>(tensor.dims[1]);
    perm.d_perm2 = dalloc<int>(tensor.dims[2]);
    CHECK_HIP(hipMemcpy(perm.d_perm0, perm.perm0.data(), tensor.dims[0] * sizeof(int),
                        hipMemcpyHostToDevice));
    CHECK_HIP(hipMemcpy(perm.d_perm1, perm.perm1.data(), tensor.dims[1] * sizeof(int),
                        hipMemcpyHostToDevice));
    CHECK_HIP(hipMemcpy(perm.d_perm2, perm.perm2.data(), tensor.dims[2] * sizeof(int),
                        hipMemcpyHostToDevice));
    return perm;
}

void apply_cadr_reordering(COOTensor& tensor, const TensorPermutation& perm)
{
    std::cout << "[CADR] Applying mode permutation to COO tensor coordinates..." << std::endl;
    for (size_t e = 0; e < tensor.nnz; ++e)
    {
        tensor.h_m0[e] = perm.perm0[size_t(tensor.h_m0[e])];
        tensor.h_m1[e] = perm.perm1[size_t(tensor.h_m1[e])];
        tensor.h_m2[e] = perm.perm2[size_t(tensor.h_m2[e])];
    }
    if (tensor.nnz && tensor.d_m0)
    {
        CHECK_HIP(hipMemcpy(tensor.d_m0, tensor.h_m0.data(), tensor.nnz * sizeof(int),
                            hipMemcpyHostToDevice));
        CHECK_HIP(hipMemcpy(tensor.d_m1, tensor.h_m1.data(), tensor.nnz * sizeof(int),
                            hipMemcpyHostToDevice));
        CHECK_HIP(hipMemcpy(tensor.d_m2, tensor.h_m2.data(), tensor.nnz * sizeof(int),
                            hipMemcpyHostToDevice));
    }
}

void unpermute_factor_matrices(double* d_A_perm, double* d_B_perm, double* d_C_perm,
                               double** d_factors_orig, const TensorPermutation& perm,
                               const size_t* dims, int R)
{
    std::cout << "[CADR] Unpermuting factor matrices back to original order..." << std::endl;
    const double* src[3] = {d_A_perm, d_B_perm, d_C_perm};
    const int* dp[3] = {perm.d_perm0, perm.d_perm1, perm.d_perm2};
    for (int m = 0; m < 3; ++m)
        API_TRY("unpermute_factor_matrices",
                cptc_unpermute_factor(src[m], d_factors_orig[m], dp[m], dims[m], R, nullptr));
    CHECK_HIP(hipDeviceSynchronize());
}

void free_cadr_permutation(TensorPermutation& perm)
{
    dfree(perm.d_perm0);
    dfree(perm.d_perm1);
    dfree(perm.d_perm2);
}

// ---------------------------------------------------------- partition.hpp --

void partition_tensor_hybrid_gpu(const COOTensor& tensor, HybridCOOTensor& hybrid,
                                 double dense_threshold, hipStream_t stream)
{
    free_hybrid_tensor(hybrid);
    cptc::DevCoo3 c;
    for (int m = 0; m < 3; ++m) c.dims[m] = tensor.dims[m];
    c.nnz = tensor.nnz;
    c.d_m[0] = tensor.d_m0;
    c.d_m[1] = tensor.d_m1;
    c.d_m[2] = tensor.d_m2;
    c.d_val = tensor.d_val;
    cptc::DevPartition3 p;
    API_TRY("partition_tensor_hybrid_gpu",
            cptc::partition3_device(c, dense_threshold, num_cus(), p, stream));
    for (int m = 0; m < 3; ++m)
    {
        hybrid.dims[m] = tensor.dims[m];
        hybrid.num_blocks[m] = p.nblk[m];
    }
    hybrid.num_dense_tiles = int(p.ntiles);
    hybrid.sparse_nnz = p.sparse_nnz;
    hybrid.d_sp_i = p.d_sp[0];
    hybrid.d_sp_j = p.d_sp[1];
    hybrid.d_sp_k = p.d_sp[2];
    hybrid.d_sp_val = p.d_sp_val;
    hybrid.d_tiles4 = p.d_tiles4;
    hybrid.d_pool_off = p.d_pool_off;
    hybrid.d_dense_coords_pool = p.d_pool_lid;
    hybrid.d_dense_values_pool = p.d_pool_val;
    hybrid.dense_nnz = p.dense_nnz;
    hybrid.dense_coords_capacity = hybrid.dense_values_capacity = p.dense_nnz;
    hybrid.dense_cutoff = p.cutoff;
    hybrid.dense_tiles.resize(size_t(p.ntiles));
    for (int64_t t = 0; t < p.ntiles; ++t)
    {
        DenseTile16& d = hybrid.dense_tiles[size_t(t)];
        for (int q = 0; q < 3; ++q) d.block_idx[q] = p.h_tiles4[4 * size_t(t) + q];
        d.nnz = p.h_tiles4[4 * size_t(t) + 3];
        d.d_coords = p.d_pool_lid + p.h_pool_off[size_t(t)];
        d.d_values = p.d_pool_val + p.h_pool_off[size_t(t)];
    }
}

void partition_tensor_hybrid(const COOTensor& tensor, HybridCOOTensor& hybrid,
                             double dense_threshold)
{
    partition_tensor_hybrid_gpu(tensor, hybrid, dense_threshold, nullptr);
    CHECK_HIP(hipDeviceSynchronize());
}

void free_hybrid_tensor(HybridCOOTensor& hybrid)
{
    dfree(hybrid.d_sp_i);
    dfree(hybrid.d_sp_j);
    dfree(hybrid.d_sp_k);
    dfree(hybrid.d_sp_val);
    for (int m = 0; m < 3; ++m)
    {
        dfree(hybrid.d_sp2_coords[m]);
        dfree(hybrid.d_sp2_val[m]);
        dfree(hybrid.d_blk_row[m]);
        dfree(hybrid.d_blk_start[m]);
        dfree(hybrid.d_blk_cnt[m]);
    }
    dfree(hybrid.d_dense_coords_pool);
    dfree(hybrid.d_dense_values_pool);
    dfree(hybrid.d_dense_k_offsets);
    dfree(hybrid.d_tiles4);
    dfree(hybrid.d_pool_off);
    dfree(hybrid.d_tile_f32);
    for (int m = 0; m < 3; ++m)
    {
        dfree(hybrid.d_tile_cmask[m]);
        dfree(hybrid.d_tile_segoff[m]);
        dfree(hybrid.d_tile_cseg[m]);
        hybrid.tile_nseg[m] = 0;
    }
    hybrid = HybridCOOTensor{};
}

void build_mttkrp_views(HybridCOOTensor& hybrid, hipStream_t stream)
{
    const uint64_t dims[3] = {hybrid.dims[0], hybrid.dims[1], hybrid.dims[2]};
    if (hybrid.sparse_nnz > 0)
    {
        cptc::DevViews3 v;
        API_TRY("build_mttkrp_views",
                cptc::views3_device(hybrid.d_sp_i, hybrid.d_sp_j, hybrid.d_sp_k, hybrid.d_sp_val,
                                    hybrid.sparse_nnz, dims, v, stream));
        take_views(hybrid, v);
    }
    hybrid.mttkrp_ready = true;
    // the residual COO is no longer needed (partition.cu:2310-2329)
    dfree(hybrid.d_sp_i);
    dfree(hybrid.d_sp_j);
    dfree(hybrid.d_sp_k);
    dfree(hybrid.d_sp_val);
}

void build_dense_mttkrp_views(HybridCOOTensor& hybrid, HybridCOOTensor& dense_out,
                              hipStream_t stream)
{
    free_hybrid_tensor(dense_out);
    for (int m = 0; m < 3; ++m) dense_out.dims[m] = hybrid.dims[m];
    if (hybrid.num_dense_tiles <= 0 || hybrid.dense_nnz == 0) return;
    const uint64_t dims[3] = {hybrid.dims[0], hybrid.dims[1], hybrid.dims[2]};
    cptc::DevViews3 v;
    API_TRY("build_dense_mttkrp_views",
            cptc::dense_views3_device(part_of(hybrid), dims, v, stream));
    dense_out.sparse_nnz = v.nnz;
    take_views(dense_out, v);
}

// ------------------------------------------------------- sparse / dense --

void compute_sparse_mttkrp_async(const HybridCOOTensor& hybrid, int target_mode,
                                 const double* d_A, const double* d_B, const double* d_C,
                                 double* d_FtV, double* d_FtF, int R, hipStream_t stream)
{
    (void)d_FtF;
    if (!hybrid.mttkrp_ready || hybrid.sparse_nnz == 0) return;
    const int m = target_mode;
    const double* F1 = m == 0 ? d_B : d_A;
    const double* F2 = m == 2 ? d_B : d_C;
    API_TRY("compute_sparse_mttkrp_async",
            cptc_mttkrp_sparse3(m, hybrid.d_sp2_coords[m], hybrid.d_sp2_val[m],
                                hybrid.d_blk_row[m], hybrid.d_blk_start[m], hybrid.d_blk_cnt[m],
                                hybrid.mttkrp_blocks[m], F1, F2, d_FtV, R, stream));
}

void compute_sparse_mttkrp_async(const HybridCOOTensor& hybrid, int target_mode,
                                 const double* d_A, const double* d_B, const double* d_C,
                                 double* d_FtV, double* d_FtF, int R, hipStream_t stream,
                                 size_t start_idx, size_t count)
{
    // sparse.cu:877-955: clamp the range; the whole residual takes the
    // row-sorted segment kernel, a strict sub-range the per-element one
    if (!hybrid.mttkrp_ready || hybrid.sparse_nnz == 0 || count == 0 ||
        start_idx >= hybrid.sparse_nnz)
        return;
    count = std::min(count, hybrid.sparse_nnz - start_idx);
    if (start_idx == 0 && count == hybrid.sparse_nnz)
    {
        compute_sparse_mttkrp_async(hybrid, target_mode, d_A, d_B, d_C, d_FtV, d_FtF, R, stream);
        return;
    }
    const int m = target_mode;
    const double* F1 = m == 0 ? d_B : d_A;
    const double* F2 = m == 2 ? d_B : d_C;
    API_TRY("compute_sparse_mttkrp_async",
            cptc_mttkrp_sparse3_range(m, hybrid.d_sp2_coords[m], hybrid.d_sp2_val[m], start_idx,
                                      count, F1, F2, d_FtV, R, stream));
}

void compute_sparse_mttkrp(const HybridCOOTensor& hybrid, int target_mode, const double* d_A,
                           const double* d_B, const double* d_C, double* d_FtV, double* d_FtF,
                           int R)
{
    compute_sparse_mttkrp_async(hybrid, target_mode, d_A, d_B, d_C, d_FtV, d_FtF, R, nullptr);
    CHECK_HIP(hipDeviceSynchronize());
}

void compute_dense_mttkrp_async(const HybridCOOTensor& hybrid, int mode, double* d_A,
                                double* d_B, double* d_C, double* d_FtV, double* d_FtF, int R,
                                hipStream_t stream)
{
    (void)d_FtF;
    if (hybrid.num_dense_tiles <= 0) return;
    const float* t = tiles_f32(hybrid, stream);
    const size_t nt = size_t(hybrid.num_dense_tiles);
    const int sw = cptc::tile_kernel_switch("ALS_TILE_KERNEL");
    if (sw < 0 ? cptc::tile_b3_auto(nt, R) : sw == 1)
    {
        // the split-bf16 kernel over the mode's compacted split image (built
        // once per tensor and mode; the dense image when the compacted one
        // exceeds the kernel's 32-bit offsets); its operand workspace is per
        // call and stream-ordered, so calls on different streams do not share it
        if (!hybrid.d_tile_cmask[mode])
        {
            hybrid.d_tile_cmask[mode] = dalloc<uint32_t>(nt * 64);
            hybrid.d_tile_segoff[mode] = dalloc<uint32_t>(nt + 1);
            API_TRY("dense tile compaction",
                    cptc_dense_tiles_compact3_mask(t, nt, mode, hybrid.d_tile_cmask[mode],
                                                   hybrid.d_tile_segoff[mode],
                                                   &hybrid.tile_nseg[mode], stream));
            if (hybrid.tile_nseg[mode] * 16u < 0xFFFFFFF0ull)
            {
                hybrid.d_tile_cseg[mode] =
                    dalloc<uint32_t>(std::max<uint64_t>(hybrid.tile_nseg[mode], 1) * 4);
                API_TRY("dense tile compaction",
                        cptc_dense_tiles_compact3_fill(t, nt, mode, hybrid.d_tile_cmask[mode],
                                                       hybrid.d_tile_segoff[mode],
                                                       hybrid.d_tile_cseg[mode], stream));
            }
        }
        const uint64_t md = uint64_t(std::max({hybrid.dims[0], hybrid.dims[1], hybrid.dims[2]}));
        const size_t wsb = cptc_tile_operands_bytes(md, R);
        void* ws = nullptr;
        CHECK_HIP(hipMallocAsync(&ws, wsb, stream));
        const int rc =
            hybrid.d_tile_cseg[mode]
                ? cptc_mttkrp_dense_tiles3_cws(
                      mode, hybrid.d_tiles4, hybrid.d_tile_cmask[mode], hybrid.d_tile_segoff[mode],
                      hybrid.d_tile_cseg[mode], hybrid.tile_nseg[mode], nt, nullptr, nullptr, 0,
                      d_A, d_B, d_C, d_FtV, R, int(hybrid.dims[0]), int(hybrid.dims[1]),
                      int(hybrid.dims[2]), ws, wsb, stream)
                : cptc_mttkrp_dense_tiles3_ws(mode, hybrid.d_tiles4, t, nt, nullptr, nullptr, 0,
                                              d_A, d_B, d_C, d_FtV, R, int(hybrid.dims[0]),
                                              int(hybrid.dims[1]), int(hybrid.dims[2]), ws, wsb,
                                              stream);
        CHECK_HIP(hipFreeAsync(ws, stream));
        API_TRY("compute_dense_mttkrp_async", rc);
        return;
    }
    API_TRY("compute_dense_mttkrp_async",
            cptc_mttkrp_dense_tiles3(mode, hybrid.d_tiles4, t, size_t(hybrid.num_dense_tiles),
                                     nullptr, nullptr, 0, d_A,
                                     d_B, d_C, d_FtV, R, int(hybrid.dims[0]), int(hybrid.dims[1]),
                                     int(hybrid.dims[2]), stream));
}

void compute_dense_mttkrp(const HybridCOOTensor& hybrid, int mode, double* d_A, double* d_B,
                          double* d_C, double* d_FtV, double* d_FtF, int R)
{
    compute_dense_mttkrp_async(hybrid, mode, d_A, d_B, d_C, d_FtV, d_FtF, R, nullptr);
    CHECK_HIP(hipDeviceSynchronize());
}

void compute_mttkrp_merged_async(const HybridCOOTensor& hybrid, int mode, double* d_A,
                                 double* d_B, double* d_C, double* d_FtV, double* d_FtF, int R,
                                 hipStream_t stream)
{
    // dense.cu:2258-2511: one grid for the tiles and the residual segments;
    // shapes the merged kernel does not take (odd R, R > 128, unaligned
    // factors) queue the two launches back to back instead
    const bool aligned = ((reinterpret_cast<uintptr_t>(d_A) | reinterpret_cast<uintptr_t>(d_B) |
                           reinterpret_cast<uintptr_t>(d_C)) & 15) == 0;
    if (R % 2 == 0 && R <= 128 && aligned)
    {
        const int m = mode;
        const bool views = hybrid.mttkrp_ready && hybrid.sparse_nnz > 0;
        const float* t = hybrid.num_dense_tiles > 0 ? tiles_f32(hybrid, stream) : nullptr;
        int every = 0, flags = 0;
        cptc::merged_switches(every, flags);
        API_TRY("compute_mttkrp_merged_async",
                cptc_mttkrp_merged3_ex(m, hybrid.d_tiles4, t, size_t(std::max<int64_t>(0, hybrid.num_dense_tiles)),
                                    nullptr, nullptr, 0, views ? hybrid.d_sp2_coords[m] : nullptr,
                                    views ? hybrid.d_sp2_val[m] : nullptr,
                                    views ? hybrid.d_blk_row[m] : nullptr,
                                    views ? hybrid.d_blk_start[m] : nullptr,
                                    views ? hybrid.d_blk_cnt[m] : nullptr,
                                    views ? size_t(hybrid.mttkrp_blocks[m]) : 0, d_A, d_B, d_C,
                                    d_FtV, R, int(hybrid.dims[0]), int(hybrid.dims[1]),
                                    int(hybrid.dims[2]), every, flags, stream));
        return;
    }
    compute_dense_mttkrp_async(hybrid, mode, d_A, d_B, d_C, d_FtV, d_FtF, R, stream);
    compute_sparse_mttkrp_async(hybrid, mode, d_A, d_B, d_C, d_FtV, d_FtF, R, stream);
}

// ------------------------------------------------------------------ sgd --

void execute_sgd_decomposition(const HybridCOOTensor& hybrid, double* d_A, double* d_B,
                               double* d_C, double* d_lambda_out, int R, int max_iters,
                               double gamma, int batch_size, unsigned long long seed)
{
    // sgd.cu:315-319
    if (hybrid.sparse_nnz == 0 || !hybrid.mttkrp_ready)
    {
        std::cerr << "[SGD] sparse views not ready." << std::endl;
        return;
    }
    const uint64_t dims[3] = {hybrid.dims[0], hybrid.dims[1], hybrid.dims[2]};
    API_TRY("execute_sgd_decomposition",
            cptc_sgd3_run(hybrid.d_sp2_coords[0], hybrid.d_sp2_val[0], hybrid.sparse_nnz, d_A,
                          d_B, d_C, dims, d_lambda_out, R, max_iters, gamma,
                          uint32_t(batch_size > 0 ? batch_size : 1), seed, 1, nullptr, nullptr));
}

// --------------------------------------------------------------- solver --

void init_svd_workspace(SVDWorkspace& ws, int R) { ws.R = R; }

void free_svd_workspace(SVDWorkspace& ws) { ws.R = 0; }

bool solve_als_system_svd_nosync(const SVDWorkspace& ws, void* blas, double* d_FtF,
                                 double* d_FtV, double* d_Factor, size_t dim_len, int R)
{
    (void)blas;
    if (R <= 0 || (ws.R && ws.R != R)) return false;
    return cptc_solve_pinv(d_FtF, d_FtV, d_Factor, dim_len, R, nullptr, nullptr) == CPTC_OK;
}

bool solve_als_system_svd(const SVDWorkspace& ws, void* blas, double* d_FtF, double* d_FtV,
                          double* d_Factor, size_t dim_len, int R)
{
    if (!solve_als_system_svd_nosync(ws, blas, d_FtF, d_FtV, d_Factor, dim_len, R)) return false;
    return hipDeviceSynchronize() == hipSuccess;
}

// ------------------------------------------------------------------ als --

void execute_als_decomposition(const COOTensor& tensor, HybridCOOTensor& hybrid,
                               const HybridCOOTensor& hybrid_dense, double* d_A, double* d_B,
                               double* d_C, double* d_lambda_out, int R, int max_iters,
                               double lambda_reg)
{
    (void)lambda_reg;
    if (R <= 0 || max_iters <= 0 || !d_A || !d_B || !d_C || !d_lambda_out)
    {
        std::cerr << "[ALS ERROR] Invalid parameters." << std::endl;
        return;
    }
    std::cout << "[ALS] Starting CP-ALS: rank=" << R << ", max_iters=" << max_iters
              << " (pseudoinverse solve, per-iter normalization)" << std::endl;
    // als.cu:523-535: MFMA tiles when the dense part has no FP64 views
    const bool use_mfma =
        hybrid.num_dense_tiles > 0 && !hybrid_dense.mttkrp_ready && hybrid.mttkrp_ready;
    float* tiles = use_mfma ? const_cast<float*>(tiles_f32(hybrid, nullptr)) : nullptr;
    const uint64_t dims[3] = {tensor.dims[0], tensor.dims[1], tensor.dims[2]};
    double fit = 0.0;
    const auto t0 = std::chrono::steady_clock::now();
    API_TRY("execute_als_decomposition",
            cptc::als3_execute(dims, part_of(hybrid), views_of(hybrid), views_of(hybrid_dense),
                               tiles, use_mfma, d_A, d_B, d_C, d_lambda_out, R, max_iters, true,
                               &fit));
    // als.cu:765-789: exact RMSE over the stored elements, fit report, lambda
    const double rmse = calculate_rmse(hybrid, hybrid_dense, d_A, d_B, d_C, d_lambda_out, R);
    print_fit_report(hybrid, hybrid_dense, d_A, d_B, d_C, d_lambda_out, R, rmse, "final");
    std::cout << "[ALS] Final RMSE=" << rmse << std::endl;
    std::vector<double> lam(size_t(R), 0.0);
    CHECK_HIP(hipMemcpy(lam.data(), d_lambda_out, size_t(R) * sizeof(double),
                        hipMemcpyDeviceToHost));
    std::cout << "[ALS] Lambda:";
    for (double x : lam) std::cout << " " << x;
    std::cout << std::endl;
    std::cout << "[ALS] Total time="
              << std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0)
                     .count()
              << " ms" << std::endl;
}

// --------------------------------------------------------------- common --

void debug_device_state()
{
    int dev = 0, n = 0;
    CHECK_HIP(hipGetDeviceCount(&n));
    CHECK_HIP(hipGetDevice(&dev));
    hipDeviceProp_t p{};
    CHECK_HIP(hipGetDeviceProperties(&p, dev));
    size_t fr = 0, tot = 0;
    CHECK_HIP(hipMemGetInfo(&fr, &tot));
    std::cout << "[Device] " << n << " device(s); using " << dev << ": " << p.name << " ("
              << p.gcnArchName << "), " << p.multiProcessorCount << " CUs, "
              << double(tot) / (1 << 30) << " GiB (" << double(fr) / (1 << 30) << " GiB free), "
              << p.clockRate / 1000 << " MHz" << std::endl;
}

void init_factors_random(double** d_factors, const size_t* dims, int R)
{
    std::mt19937 gen(42);
    std::uniform_real_distribution<double> dis(0.0, 1.0);
    for (int m = 0; m < 3; ++m)
    {
        std::vector<double> h(dims[m] * size_t(R));
        for (double& x : h) x = dis(gen);
        CHECK_HIP(hipMemcpy(d_factors[m], h.data(), h.size() * sizeof(double),
                            hipMemcpyHostToDevice));
    }
}

void clamp_factor_thrust(double* d_factor, size_t size, double min_val, double max_val)
{
    if (!d_factor || size == 0) return;
    API_TRY("clamp_factor_thrust", cptc_clamp(d_factor, size, min_val, max_val, nullptr));
    CHECK_HIP(hipDeviceSynchronize());
}

void compute_residual_and_norm_sq(const HybridCOOTensor& h1, const HybridCOOTensor& h2,
                                  const double* d_A, const double* d_B, const double* d_C,
                                  const double* d_lambda, bool has_lambda, int R,
                                  double& h_res_sq, double& h_x_sq)
{
    double* d2 = dalloc<double>(2);
    CHECK_HIP(hipMemset(d2, 0, 2 * sizeof(double)));
    const double* lam = has_lambda ? d_lambda : nullptr;
    for (const HybridCOOTensor* h : {&h1, &h2})
        if (h->mttkrp_ready && h->sparse_nnz > 0)
            API_TRY("compute_residual_and_norm_sq",
                    cptc_residual3_view(h->d_sp2_coords[0], h->d_sp2_val[0], h->sparse_nnz, d_A,
                                        d_B, d_C, lam, R, d2, nullptr));
    if (h1.num_dense_tiles > 0 && !h2.mttkrp_ready)
        API_TRY("compute_residual_and_norm_sq",
                cptc_residual3_tiles(h1.d_tiles4, h1.d_pool_off, h1.d_dense_coords_pool,
                                     h1.d_dense_values_pool, size_t(h1.num_dense_tiles), d_A, d_B,
                                     d_C, lam, R, d2, nullptr));
    double h[2] = {0, 0};
    CHECK_HIP(hipMemcpy(h, d2, sizeof(h), hipMemcpyDeviceToHost));
    dfree(d2);
    h_res_sq = h[0];
    h_x_sq = h[1];
}

static size_t stored_nnz(const HybridCOOTensor& h1, const HybridCOOTensor& h2)
{
    return h1.sparse_nnz + (h2.mttkrp_ready ? h2.sparse_nnz : h1.dense_nnz);
}

double calculate_rmse(const HybridCOOTensor& h1, const HybridCOOTensor& h2, double* d_A,
                      double* d_B, double* d_C, const double* d_lambda, int R)
{
    double res = 0.0, x2 = 0.0;
    compute_residual_and_norm_sq(h1, h2, d_A, d_B, d_C, d_lambda, d_lambda != nullptr, R, res, x2);
    const size_t n = stored_nnz(h1, h2);
    return n ? std::sqrt(std::max(res, 0.0) / double(n)) : 0.0;
}

double compute_fit(const HybridCOOTensor& h1, const HybridCOOTensor& h2, const double* d_A,
                   const double* d_B, const double* d_C, const double* d_lambda, int R)
{
    double res = 0.0, x2 = 0.0;
    compute_residual_and_norm_sq(h1, h2, d_A, d_B, d_C, d_lambda, d_lambda != nullptr, R, res, x2);
    const double xn = std::sqrt(x2), rn = std::sqrt(std::max(res, 0.0));
    double fit = xn > 0.0 ? 1.0 - rn / xn : 0.0;
    if (fit < 0.0 && fit > -1e-10) fit = 0.0;
    if (fit > 1.0 && fit < 1.0 + 1e-10) fit = 1.0;
    const size_t n = stored_nnz(h1, h2);
    std::cout << "[Fit] ||X||_F = " << xn << " ||X-Xhat||_F = " << rn
              << " RMSE = " << (n ? std::sqrt(std::max(res, 0.0) / double(n)) : 0.0)
              << " fit = " << fit << std::endl;
    return fit;
}

void print_fit_report(const HybridCOOTensor& h1, const HybridCOOTensor& h2, const double* d_A,
                      const double* d_B, const double* d_C, const double* d_lambda, int R,
                      double rmse, const char* tag)
{
    if (!tag) tag = "";
    const double fit = compute_fit(h1, h2, d_A, d_B, d_C, d_lambda, R);
    std::cout << "\n[Fit Report] " << tag << " R=" << R << " RMSE=" << rmse << " fit=" << fit
              << " (" << fit * 100.0 << "% Frobenius energy explained)\n"
              << std::endl;
}

// -------------------------------------------------------------- generic --

int probe_tns_nmodes(const char* path) { return cptc_tns_probe_nmodes(path); }

bool load_tns_generic(const char* path, GTensor& t, double* load_ms_out)
{
    const auto t0 = std::chrono::steady_clock::now();
    cptc_coo c{};
    if (cptc_tns_load_generic(path, &c) != CPTC_OK)
    {
        std::cerr << "[GEN] cannot load " << path << ": " << cptc_last_error() << std::endl;
        return false;
    }
    t = GTensor{};
    t.nmodes = c.nmodes;
    t.nnz = c.nnz;
    t.dims.assign(c.dims, c.dims + c.nmodes);
    t.h_vals.assign(c.val, c.val + c.nnz);
    t.h_coords.resize(size_t(c.nmodes));
    for (int m = 0; m < c.nmodes; ++m)
        t.h_coords[size_t(m)].assign(c.idx + size_t(m) * c.nnz, c.idx + size_t(m + 1) * c.nnz);
    cptc_coo_free(&c);
    if (load_ms_out)
        *load_ms_out =
            std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0)
                .count();
    return true;
}

int run_dense_selftest()
{
    int failures = 0;
    if (cptc_gen_selftest(1, &failures) != CPTC_OK)
    {
        std::cerr << "[SELFTEST] " << cptc_last_error() << std::endl;
        return 1;
    }
    return failures ? 1 : 0;
}

int run_generic_cp(GTensor& t, int max_iters, int R, unsigned int seed)
{
    if (t.nmodes < 2 || t.nmodes > CPTC_MAX_MODES || t.nnz == 0 || R <= 0 || R > 32)
    {
        std::cerr << "[GEN] invalid run config (nmodes=" << t.nmodes << " nnz=" << t.nnz
                  << " R=" << R << ")" << std::endl;
        return -1;
    }
    if (max_iters <= 0) max_iters = 1;
    const int N = t.nmodes;
    std::vector<uint32_t> idx(size_t(N) * t.nnz);
    for (int m = 0; m < N; ++m)
        std::copy(t.h_coords[size_t(m)].begin(), t.h_coords[size_t(m)].end(),
                  idx.begin() + size_t(m) * t.nnz);
    cptc_coo c{};
    c.nmodes = N;
    for (int m = 0; m < N; ++m) c.dims[m] = t.dims[size_t(m)];
    c.nnz = t.nnz;
    c.idx = idx.data();
    c.val = t.h_vals.data();
    cptc_gen_opts o;
    cptc_gen_default_opts(&o);
    o.R = R;
    o.seed = seed;
    o.verbose = 1;
    void* h = nullptr;
    if (cptc_gen_create(&c, &o, &h) != CPTC_OK)
    {
        std::cerr << cptc_last_error() << std::endl;
        return -1;
    }
    // the reference reorders the caller's tensor in place
    std::vector<uint32_t> rank;
    for (int m = 0; m < N; ++m)
    {
        rank.resize(t.dims[size_t(m)]);
        cptc_gen_rank(h, m, rank.data());
        for (uint32_t& x : t.h_coords[size_t(m)]) x = rank[x];
    }
    const auto t0 = std::chrono::steady_clock::now();
    int rc = cptc_gen_run(h, max_iters, nullptr, nullptr, nullptr, nullptr);
    if (rc == CPTC_OK)
        if (const char* base = std::getenv("GEN_DUMP"))
        {
            const char* orig = std::getenv("GEN_DUMP_ORIGINAL");
            const int input_order = (orig && std::atoi(orig) != 0) ? 1 : 0;
            if (cptc_gen_dump_ex(h, base, input_order) == CPTC_OK)
                std::cout << "[GEN] factors dumped to " << base << ".factors.txt" << std::endl;
            else
                std::cerr << "[GEN] factor dump failed: " << cptc_last_error() << std::endl;
        }
    if (rc == CPTC_OK)
    {
        std::cout << "[GEN] ALS total = "
                  << std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() -
                                                               t0)
                         .count()
                  << " ms" << std::endl;
        if (o.profile)
        {
            double p[5];
            int it = 0;
            cptc_gen_profile(h, p, &it, 0);
            const double n = it > 0 ? double(it) : 1.0;
            const double tot = p[0] + p[1] + p[2] + p[3] + p[4];
            std::cout << "[GEN][profile] avg/iter over " << it << " iters: gram=" << p[0] / n
                      << " mttkrp=" << p[1] / n << " solve=" << p[2] / n << " norm=" << p[3] / n
                      << " fit=" << p[4] / n << " (sum=" << tot / n << " ms)" << std::endl;
            if (tot > 0.0)
                std::cout << "[GEN][profile] share: gram=" << 100.0 * p[0] / tot
                          << "% mttkrp=" << 100.0 * p[1] / tot << "% solve=" << 100.0 * p[2] / tot
                          << "% norm=" << 100.0 * p[3] / tot << "% fit=" << 100.0 * p[4] / tot
                          << "%" << std::endl;
        }
        double res2 = 0.0, x2 = 0.0;
        rc = cptc_gen_residual(h, &res2, &x2);
        if (rc == CPTC_OK)
        {
            const double res = std::sqrt(std::max(res2, 0.0)), xn = std::sqrt(x2);
            std::cout << "[GEN] exact: ||X-Xhat||_F=" << res
                      << " RMSE=" << res / std::sqrt(double(t.nnz))
                      << " fit=" << (xn > 0.0 ? 1.0 - res / xn : 0.0) << " (||X||_F=" << xn
                      << ")" << std::endl;
            std::vector<double> lam(size_t(R), 0.0);
            cptc_gen_lambda(h, lam.data());
            std::cout << "[GEN] lambda = ";
            for (int r = 0; r < R; ++r) std::cout << (r ? " " : "") << lam[size_t(r)];
            std::cout << std::endl;
        }
    }
    if (rc != CPTC_OK) std::cerr << "[GEN] " << cptc_last_error() << std::endl;
    cptc_gen_destroy(h);
    return rc == CPTC_OK ? 0 : -1;
}
