// Device-resident layout of an order-3 tensor: the hybrid 16^3 partition and
// the per-mode row-sorted views.  HIP-native counterpart of the reference's
// HybridCOOTensor (tensor.hpp:71-339); buffers are owned by the struct and
// released with free_*().
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <vector>

namespace cptc {

constexpr int TILE = 16;  // TILE_DIM (partition.hpp:10-12)

struct DevCoo3
{
    uint64_t dims[3] = {0, 0, 0};
    size_t nnz = 0;
    int32_t* d_m[3] = {nullptr, nullptr, nullptr};
    double* d_val = nullptr;
};

struct DevPartition3
{
    int cutoff = 0;
    uint64_t nblk[3] = {0, 0, 0};
    int64_t ntiles = 0;
    int32_t* d_tiles4 = nullptr;      // ntiles x {bi, bj, bk, nnz}
    uint64_t* d_pool_off = nullptr;   // ntiles + 1
    size_t dense_nnz = 0;
    int32_t* d_pool_lid = nullptr;    // (li*16 + lj)*16 + lk
    double* d_pool_val = nullptr;
    size_t sparse_nnz = 0;
    uint32_t* d_sp[3] = {nullptr, nullptr, nullptr};
    double* d_sp_val = nullptr;
    std::vector<int32_t> h_tiles4;
    std::vector<uint64_t> h_pool_off;
};

struct DevViews3
{
    size_t nnz = 0;
    bool ready = false;
    uint64_t* d_coords[3] = {nullptr, nullptr, nullptr};
    double* d_vals[3] = {nullptr, nullptr, nullptr};
    size_t nseg[3] = {0, 0, 0};
    uint32_t* d_blk_row[3] = {nullptr, nullptr, nullptr};
    uint32_t* d_blk_start[3] = {nullptr, nullptr, nullptr};
    uint32_t* d_blk_cnt[3] = {nullptr, nullptr, nullptr};
};

// Blocked residual views for mttkrp3_blk_kernel (R in (64, 128]): per mode
// the reference view re-sorted by (target >> lg_tb, o1 >> lg_kb), stable, so
// each block pair keeps (target, o1, o0) order; spans = one staged block pair
// or consecutive unstaged ones (span_kb = o1 block | 1 << 31 when staged);
// chunks = consecutive spans of one target row block (one workgroup each).
struct DevBlk3
{
    bool ready = false;
    size_t nnz = 0;
    int lg_tb = 5, lg_kb = 4;
    uint64_t* d_coords[3] = {nullptr, nullptr, nullptr};
    double* d_vals[3] = {nullptr, nullptr, nullptr};
    size_t nspan[3] = {0, 0, 0}, nchunk[3] = {0, 0, 0};
    uint32_t* d_span_start[3] = {nullptr, nullptr, nullptr};
    uint32_t* d_span_cnt[3] = {nullptr, nullptr, nullptr};
    uint32_t* d_span_kb[3] = {nullptr, nullptr, nullptr};
    uint32_t* d_chunk_span0[3] = {nullptr, nullptr, nullptr};
    uint32_t* d_chunk_nspan[3] = {nullptr, nullptr, nullptr};
    uint32_t* d_chunk_tb[3] = {nullptr, nullptr, nullptr};
};

void free_coo(DevCoo3& c);
void free_partition(DevPartition3& p);
void free_views(DevViews3& v);
void free_blk(DevBlk3& b);

// COO host arrays (uint32 mode-major, as cptc_coo) -> device int32 + values.
int upload_coo3(const uint32_t* idx, const double* val, size_t nnz, const uint64_t dims[3],
                DevCoo3& out, hipStream_t s);

// CADR: degrees on the device, relabel order by the reference's std::sort on
// the host, relabel on the device.  perm[m][old] = new.
int cadr3_device(DevCoo3& c, std::vector<int32_t> perm[3], int32_t* d_perm[3], int relabel,
                 hipStream_t s);

// Hybrid partition (partition.cu:581-1493).  num_cus scales the auto-balance
// rates as the reference scales them by its SM count.
int partition3_device(const DevCoo3& c, double threshold, int num_cus, DevPartition3& out,
                      hipStream_t s);

// Row-sorted views (partition.cu:1865-2329) of coordinates i, j, k + values.
int views3_device(const uint32_t* d_i, const uint32_t* d_j, const uint32_t* d_k,
                  const double* d_val, size_t nnz, const uint64_t dims[3], DevViews3& out,
                  hipStream_t s);

// Blocked views of the residual views v (see DevBlk3); chunk = elements per
// workgroup, stage_min = elements of a block pair from which its run-level
// rows are staged in LDS.
int blk_views3_device(const DevViews3& v, const uint64_t dims[3], int lg_tb, int lg_kb,
                      uint32_t chunk, uint32_t stage_min, DevBlk3& out, hipStream_t s);

// Dense-pool decode + views (partition.cu:2335-2517).
int dense_views3_device(const DevPartition3& p, const uint64_t dims[3], DevViews3& out,
                        hipStream_t s);

// The order-3 ALS iteration on a borrowed layout and caller-owned factors
// (execute_als_decomposition, als.cu:362-821); writes lambda_out (device, R)
// and the last Gram fit.  tile_f32 = packed FP32 tiles (MFMA path) or null.
int als3_execute(const uint64_t dims[3], const DevPartition3& part, const DevViews3& views,
                 const DevViews3& dviews, float* tile_f32, bool use_mfma, double* A, double* B,
                 double* C, double* lambda_out, int R, int iters, bool verbose, double* fit_last);

}  // namespace cptc
