// C++ interface of the MI355X engine, after the reference's tensor.hpp
// (tensor.hpp:22-355): the order-3 COO tensor, dense 16^3 tiles and the
// hybrid (dense tiles + row-sorted sparse views) layout.
//
// Same names, fields and ownership rules as the reference; device pointers
// are HIP allocations.  Fields below "MI355X layout" have no counterpart in
// the reference: they carry the tile headers and pool offsets that the MFMA
// kernels index, and the FP32 tile images they read.
#ifndef TENSOR_HPP
#define TENSOR_HPP

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

// tensor.hpp:22-51.  Host arrays h_*, device copies d_* (0-based).
struct COOTensor {
    size_t dims[3] = {0, 0, 0};
    size_t nnz = 0;
    int* d_m0 = nullptr;
    int* d_m1 = nullptr;
    int* d_m2 = nullptr;
    double* d_val = nullptr;
    std::vector<int> h_m0;
    std::vector<int> h_m1;
    std::vector<int> h_m2;
    std::vector<double> h_val;
};

// tensor.hpp:71-80: one dense 16^3 tile; d_coords / d_values point into the
// hybrid tensor's pools (local id (li*16 + lj)*16 + lk, fp64 value).
struct DenseTile16 {
    int block_idx[3] = {0, 0, 0};
    int nnz = 0;
    int* d_coords = nullptr;
    double* d_values = nullptr;
};
using DenseTile = DenseTile16;

// tensor.hpp:142-339
struct HybridCOOTensor {
    size_t dims[3] = {0, 0, 0};
    int num_dense_tiles = 0;
    size_t sparse_nnz = 0;

    // residual COO after partitioning (released by build_mttkrp_views)
    uint32_t* d_sp_i = nullptr;
    uint32_t* d_sp_j = nullptr;
    uint32_t* d_sp_k = nullptr;
    double* d_sp_val = nullptr;

    // per-mode row-sorted views: packed (i << 30) | (j << 15) | k, values,
    // <= 1024-element row segments
    uint64_t* d_sp2_coords[3] = {nullptr, nullptr, nullptr};
    double* d_sp2_val[3] = {nullptr, nullptr, nullptr};
    uint32_t* d_blk_row[3] = {nullptr, nullptr, nullptr};
    uint32_t* d_blk_start[3] = {nullptr, nullptr, nullptr};
    uint32_t* d_blk_cnt[3] = {nullptr, nullptr, nullptr};
    size_t mttkrp_blocks[3] = {0, 0, 0};
    bool mttkrp_ready = false;

    size_t num_blocks[3] = {0, 0, 0};
    std::vector<DenseTile16> dense_tiles;
    int* d_dense_coords_pool = nullptr;
    double* d_dense_values_pool = nullptr;
    int* d_dense_k_offsets = nullptr;   // unused here (always null)
    size_t dense_coords_capacity = 0;
    size_t dense_values_capacity = 0;

    // MI355X layout
    int32_t* d_tiles4 = nullptr;        // num_dense_tiles x {bi, bj, bk, nnz}
    uint64_t* d_pool_off = nullptr;     // num_dense_tiles + 1 pool offsets
    mutable float* d_tile_f32 = nullptr;  // FP32 tile images, packed on first MFMA use
    // compacted split tile images of the split-bf16 kernel, one per target
    // mode, each built on the mode's first use
    mutable uint32_t* d_tile_cmask[3] = {nullptr, nullptr, nullptr};
    mutable uint32_t* d_tile_segoff[3] = {nullptr, nullptr, nullptr};
    mutable void* d_tile_cseg[3] = {nullptr, nullptr, nullptr};
    mutable uint64_t tile_nseg[3] = {0, 0, 0};
    size_t dense_nnz = 0;
    int dense_cutoff = 0;
};

// tensor.cu:24-271: parse an order-3 .tns file (the reference's rules) into
// host arrays and upload them.  Exits the process on failure.
void load_tns_file(const std::string& filename, COOTensor& tensor);

// tensor.cu: release the device arrays and clear the host ones.
void free_coo_tensor(COOTensor& tensor);

#endif  // TENSOR_HPP
