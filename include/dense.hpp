// Dense 16^3 tile MTTKRP on FP32 MFMA with an FP64 epilogue (dense.hpp:1-37,
// dense.cu:1569-2246).  d_FtV is accumulated into; d_FtF is unused.
#pragma once

#include <hip/hip_runtime_api.h>

#include "common.hpp"
#include "tensor.hpp"

// dense.cu:2072-2246: every dense tile of `hybrid` for `mode` on `stream`.
// The FP32 tile images (and, for the split-bf16 kernel the drivers' rule
// picks — R > 16 and enough tiles, ALS_TILE_KERNEL to force — the compacted
// image) are built from the pools on first use.
void compute_dense_mttkrp_async(const HybridCOOTensor& hybrid, int mode, double* d_A,
                                double* d_B, double* d_C, double* d_FtV, double* d_FtF, int R,
                                hipStream_t stream);

void compute_dense_mttkrp(const HybridCOOTensor& hybrid, int mode, double* d_A, double* d_B,
                          double* d_C, double* d_FtV, double* d_FtF, int R);

// dense.cu:1914-2058, 2258-2511 (the reference's single-grid R == 32
// kernel): one launch of cptc_mttkrp_merged3 over the dense tiles and the
// residual segments for even R <= 128 with 16-byte aligned factors; other
// shapes queue the two launches back to back on `stream`.
void compute_mttkrp_merged_async(const HybridCOOTensor& hybrid, int mode, double* d_A,
                                 double* d_B, double* d_C, double* d_FtV, double* d_FtF, int R,
                                 hipStream_t stream);
