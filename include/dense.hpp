// Dense 16^3 tile MTTKRP on FP32 MFMA with an FP64 epilogue (dense.hpp:1-37,
// dense.cu:1569-2246).  d_FtV is accumulated into; d_FtF is unused.
#pragma once

#include <hip/hip_runtime_api.h>

#include "common.hpp"
#include "tensor.hpp"

// dense.cu:2072-2246: every dense tile of `hybrid` for `mode` on `stream`.
// The FP32 tile images are built from the pools on first use.
void compute_dense_mttkrp_async(const HybridCOOTensor& hybrid, int mode, double* d_A,
                                double* d_B, double* d_C, double* d_FtV, double* d_FtF, int R,
                                hipStream_t stream);

void compute_dense_mttkrp(const HybridCOOTensor& hybrid, int mode, double* d_A, double* d_B,
                          double* d_C, double* d_FtV, double* d_FtF, int R);

// dense.cu:1569-1621 (the reference's single-grid R == 32 kernel): here the
// dense tiles and the sparse views are queued back to back on `stream`,
// any R.
void compute_mttkrp_merged_async(const HybridCOOTensor& hybrid, int mode, double* d_A,
                                 double* d_B, double* d_C, double* d_FtV, double* d_FtF, int R,
                                 hipStream_t stream);
