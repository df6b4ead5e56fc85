// Dense 16^3 tile MTTKRP on the matrix cores with FP64 output accumulation
// (dense.hpp:1-37, dense.cu:1569-2246): the split-bf16 kernel
// (v_mfma_f32_32x32x16_bf16 over hi/lo bf16 halves, FP32 weights) for
// R > 16 with enough tiles, the FP32 MFMA kernel otherwise (ALS_TILE_KERNEL
// = fp32 | bf16x3 forces one).  d_FtV is accumulated into; d_FtF is unused.
#pragma once

#include <hip/hip_runtime_api.h>

#include "common.hpp"
#include "tensor.hpp"

// dense.cu:2072-2246: every dense tile of `hybrid` for `mode` on `stream`.
// The FP32 tile images (and, for the split-bf16 kernel the drivers' rule
// picks — R > 16 and enough tiles, ALS_TILE_KERNEL to force — the mode's
// compacted split image) are built from the pools on first use: the first
// call per mode of the split-bf16 kernel waits on `stream` twice while it
// sizes and fills that image (later calls do not wait).  The kernel's
// operand workspace is allocated and freed stream-ordered on every call
// (hipMallocAsync / hipFreeAsync), as the reference allocates its tile
// metadata per call (dense.cu:2117-2150), so calls on different streams
// never share it; such calls cannot be captured into a HIP graph.
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
