// FP64 sparse MTTKRP over the row-sorted views (sparse.hpp:1-114,
// sparse.cu:614-900).  d_FtV is accumulated into (the caller zeroes it);
// d_FtF is unused, as in the reference.
#ifndef SPARSE_HPP
#define SPARSE_HPP

#include <hip/hip_runtime_api.h>

#include <cstddef>

#ifndef MTTKRP_BLOCK
#define MTTKRP_BLOCK 128
#endif
#ifndef MTTKRP_ITEMS
#define MTTKRP_ITEMS 8
#endif
#ifndef MTTKRP_CHUNK
#define MTTKRP_CHUNK (MTTKRP_BLOCK * MTTKRP_ITEMS)   // row-segment length, 1024
#endif

struct HybridCOOTensor;

// Range form (sparse.cu:856-965).  With views built, a range covering the
// whole residual runs the row-sorted segment kernel; a strict sub-range runs
// cptc_mttkrp_sparse3_range over those elements of the target mode's view
// (one atomic per element and rank, as mttkrp_range_generic_kernel).  The
// range is clamped to the residual; nothing runs before build_mttkrp_views.
void compute_sparse_mttkrp_async(const HybridCOOTensor& hybrid, int target_mode,
                                 const double* d_A, const double* d_B, const double* d_C,
                                 double* d_FtV, double* d_FtF, int R, hipStream_t stream,
                                 size_t start_idx, size_t count);

// sparse.cu:821-854: the whole residual on `stream`; a no-op before
// build_mttkrp_views or when the residual is empty.
void compute_sparse_mttkrp_async(const HybridCOOTensor& hybrid, int target_mode,
                                 const double* d_A, const double* d_B, const double* d_C,
                                 double* d_FtV, double* d_FtF, int R, hipStream_t stream);

// Synchronous form (waits for the launch).
void compute_sparse_mttkrp(const HybridCOOTensor& hybrid, int target_mode, const double* d_A,
                           const double* d_B, const double* d_C, double* d_FtV, double* d_FtF,
                           int R);

#endif  // SPARSE_HPP
