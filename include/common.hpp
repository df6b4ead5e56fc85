// Shared utilities (common.hpp:1-37, common.cu:1-716).
#ifndef COMMON_HPP
#define COMMON_HPP

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdlib>
#include <iostream>

#include "tensor.hpp"

// common.hpp:9-17, for HIP calls: print and exit on error.
#define CHECK_HIP(call)                                                                    \
    do                                                                                     \
    {                                                                                      \
        hipError_t err_ = (call);                                                          \
        if (err_ != hipSuccess)                                                            \
        {                                                                                  \
            std::cerr << "HIP error at " << __FILE__ << ":" << __LINE__ << " code=" << err_ \
                      << " \"" << hipGetErrorString(err_) << "\"" << std::endl;            \
            std::exit(EXIT_FAILURE);                                                       \
        }                                                                                  \
    } while (0)

// Prints the device's name, CU count, memory and clocks.
void debug_device_state();

// common.cu:66-123: d_factors[m] (dims[m] x R, row-major) filled with
// mt19937(42) U[0,1) draws, mode 0 then 1 then 2.
void init_factors_random(double** d_factors, const size_t* dims, int R);

// common.cu:160-190: clamp every element of d_factor to [min_val, max_val]
// (the name is the reference's; no Thrust is involved).
void clamp_factor_thrust(double* d_factor, size_t size, double min_val, double max_val);

// common.cu:517-650: sqrt(sum over all stored elements (v - xhat)^2 / nnz)
// over h1's views (and tiles when h2 has no views) and h2's views.
double calculate_rmse(const HybridCOOTensor& h1, const HybridCOOTensor& h2, double* d_A,
                      double* d_B, double* d_C, const double* d_lambda, int R);

// common.cu:251-505: h_res_sq = sum (v - xhat)^2, h_x_sq = sum v^2 over
// every stored element; has_lambda = false uses unit weights.
void compute_residual_and_norm_sq(const HybridCOOTensor& h1, const HybridCOOTensor& h2,
                                  const double* d_A, const double* d_B, const double* d_C,
                                  const double* d_lambda, bool has_lambda, int R,
                                  double& h_res_sq, double& h_x_sq);

#endif  // COMMON_HPP
