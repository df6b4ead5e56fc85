// Exact fit of the final model (compute_fit.hpp, compute_fit.cu:20-175).
#ifndef COMPUTE_FIT_HPP
#define COMPUTE_FIT_HPP

#include "common.hpp"
#include "tensor.hpp"

// fit = 1 - ||X - Xhat|| / ||X|| over every stored element (d_lambda null:
// unit weights).
double compute_fit(const HybridCOOTensor& h1, const HybridCOOTensor& h2, const double* d_A,
                   const double* d_B, const double* d_C, const double* d_lambda, int R);

// Prints "[Fit] ..." and "[Fit Report] ..." lines as the reference.
void print_fit_report(const HybridCOOTensor& h1, const HybridCOOTensor& h2, const double* d_A,
                      const double* d_B, const double* d_C, const double* d_lambda, int R,
                      double rmse, const char* tag = "");

#endif  // COMPUTE_FIT_HPP
