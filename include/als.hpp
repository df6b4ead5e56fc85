// The order-3 CP-ALS iteration (als.hpp, als.cu:362-821).
#ifndef ALS_HPP
#define ALS_HPP

#include "partition.hpp"
#include "tensor.hpp"

// Runs max_iters ALS iterations on the caller's layout and factors: mode
// order A, B, C; per mode FtF = Hadamard of the other Grams, MTTKRP (MFMA
// dense tiles of `hybrid` when it has tiles and `hybrid_dense` has no views,
// FP64 dense views of `hybrid_dense` when it has them, FP64 residual views of
// `hybrid`), F = FtV pinv(FtF) / lambda, column normalisation into lambda;
// the Gram fit is printed per iteration ("[ALS] iter k/n time=X ms fit=Y").
// d_A, d_B, d_C are updated in place; d_lambda_out (R) receives the
// weights.  lambda_reg is unused (the pseudoinverse needs no ridge).
void execute_als_decomposition(const COOTensor& tensor, HybridCOOTensor& hybrid,
                               const HybridCOOTensor& hybrid_dense, double* d_A, double* d_B,
                               double* d_C, double* d_lambda_out, int R, int max_iters,
                               double lambda_reg);

#endif  // ALS_HPP
