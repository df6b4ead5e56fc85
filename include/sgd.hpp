// CP-SGD on the order-3 sparse residual (sgd.hpp, sgd.cu:302-467).
#ifndef SGD_HPP
#define SGD_HPP

#include "tensor.hpp"

// max_iters iterations of the reference's loop on hybrid's mode-0 residual
// view: a batch of batch_size elements sampled with seed + it, one
// asynchronous SGD step per element (learning rate gamma), every fifth
// iteration the factors normalised with lambda = column norms, the batch
// RMSE printed every tenth and at the last.  d_A, d_B, d_C and
// d_lambda_out (the caller initialises lambda, main.cu:466-471: 1) are
// updated in place.  Fatal on error, like the reference.
void execute_sgd_decomposition(const HybridCOOTensor& hybrid, double* d_A, double* d_B,
                               double* d_C, double* d_lambda_out, int R, int max_iters,
                               double gamma, int batch_size, unsigned long long seed);

#endif  // SGD_HPP
