// Internal entry points of kernels/small_la.hip for the order-3 driver.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>

namespace cptc {

// Work for the next mode that a mode's update hands to its last launch (the
// column scaling of the new factor), so that it needs no launch of its own:
// zero[0, nzero) is cleared (the next MTTKRP's output, read by this mode's
// apply before), and ftf = ga .* gb over R x R entries is formed (the next
// mode's FtF, cptc_hadamard's product bit for bit).  Null members: nothing.
struct TailJobs
{
    double* zero = nullptr;
    size_t nzero = 0;
    const double* ga = nullptr;
    const double* gb = nullptr;
    double* ftf = nullptr;
};

// cptc_gram_normalize_absorb with the tail jobs t (may be null)
int gram_normalize_absorb_tail(double* d_F, size_t rows, int R, double* d_G, double* d_norms,
                               double* d_lambda, const TailJobs* t, hipStream_t s);
// cptc_gram_normalize_absorb_next with the tail jobs t (may be null)
int gram_normalize_absorb_next_tail(double* d_F, size_t rows, int R, double* d_G,
                                    double* d_norms, double* d_lambda, const double* d_other,
                                    double* d_FtF, const TailJobs* t, hipStream_t s);

// cptc_update_small3: a small mode's whole update in one launch
// (rows <= UPDATE3_SMALL_MAX_ROWS, R <= 32)
constexpr size_t UPDATE3_SMALL_MAX_ROWS = 4096;
int update3_small(double* d_FtV, double* d_Ainv, double* d_F, size_t rows, int R, double* d_G,
                  double* d_norms, double* d_lambda, const double* d_other, double* d_FtF,
                  size_t nzero, const double* d_grams, double* d_fit, int next_pinv,
                  hipStream_t s);

}  // namespace cptc
