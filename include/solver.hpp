// The ALS least-squares solve F = FtV * pinv(FtF) (solver.hpp:9-60,
// solver.cu:815-1096).  The pseudoinverse uses the reference's truncation
// rule (singular values <= R * ulp(sigma_max) dropped); on the device it is
// a Cholesky inverse with an exact cyclic-Jacobi fallback instead of
// cuSOLVER gesvdj, and no BLAS handle is needed (the `blas` argument is
// accepted for signature compatibility and ignored).
#ifndef SOLVER_HPP
#define SOLVER_HPP

#include <cstddef>

// The fused solve keeps its work arrays in library-owned device scratch; the
// workspace records the rank it was initialised for.
struct SVDWorkspace {
    int R = 0;
};

void init_svd_workspace(SVDWorkspace& ws, int R);
void free_svd_workspace(SVDWorkspace& ws);

// solver.cu:900-1002: d_Factor (dim_len x R) = d_FtV * pinv(d_FtF); waits for
// the result.  Returns false on invalid arguments or a device error.
bool solve_als_system_svd(const SVDWorkspace& ws, void* blas, double* d_FtF, double* d_FtV,
                          double* d_Factor, size_t dim_len, int R);

// solver.cu:1008-1096: the same, queued on the null stream without waiting.
bool solve_als_system_svd_nosync(const SVDWorkspace& ws, void* blas, double* d_FtF,
                                 double* d_FtV, double* d_Factor, size_t dim_len, int R);

#endif  // SOLVER_HPP
