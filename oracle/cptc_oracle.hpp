// CPU oracle for the CP-ALS hot path — TEST INFRASTRUCTURE ONLY.
//
// A plain C++17 restatement of the reference's algorithms, used by tests/,
// __graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker and
// the CPU baseline.  Nothing in the product (cptc_amd/, include/) links,
// loads or calls this code.  Every function cites the reference file:line it
// follows (paths relative to the reference repository root).
//
// Pinning (see tests/test_oracle_*.py):
//   load_tns3            hand-written .tns fixtures with known answers
//   cadr3                invariants + tie-free closed form (numpy argsort);
//                        tie order = libstdc++ std::sort, same call as the
//                        reference (identical by construction)
//   partition3 / views3  independent numpy restatement (stable lexsort) on
//                        random inputs; invariants
//   mttkrp3_*            closed form Y = X_(n) (khatri-rao) via numpy einsum
//                        on dense tensors; brute force
//   pinv_sym             numpy.linalg.pinv / inverse; A pinv A = A
//   als3                 Gram fit == exact fit (independent formula);
//                        fixed-point checks on exact low-rank tensors
// Functions without such a check: none (the header of each test says which).
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace oracle {

struct Coo3
{
    size_t dims[3] = {0, 0, 0};
    std::vector<int32_t> m0, m1, m2;
    std::vector<double> val;
    size_t nnz() const { return val.size(); }
};

// tensor.cu:24-271
bool load_tns3(const std::string& path, Coo3& out);

// cadr.cu:23-66 (perm[old] = new), cadr.cu:69-81 (relabel)
void cadr3(const Coo3& t, std::vector<int32_t> perm[3]);
void apply_cadr3(Coo3& t, const std::vector<int32_t> perm[3]);

// common.cu:66-123 — mt19937(seed), uniform_real_distribution<double>(0,1),
// mode 0 then 1 then 2, row-major [i*R + r]
void init_factors3(const size_t dims[3], int R, unsigned seed, std::vector<double> F[3]);

struct Tile
{
    int32_t b[3];
    int32_t nnz;
    size_t off;
};

struct Partition3
{
    int cutoff = 0;
    size_t nblk[3] = {0, 0, 0};
    std::vector<Tile> tiles;            // ascending block_id
    std::vector<int32_t> pool_lid;      // (li*16+lj)*16+lk, run (input) order
    std::vector<double> pool_val;
    std::vector<uint32_t> sp_i, sp_j, sp_k;  // residual, block-sorted (stable)
    std::vector<double> sp_val;
};

// CU count used by the auto-balance cutoff (partition.cu:1040-1060 scales its
// per-element rates by the device's SM count); default 256 (MI355X).
void set_num_cus(int n);

// partition.cu:581-1493 (threshold > 0: cutoff = clamp((int)(4096*thr), 1, 4096);
// threshold <= 0: auto-balance, partition.cu:1030-1098)
void partition3(const Coo3& t, double threshold, Partition3& p);

struct View3
{
    size_t nnz = 0;
    std::vector<uint64_t> coords[3];
    std::vector<double> vals[3];
    std::vector<uint32_t> blk_row[3], blk_start[3], blk_cnt[3];
};

// partition.cu:1691-1810, 1865-2329 (stable sort on (target, o1, o0),
// 1024-element row segments).  Throws if a dim >= 32768.
void views3(const std::vector<uint32_t>& i, const std::vector<uint32_t>& j,
            const std::vector<uint32_t>& k, const std::vector<double>& v, const size_t dims[3],
            View3& out);

// partition.cu:2335-2379 + 2387-2517: decode the dense pool (tile order, pool
// order) into coordinates and build views of them.
void dense_views3(const Partition3& p, const size_t dims[3], View3& out);

// sparse.cu:614-711 (and 271-333): per segment acc_r = sum_e (v*F1[o0,r])*F2[o1,r],
// FtV[row] += acc.  FtV (dim x R) is accumulated into (caller zeroes it).
// Rows are processed in parallel (OpenMP), each row's segments in order: the
// result is independent of the thread count.
void mttkrp3_view(const View3& v, int mode, const double* A, const double* B, const double* C,
                  int R, double* FtV);

// dense.cu:89-1077 in exact FP64: tile cells hold the last pool entry per lid
// (clamped to +-FLT_MAX); mode 0: FtV[i,r] += sum_{j,k} T[i,j,k] B[j,r] C[k,r], etc.
void mttkrp3_tiles(const Partition3& p, int mode, const double* A, const double* B,
                   const double* C, int R, const size_t dims[3], double* FtV);

// G = F^T F (row-major F rows x R).  als.cu:115-134.
void gram(const double* F, size_t rows, int R, double* G);

// solver.cu:900-1002: pinv via the symmetric eigen-decomposition (cyclic
// Jacobi), dropping |lambda_i| <= R * ulp(max |lambda|).  Returns sweeps used.
int pinv_sym(const double* A, int R, double* Ainv);

// Order-3 CP-ALS (als.cu:362-821) over pre-built views.
struct Als3State
{
    int R = 0;
    size_t dims[3] = {0, 0, 0};
    std::vector<double> F[3];
    std::vector<double> lambda;
};

struct Als3Input
{
    const View3* residual = nullptr;   // h1 views (may hold 0 nnz)
    const View3* dense_view = nullptr; // h2 views (FP64 dense path) or null
    const Partition3* tiles = nullptr; // dense tiles (MFMA path) or null
    double x_sq = 0.0;                 // ||X||^2 as als.cu:439-450 computes it
};

// Runs `iters` iterations; fits[it] = Gram fit; ms[it] = wall ms of the
// iteration; mttkrp_ms[it] = wall ms of the three MTTKRPs.
void als3_iterate(const Als3Input& in, Als3State& st, int iters, double* fits, double* ms,
                  double* mttkrp_ms);

// ||X||^2 and exact residual (common.cu:517-650) over views + tiles.
void residual3(const Als3Input& in, const Als3State& st, bool with_lambda, double* res_sq,
               double* x_sq);

// CP-SGD (sgd.cu:51-467).  sgd3_sample: cpsgd_sample_kernel's hash.
// sgd3_step: the batch's elements applied one after another in batch order
// (the reference runs them concurrently with atomics; both agree when no two
// elements of the batch share a factor row).  sgd3_normalize: F[:, r] /= n_r,
// lambda_r = n_r (both 0 below 1e-14).  sgd3_loss: sum of (v - xhat)^2.
std::vector<uint32_t> sgd3_sample(uint64_t seed, uint32_t batch, uint64_t nnz);
void sgd3_step(const std::vector<uint64_t>& coords, const std::vector<double>& vals,
               const std::vector<uint32_t>& idx, double* A, double* B, double* C,
               const double* lambda, int R, double gamma);
void sgd3_normalize(double* F, size_t rows, int R, double* lambda);
double sgd3_loss(const std::vector<uint64_t>& coords, const std::vector<double>& vals,
                 const std::vector<uint32_t>& idx, const double* A, const double* B,
                 const double* C, const double* lambda, int R);

}  // namespace oracle
