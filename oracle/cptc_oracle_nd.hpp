// CPU oracle for the generic N-order CP-ALS path — TEST INFRASTRUCTURE ONLY.
//
// A plain C++17 restatement of the reference's generic.cu, used by tests/,
// __graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker.
// Nothing in the product links, loads or calls this code.
//
// Pinning (tests/test_oracle_nd.py): reorder_nd against an independent numpy
// restatement (HITS with np.add.at in element order, CADR by lexsort);
// dense_nd against a numpy restatement of the hashed unit selection;
// views_nd against a stable argsort; mttkrp_nd (segment and unit parts)
// against numpy einsum on dense 4/5-order tensors; chol_solve_nd against
// numpy's Cholesky with the same ridge; als_nd against an independent numpy
// ALS; the GEN_SELFTEST construction against its own exact MTTKRP.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace oracle {

struct CooN
{
    int N = 0;
    std::vector<size_t> dims;
    std::vector<std::vector<uint32_t>> c;  // c[m][e], 0-based
    std::vector<double> val;
    size_t nnz() const { return val.size(); }
};

// generic.cu:1176-1376.  how = "hits" | "cadr" | "none" | "auto"; rank[m][old]
// = new (empty when no permutation was applied).  Coordinates are relabelled
// in place.  `sample_budget` = GEN_REORDER_SAMPLE (default 8e6).
void reorder_nd(CooN& t, const std::string& how, int rounds, size_t sample_budget,
                std::vector<std::vector<uint32_t>>& rank);

// generic.cu:39-45
uint64_t splitbit_hash(uint64_t x);

struct UnitsN
{
    int cutoff = 0;
    int inner[3] = {0, 1, 2};             // modes of tile slots a, b, c
    std::vector<int> outer;               // outer modes, ascending
    // per unit: bi, bj, bk, nnz, start, outer_off
    std::vector<uint32_t> unit6;
    std::vector<uint32_t> outer_coords;   // (N-3) per unit
    std::vector<uint32_t> lid;            // a*256 + b*16 + c, element order per unit
    std::vector<double> val;
    std::vector<uint8_t> is_dense;        // per element (input order)
    size_t n_units() const { return unit6.size() / 6; }
};

// generic.cu:564-725; `inner` = the three tile-slot modes (default 0, 1, 2)
void dense_nd(const CooN& t, double threshold, const int inner[3], UnitsN& u);

struct ViewN
{
    // per mode n: (N-1) x nnz coords (other modes ascending), vals, skip (view
    // order), segments (row, start, cnt, single)
    std::vector<std::vector<uint32_t>> sc;
    std::vector<std::vector<double>> sv;
    std::vector<std::vector<uint8_t>> skip;
    std::vector<std::vector<uint32_t>> row, start, cnt;
    std::vector<std::vector<uint8_t>> single;
};

// generic.cu:1848-1958.  Modes whose bit is set in `force_accumulate` (the
// inner modes when the dense path is on) get single = 0.
void views_nd(const CooN& t, const std::vector<uint8_t>& is_dense, unsigned force_accumulate,
              ViewN& v);

// generic.cu:271-343: segment MTTKRP (skip honoured when `use_skip`), FP64;
// FtV (dim_n x R) accumulated (single segments store, others add).
void mttkrp_seg_nd(const CooN& t, const ViewN& v, int n, bool use_skip,
                   const std::vector<std::vector<double>>& F, int R, double* FtV);

// generic.cu:429-561 in exact FP64 (duplicates inside a unit summed):
// contribution of the dense units to the MTTKRP of inner mode n (n must be
// one of u.inner; the factors are indexed by mode, not by slot).
void mttkrp_units_nd(const CooN& t, const UnitsN& u, int n,
                     const std::vector<std::vector<double>>& F, int R, double* FtV);

// generic.cu:746-819: (FtF + eps I) x = FtV per row.
void chol_solve_nd(const double* FtF, const double* FtV, double* F, size_t dim, int R);

struct AlsNOpts
{
    int R = 16;
    unsigned seed = 42;
    bool svd = false;            // GEN_SOLVER=svd
    bool dense = true;           // GEN_DENSE
    double threshold = 0.03;     // GEN_DENSE_THRESHOLD
    int inner[3] = {0, 1, 2};    // GEN_DENSE_INNER
};

struct AlsNState
{
    std::vector<std::vector<double>> F;
    std::vector<double> lambda;
    std::vector<double> fits, iprod, model2;
    std::vector<double> ms;   // wall time of each iteration (CPU baseline)
};

// generic.cu:1639-2366 over a tensor that is already reordered; `rank` (old ->
// new, may be empty) permutes the initial factor rows.
void als_nd(const CooN& t, const std::vector<std::vector<uint32_t>>& rank, const AlsNOpts& o,
            int iters, AlsNState& st);

// generic.cu:936-967
double residual_nd(const CooN& t, const std::vector<std::vector<double>>& F,
                   const std::vector<double>& lambda, int R);

// generic.cu:1389-1462: the GEN_SELFTEST tensor (dims 40x24x36x3, R = 8,
// mt19937(1234)) and its factors.
void selftest_tensor(CooN& t, std::vector<std::vector<double>>& F);

}  // namespace oracle
