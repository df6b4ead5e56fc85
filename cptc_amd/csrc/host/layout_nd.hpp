// Device-resident layout of the generic N-order path: the dense units
// (GDense, generic.cu:564-725) and one row-segmented view per mode
// (ModeView, generic.cu:1848-1958).  Buffers are owned by the structs and
// released with free_*().
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace cptc {

struct DevUnitsN
{
    int cutoff = 0;
    int inner[3] = {0, 1, 2};
    std::vector<int> outer;              // outer modes, ascending
    uint64_t nunits = 0;
    uint64_t dense_nnz = 0;
    uint32_t* d_unit6 = nullptr;         // nunits x {bi, bj, bk, nnz, start, outer_off}
    uint32_t* d_outer_coords = nullptr;  // nunits x outer.size()
    uint32_t* d_lid = nullptr;           // dense_nnz, la*256 + lb*16 + lc
    double* d_val = nullptr;             // dense_nnz
    uint8_t* d_is_dense = nullptr;       // nnz, element order
};

struct DevViewN
{
    uint64_t nnz = 0;
    uint64_t nseg = 0;
    std::vector<int> level_modes;  // mode of each d_sc row (reference views: ascending)
    uint32_t* d_sc = nullptr;      // (N-1) x nnz
    double* d_vals = nullptr;
    uint8_t* d_skip = nullptr;     // view order; null when no dense units
    uint32_t* d_row = nullptr;
    uint32_t* d_start = nullptr;
    uint32_t* d_cnt = nullptr;
    uint8_t* d_single = nullptr;
    // kernel views: the level coordinates packed into one key per element
    // (level 0 in the top bits); key_bytes 0 when they need more than 64 bits
    void* d_key = nullptr;
    int key_bytes = 0;
    std::vector<int> level_bits;
};

// The reference's generic reordering (hits / cadr / auto / none,
// generic.cu:1176-1376) on the device: relabels d_coords (N x nnz,
// mode-major) in place and returns the per-mode ranks on the host (empty
// when nothing was applied) and the method applied in `used`.  Bit-exact
// with the reference's host code.
int reorder_nd_device(int N, const uint64_t* dims, uint32_t* d_coords, uint64_t nnz,
                      std::string how, int rounds, uint64_t budget,
                      std::vector<std::vector<uint32_t>>& rank, std::string& used, bool verbose,
                      hipStream_t s);

void free_units(DevUnitsN& u);
void free_view(DevViewN& v);

// Dense units of a device COO (coords N x nnz mode-major).  Units are the
// hash keys with count >= cutoff = int(4096 * threshold), numbered by first
// occurrence; pools hold each unit's elements in element order.
int units_nd_device(int N, const uint64_t* dims, const uint32_t* d_coords, const double* d_vals,
                    uint64_t nnz, double threshold, const int inner[3], DevUnitsN& out,
                    hipStream_t s);

// Mode n's view: elements stably sorted by coordinate n, rows cut into
// <= 1024-element segments; single = the row's only segment unless
// force_accumulate.  d_is_dense (element order) may be null.
int view_nd_device(int N, const uint64_t* dims, int n, const uint32_t* d_coords,
                   const double* d_vals, const uint8_t* d_is_dense, bool force_accumulate,
                   uint64_t nnz, DevViewN& out, hipStream_t s);

// The view the MTTKRP kernel runs on.  Dense elements (d_is_dense, may be
// null) are dropped; each row is sorted lexicographically over the other
// modes, smallest dimension first (level_modes), so equal coordinate
// prefixes form runs whose factor rows the kernel gathers once per run.
// Every segment accumulates when force_accumulate, else a row's only segment
// stores.
int work_view_nd_device(int N, const uint64_t* dims, int n, const uint32_t* d_coords,
                        const double* d_vals, const uint8_t* d_is_dense, bool force_accumulate,
                        uint64_t nnz, DevViewN& out, hipStream_t s);

}  // namespace cptc
