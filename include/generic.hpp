// The generic N-order path (generic.hpp:1-45, generic.cu).
#ifndef GENERIC_HPP
#define GENERIC_HPP

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

struct GTensor {
    int nmodes = 0;
    std::vector<size_t> dims;
    size_t nnz = 0;
    std::vector<double> h_vals;
    std::vector<std::vector<uint32_t>> h_coords;   // h_coords[m][e], 0-based
};

// generic.cu:983-1021: index columns of the first numeric line, -1 on error.
int probe_tns_nmodes(const char* path);

// generic.cu:1023-1155: any-order .tns (1-based -> 0-based); false on error.
bool load_tns_generic(const char* path, GTensor& t, double* load_ms_out);

// generic.cu:1389-1637: the dense-unit known-answer test; 0 = passed.
int run_dense_selftest();

// generic.cu:1639-2366: reorders t in place (GEN_REORDER, default hits for
// N >= 4, cadr otherwise), then CP-ALS with the GEN_* switches, printing the
// reference's [GEN] lines.  0 on success, -1 on an invalid configuration
// (R outside 1..32, nnz outside 1..0x7FFFFFFF) or a device error.
int run_generic_cp(GTensor& t, int max_iters, int R, unsigned int seed);

#endif  // GENERIC_HPP
