// CADR degree-descending mode relabelling (cadr.hpp:8-33, cadr.cu:9-112).
#ifndef CADR_HPP
#define CADR_HPP

#include <vector>

#include "tensor.hpp"

// perm*[old_idx] = new_idx, host and device copies.
struct TensorPermutation {
    std::vector<int> perm0;
    std::vector<int> perm1;
    std::vector<int> perm2;
    int* d_perm0 = nullptr;
    int* d_perm1 = nullptr;
    int* d_perm2 = nullptr;
};

// cadr.cu:23-61: degrees of every index; new order = std::sort(iota,
// deg[a] > deg[b]) (libstdc++, no tie-break), as the reference.
TensorPermutation compute_cadr_reordering(const COOTensor& tensor);

// cadr.cu:63-81: relabel the host coordinates and re-upload them.
void apply_cadr_reordering(COOTensor& tensor, const TensorPermutation& perm);

// cadr.cu:84-103: orig[old, :] = F[perm[old], :] for the three modes
// (d_factors_orig[0..2] are caller allocations of dims[m] x R).
void unpermute_factor_matrices(double* d_A_perm, double* d_B_perm, double* d_C_perm,
                               double** d_factors_orig, const TensorPermutation& perm,
                               const size_t* dims, int R);

void free_cadr_permutation(TensorPermutation& perm);

#endif  // CADR_HPP
