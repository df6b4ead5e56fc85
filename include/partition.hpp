// Hybrid partition of an order-3 tensor into dense 16^3 tiles and a sparse
// residual, and the row-sorted MTTKRP views (partition.hpp:1-404,
// partition.cu:581-2517).  The block / local-id helpers keep the
// reference's encodings.
#ifndef PARTITION_HPP
#define PARTITION_HPP

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>

#include "tensor.hpp"

#ifndef TILE_DIM
#define TILE_DIM 16
#endif

using BlockId = std::uint64_t;
using LocalId = std::uint16_t;

inline std::size_t num_blocks_for_dim(int dim)
{
    return (static_cast<std::size_t>(dim) + TILE_DIM - 1) / TILE_DIM;
}

// block_id = (bi * nbj + bj) * nbk + bk
inline BlockId encode_block_id(std::size_t block_i, std::size_t block_j, std::size_t block_k,
                               std::size_t num_blocks_j, std::size_t num_blocks_k)
{
    return (BlockId(block_i) * BlockId(num_blocks_j) + BlockId(block_j)) * BlockId(num_blocks_k) +
           BlockId(block_k);
}

inline void decode_block_id(BlockId block_id, std::size_t num_blocks_j, std::size_t num_blocks_k,
                            std::size_t& block_i, std::size_t& block_j, std::size_t& block_k)
{
    block_k = std::size_t(block_id % BlockId(num_blocks_k));
    const BlockId rest = block_id / BlockId(num_blocks_k);
    block_j = std::size_t(rest % BlockId(num_blocks_j));
    block_i = std::size_t(rest / BlockId(num_blocks_j));
}

// local_id = (li * 16 + lj) * 16 + lk
constexpr LocalId encode_local_id(int local_i, int local_j, int local_k)
{
    return LocalId((local_i * TILE_DIM + local_j) * TILE_DIM + local_k);
}

constexpr void decode_local_id(LocalId local_id, int& local_i, int& local_j, int& local_k)
{
    local_k = int(local_id) % TILE_DIM;
    local_j = (int(local_id) / TILE_DIM) % TILE_DIM;
    local_i = int(local_id) / (TILE_DIM * TILE_DIM);
}

inline void encode_coordinate(int i, int j, int k, std::size_t num_blocks_j,
                              std::size_t num_blocks_k, BlockId& block_id, LocalId& local_id)
{
    block_id = encode_block_id(std::size_t(i) / TILE_DIM, std::size_t(j) / TILE_DIM,
                               std::size_t(k) / TILE_DIM, num_blocks_j, num_blocks_k);
    local_id = encode_local_id(i % TILE_DIM, j % TILE_DIM, k % TILE_DIM);
}

inline void decode_coordinate(BlockId block_id, LocalId local_id, std::size_t num_blocks_j,
                              std::size_t num_blocks_k, int& i, int& j, int& k)
{
    std::size_t bi, bj, bk;
    decode_block_id(block_id, num_blocks_j, num_blocks_k, bi, bj, bk);
    int li, lj, lk;
    decode_local_id(local_id, li, lj, lk);
    i = int(bi * TILE_DIM + li);
    j = int(bj * TILE_DIM + lj);
    k = int(bk * TILE_DIM + lk);
}

// partition.cu:1500-1515 (null stream, synchronous)
void partition_tensor_hybrid(const COOTensor& tensor, HybridCOOTensor& hybrid,
                             double dense_threshold = 0.03);

// partition.cu:581-1493: tiles with >= int(4096 * threshold) elements are
// dense (threshold <= 0: the CU-scaled auto balance); the rest is the
// residual COO.  Reads tensor.d_m0..d_val.
void partition_tensor_hybrid_gpu(const COOTensor& tensor, HybridCOOTensor& hybrid,
                                 double dense_threshold, hipStream_t stream);

// partition.cu:1517-1560
void free_hybrid_tensor(HybridCOOTensor& hybrid);

// partition.cu:1865-2329: per-mode row-sorted views of the residual; the
// residual COO arrays are released afterwards.
void build_mttkrp_views(HybridCOOTensor& hybrid, hipStream_t stream);

// partition.cu:2387-2517: the dense pools decoded into a second hybrid
// tensor's views (the FP64 path for the dense part).
void build_dense_mttkrp_views(HybridCOOTensor& hybrid, HybridCOOTensor& dense_out,
                              hipStream_t stream);

inline void create_hybrid_format(const COOTensor& coo, HybridCOOTensor& hybrid,
                                 double density_threshold = 0.03)
{
    partition_tensor_hybrid(coo, hybrid, density_threshold);
}

inline void free_hybrid_format(HybridCOOTensor& hybrid) { free_hybrid_tensor(hybrid); }

#endif  // PARTITION_HPP
