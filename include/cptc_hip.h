/*
 * cptc_hip.h — the C ABI of the MI355X CP-ALS engine (libcptc.so).
 *
 * Plain pointers, sizes and an opaque HIP stream (`void* stream`, a
 * hipStream_t; NULL = the null stream).  Every entry point returns an int
 * status: CPTC_OK (0) or a negative CPTC_ERR_* code; none of them exits the
 * process.  The C++ interface in include/{tensor,cadr,partition,sparse,dense,
 * solver,als,common,compute_fit,generic}.hpp sits on top of these and keeps
 * the fatal-exit behaviour of the reference's C++ API.
 *
 * Layout conventions (identical to the reference's, cited per entry point):
 *   factor matrices   row-major [row * R + r], fp64
 *   Gram / FtF        R x R, fp64, symmetric
 *   packed coords     (i << 30) | (j << 15) | k, 15-bit fields, uint64
 *   row segments      blk_row / blk_start / blk_cnt, <= 1024 elements each
 *   FtV               zeroed by the caller before a mode's MTTKRP launches;
 *                     kernels only accumulate into it.
 *
 * Device pointers are marked d_; everything else is host memory.
 */
#ifndef CPTC_HIP_H
#define CPTC_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CPTC_MAX_MODES 8
#define CPTC_SEG 1024 /* row-segment length: MTTKRP_CHUNK, sparse.hpp:14-24 */

enum {
    CPTC_OK = 0,
    CPTC_ERR_ARG = -1,
    CPTC_ERR_HIP = -2,
    CPTC_ERR_UNSUPPORTED = -3,
    CPTC_ERR_IO = -4,
    CPTC_ERR_NUMERIC = -5,
    CPTC_ERR_STATE = -6
};

enum { CPTC_VAL_LOGNORMAL = 0, CPTC_VAL_NORMAL = 1, CPTC_VAL_POISSON1P2 = 2 };

/* Host COO tensor: idx is mode-major, idx[m * nnz + e], 0-based. */
typedef struct cptc_coo {
    int nmodes;
    uint64_t dims[CPTC_MAX_MODES];
    uint64_t nnz;
    uint32_t* idx;
    double* val;
} cptc_coo;

/* Frees idx/val of a cptc_coo filled by this library. */
void cptc_coo_free(cptc_coo* c);

/* Library status ---------------------------------------------------------- */
const char* cptc_version(void);
/* Last error message of the calling thread ("" if none). */
const char* cptc_last_error(void);
/* Number of visible HIP devices (0 on a host without a GPU; never faults). */
int cptc_device_count(void);

/* Device-memory plumbing for callers without a HIP runtime of their own
 * (tests, bench, scripting hosts): the library's runtime does the allocation
 * and copies, so one process never loads two HIP runtimes.  No reference
 * counterpart (the reference calls cudaMalloc/cudaMemcpy directly). */
int cptc_dev_malloc(size_t bytes, void** d_ptr);
int cptc_dev_free(void* d_ptr);
int cptc_dev_upload(void* d_dst, const void* src, size_t bytes);
int cptc_dev_download(void* dst, const void* d_src, size_t bytes);
int cptc_dev_memset(void* d_ptr, int value, size_t bytes);
/* hipDeviceSynchronize, reporting any pending asynchronous error. */
int cptc_dev_sync(void);

/* ========================================================================
 * Ingest.
 * ======================================================================== */

/* Order-3 `.tns` parser with the reference's semantics: `i j k v` per line,
 * ' '/'\t' separators, '#' lines and lines without a parsable value skipped,
 * index m -> (m > 0 ? m - 1 : 0), dims = max + 1.
 * Replaces load_tns_file (tensor.cu:39-271; tensor.hpp:346-349). */
int cptc_tns_load3(const char* path, cptc_coo* out);

/* Number of index columns of the first numeric line, or < 0.
 * Replaces probe_tns_nmodes (generic.cu:983-1021; generic.hpp:30). */
int cptc_tns_probe_nmodes(const char* path);

/* N-order `.tns` parser with the generic driver's semantics.
 * Replaces load_tns_generic (generic.cu:1023-1155; generic.hpp:31-34). */
int cptc_tns_load_generic(const char* path, cptc_coo* out);

/* Writes 1-based `.tns` text (shortest round-trip values). */
int cptc_tns_write(const char* path, const cptc_coo* c);

/* ========================================================================
 * Synthetic inputs (deterministic for a seed; no reference counterpart).
 * ======================================================================== */
int cptc_synth_config(int config, uint64_t seed, cptc_coo* out);
int cptc_synth_zipf(int nmodes, const uint64_t* dims, const double* exponents, uint64_t nnz,
                    int value_kind, uint64_t seed, cptc_coo* out);
int cptc_synth_lowrank3(uint64_t n, int rank, double keep_p, double noise_sigma, uint64_t seed,
                        cptc_coo* out);
int cptc_synth_blocks3(uint64_t n, int nblocks, double fill_lo, double fill_hi, double bg_density,
                       uint64_t seed, cptc_coo* out);
int cptc_synth_units5(const uint64_t* dims, int nunits, double fill_lo, double fill_hi,
                      uint64_t total_nnz, int signal_rank, uint64_t seed, cptc_coo* out);

/* ========================================================================
 * Layout (bit-exact with the reference).
 * ======================================================================== */

/* CADR degree-descending relabel of an order-3 COO (host arrays).  Degrees
 * are counted on the device; the relabel order is the reference's
 * std::sort(iota, deg[a] > deg[b]) run on the host.  perm[m][old] = new.
 * If `relabel` != 0 the coordinates are rewritten in place.
 * Replaces compute_cadr_reordering + apply_cadr_reordering (cadr.cu:23-81). */
int cptc_cadr3(int32_t* m0, int32_t* m1, int32_t* m2, size_t nnz, const uint64_t dims[3],
               int32_t* perm0, int32_t* perm1, int32_t* perm2, int relabel);

/* orig[old, :] = perm_factor[perm[old], :] on the device.
 * Replaces unpermute_factor_kernel / unpermute_factor_matrices (cadr.cu:9-20, 84-103). */
int cptc_unpermute_factor(const double* d_perm_factor, double* d_orig, const int32_t* d_perm,
                          size_t dim, int R, void* stream);

/* ========================================================================
 * Order-3 kernels.
 * ======================================================================== */

/* FtV[row, r] += sum_e v_e * F1[o0_e, r] * F2[o1_e, r] over the row segments
 * of one mode's row-sorted view; (F1, F2) = (B, C), (A, C), (A, B) for
 * mode 0, 1, 2 and (o0, o1) = (j, k), (i, k), (i, j).  Any R >= 1.
 * Replaces compute_sparse_mttkrp_async -> launch_mttkrp_rowsorted ->
 * mttkrp_rowsorted_coalesced_kernel<R> / mttkrp_rowsorted_generic_kernel
 * (sparse.cu:271-333, 614-711, 717-854). */
int cptc_mttkrp_sparse3(int mode, const uint64_t* d_coords, const double* d_vals,
                        const uint32_t* d_blk_row, const uint32_t* d_blk_start,
                        const uint32_t* d_blk_cnt, size_t nblocks, const double* d_F1,
                        const double* d_F2, double* d_FtV, int R, void* stream);

/* The same sum over elements [start, start + count) of one mode's view only,
 * one atomic per (element, rank) of v * F1[o0, r] * F2[o1, r]: the
 * sub-range path of compute_sparse_mttkrp_async(..., start_idx, count)
 * (mttkrp_range_generic_kernel, sparse.cu:340-397, 877-955).  The caller
 * clamps the range to the view. */
int cptc_mttkrp_sparse3_range(int mode, const uint64_t* d_coords, const double* d_vals,
                              size_t start, size_t count, const double* d_F1, const double* d_F2,
                              double* d_FtV, int R, void* stream);

/* Dense 16^3 tiles of an order-3 tensor on FP32 MFMA with an FP64 epilogue.
 * d_tiles: ntiles x {bi, bj, bk, nnz} int32; d_tile_f32: ntiles x 4096 fp32
 * cell values (layout (li*16 + lj)*16 + lk), built by cptc_dense_tiles_pack3.
 * Replaces compute_dense_mttkrp_async -> dense_mttkrp_wmma_kernel ->
 * dense_tile_mttkrp_wmma (dense.cu:89-1077, 1569-1621, 2072-2246). */
int cptc_mttkrp_dense_tiles3(int mode, const int32_t* d_tiles, const float* d_tile_f32,
                             size_t ntiles, const uint32_t* d_order, const uint32_t* d_group_off,
                             size_t ngroups, const double* d_A, const double* d_B,
                             const double* d_C, double* d_FtV, int R, int dimI, int dimJ,
                             int dimK, void* stream);

/* The same sum on the bf16 matrix cores (v_mfma_f32_32x32x16_bf16) with a
 * three-term split: every tile cell and contracted-factor value x is
 * hi + lo (bf16, round to nearest even), x*y ~ hi*hi + hi*lo + lo*hi in
 * FP32, the third factor applied in FP32 on the vector ALUs, the output in
 * FP64 as above.  Relative error per product a few 2^-18 (inputs finer than
 * the reference's TF32, coarser than FP32).  d_ws: device workspace of
 * ws_bytes >= cptc_tile_operands_bytes(max(dimI, dimJ, dimK), R), 256-byte
 * aligned, rewritten by every call (the split operand images): calls that
 * share one workspace must be ordered.  Same tile, group and output
 * conventions as cptc_mttkrp_dense_tiles3, which it replaces in the drivers
 * for R > 16 and enough tiles (ALS_TILE_KERNEL=fp32 / bf16x3 forces the
 * choice). */
size_t cptc_tile_operands_bytes(uint64_t max_dim, int R);
int cptc_mttkrp_dense_tiles3_ws(int mode, const int32_t* d_tiles, const float* d_tile_f32,
                                size_t ntiles, const uint32_t* d_order,
                                const uint32_t* d_group_off, size_t ngroups, const double* d_A,
                                const double* d_B, const double* d_C, double* d_FtV, int R,
                                int dimI, int dimJ, int dimK, void* d_ws, size_t ws_bytes,
                                void* stream);

/* Compacted split image of one target slot for the split-bf16 kernel: its
 * A operand, stored once instead of split on every launch.  Tile cell
 * (a, w, c) = (target, weight, contracted coordinate of `slot`) is image
 * cell (a, c, w) for slot 0, (c, a, w) for slot 1 and (c, w, a) for slot 2.
 * Segment a * 64 + w * 4 + e of a tile = the bf16 hi halves of cells
 * (a, w, 4e .. 4e + 3), then their bf16 lo halves (x = hi + lo, round to
 * nearest even; 16 bytes); only segments with a nonzero bit in one of their
 * 4 FP32 cells are stored, in order, with per tile 32 occupancy words and 32
 * running counts.  _mask: d_cmask (ntiles x 64 uint32) and d_segoff
 * (ntiles + 1 uint32: first segment of each tile, then the total), the total
 * in *total_segments (host; synchronises the stream).  _fill: the segments
 * into d_seg (total x 16 bytes, 16-byte aligned).  No reference counterpart
 * (the reference builds dense tiles per call, dense.cu:150-190). */
int cptc_dense_tiles_compact3_mask(const float* d_tile_f32, size_t ntiles, int slot,
                                   uint32_t* d_cmask, uint32_t* d_segoff,
                                   uint64_t* total_segments, void* stream);
int cptc_dense_tiles_compact3_fill(const float* d_tile_f32, size_t ntiles, int slot,
                                   const uint32_t* d_cmask, const uint32_t* d_segoff, void* d_seg,
                                   void* stream);

/* cptc_mttkrp_dense_tiles3_ws over the compacted split image of slot `mode`
 * (nseg segments, nseg * 16 below 2^32 - 16); the same FP64 contributions
 * per tile. */
int cptc_mttkrp_dense_tiles3_cws(int mode, const int32_t* d_tiles, const uint32_t* d_cmask,
                                 const uint32_t* d_segoff, const void* d_seg, uint64_t nseg,
                                 size_t ntiles, const uint32_t* d_order,
                                 const uint32_t* d_group_off, size_t ngroups, const double* d_A,
                                 const double* d_B, const double* d_C, double* d_FtV, int R,
                                 int dimI, int dimJ, int dimK, void* d_ws, size_t ws_bytes,
                                 void* stream);

/* Tile groups for the grouped MFMA launches (no reference counterpart; the
 * reference issues one atomic per (row, rank, tile)).  hdr: ntiles x
 * hdr_words int32 on the host ({bi, bj, bk, ...}: 4 words for order-3 tiles,
 * 6 for generic units).  The tiles sorted by (block of `slot`, then the
 * other two blocks) are cut into runs of <= max_group tiles with one target
 * block; the runs are then ordered longest first (equal lengths keep that
 * order), so a launch ends on its shortest groups.  order_out (ntiles) =
 * the tile indices run after run; group_off_out (ntiles + 1) = run
 * boundaries; *ngroups_out = number of runs.  Passing d_order / d_group_off / ngroups (device copies)
 * to cptc_mttkrp_dense_tiles3 or cptc_mttkrp_units_nd makes one wave sum
 * a group in LDS and issue one atomic per (row, rank) per group (R <= 128;
 * NULL / larger R: one atomic per tile).  Host code. */
int cptc_dense_groups(const int32_t* hdr, int hdr_words, size_t ntiles, int slot, int max_group,
                      uint32_t* order_out, uint32_t* group_off_out, size_t* ngroups_out);

/* Materialises dense tiles: cell (lid) of tile t holds the value of the last
 * pool entry with that lid (pool order), clamped to +-FLT_MAX, as fp32;
 * untouched cells are 0.  d_pool_off: ntiles+1 offsets into the pools.
 * Same tile contents as the reference's per-call shared-memory build
 * (dense.cu:150-190). */
int cptc_dense_tiles_pack3(const int32_t* d_pool_lid, const double* d_pool_val,
                           const uint64_t* d_pool_off, size_t ntiles, float* d_tile_f32,
                           void* stream);

/* G = F^T F for row-major F (rows x R); deterministic (fixed reduction order).
 * Replaces compute_gram_matrix (cublasDgemm, als.cu:115-134) and g_gram_kernel
 * (generic.cu:203-258). */
int cptc_gram(const double* d_F, size_t rows, int R, double* d_G, void* stream);

/* The update tail of one mode in one pass over the Gram: G = F^T F of the
 * unnormalised factor, n_r = sqrt(G_rr) (= the column norms, into d_norms),
 * F[:, r] /= n_r and lambda_r *= n_r (both 0 when n_r < 1e-14), and G scaled
 * to the Gram of the normalised factor (G_rs / (n_r n_s), 0 for a zero
 * column).  Same results as cptc_colnorms + cptc_normalize_absorb + cptc_gram
 * (column_norms_kernel2, normalize_absorb_lambda and compute_gram_matrix,
 * als.cu:480-517, 616-641) up to rounding, with one pass over F fewer.
 * R <= 1024. */
int cptc_gram_normalize_absorb(double* d_F, size_t rows, int R, double* d_G, double* d_norms,
                               double* d_lambda, void* stream);
/* d_p[0 .. n) = 0 by a kernel (a hipMemsetAsync node in a captured HIP graph
 * is what the drivers' graph path avoids).  No reference counterpart. */
int cptc_zero(double* d_p, size_t n, void* stream);

/* The same for R <= 1024 and rows >= 1, and, when d_other is given (with
 * d_FtF), the next mode's d_FtF = G .* d_other (cptc_hadamard) from the
 * launch that normalises G; for R <= 32 the Gram's partial sums, the norms and
 * the normalisation of G run in one workgroup launch.  Bit for bit the results
 * of cptc_gram_normalize_absorb + cptc_hadamard.  No reference counterpart. */
int cptc_gram_normalize_absorb_next(double* d_F, size_t rows, int R, double* d_G,
                                    double* d_norms, double* d_lambda, const double* d_other,
                                    double* d_FtF, void* stream);

/* One mode's whole update for a small factor in one launch (1 <= rows <=
 * 4096, R <= 32; FP64 matrix cores): F = (d_FtV * d_Ainv) /
 * lambda (cptc_apply_pinv's product with d_Ainv = pinv(FtF) given), then
 * cptc_gram_normalize_absorb_next on it (G, norms, lambda, F scaled, the
 * next FtF = G .* d_other when d_other / d_FtF are given), then
 * d_FtV[0, nzero) = 0 (the next MTTKRP's output; d_FtV is read before).
 * With d_fit (and d_grams = G_0, G_1 of an order-3 model, this call's G
 * being G_2), also the Gram fit scalars of cptc_fit_gram over the new
 * factor and d_FtV: d_fit[0] = iprod, d_fit[1] = model^2.  With next_pinv
 * (which needs d_other / d_FtF), d_Ainv is then overwritten with
 * cptc_pinv_sym of the new d_FtF (the same bits when the fast path accepts
 * it; the Jacobi pseudoinverse otherwise).  Results equal the separate
 * calls' up to summation order (als.cu:480-517, 659-715; solver.cu:900-1002).
 * Uses the library's Gram and pinv scratch and a device counter: calls that
 * overlap on one GPU race.  No reference counterpart: the reference runs
 * these as separate kernels. */
int cptc_update_small3(double* d_FtV, double* d_Ainv, double* d_F, size_t rows, int R,
                       double* d_G, double* d_norms, double* d_lambda, const double* d_other,
                       double* d_FtF, size_t nzero, const double* d_grams, double* d_fit,
                       int next_pinv, void* stream);

/* C = A o B elementwise over n doubles (C may alias A or B).
 * Replaces elementwise_mult_kernel (als.cu:101-106) and g_mul_kernel
 * (generic.cu:50-88). */
int cptc_hadamard(const double* d_A, const double* d_B, double* d_C, size_t n, void* stream);

/* F = FtV * pinv(FtF) (row-major dim x R), then F[:, r] /= div[r] when
 * d_div != NULL.  pinv by the truncated rule of the reference: singular
 * values <= R * ulp(sigma_max) are dropped.  SPD fast path (register sweep
 * for R <= 64, blocked Cholesky inverse above) when every pivot exceeds
 * 1e-10 * max diag and ||FtF||_F ||inverse||_F < 1 / (64 R DBL_EPSILON),
 * which proves that no singular value is dropped; otherwise an on-device
 * cyclic Jacobi eigen-decomposition applies the truncation rule exactly.
 * Replaces solve_als_system_svd / _nosync + factor_divide_lambda_kernel
 * (solver.cu:900-1096; als.cu:345-360, 485-499). */
int cptc_solve_pinv(const double* d_FtF, const double* d_FtV, double* d_F, size_t dim, int R,
                    const double* d_div, void* stream);

/* cptc_solve_pinv without any device allocation: no counterpart in the
 * reference.  For callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, hosts that forbid hipMalloc).
 * Same kernels and result as cptc_solve_pinv, for 1 <= R <= 128 (larger R
 * returns CPTC_ERR_ARG).  The solve's workspace is a static device array
 * of 2 * 128^2 doubles + 256 B (about 256 KB) that each GPU holds until the
 * process ends; the first call on a device looks up its address.  Calls
 * that overlap on one GPU (other streams or threads) share that array and
 * race: serialise them. */
int cptc_solve_pinv_noalloc(const double* d_FtF, const double* d_FtV, double* d_F, size_t dim,
                            int R, const double* d_div, void* stream);

/* The FP64 residual MTTKRP of cptc_mttkrp_sparse3 over the blocked layout the
 * order-3 driver builds for R in (64, 128] (even R): the mode's view re-sorted
 * by (target row block, run-level row block) with span and chunk tables
 * (span_kb = run-level block | 1 << 31 when that block's rows are staged in
 * LDS; one workgroup per chunk of one target row block).  Same sum as
 * sparse.cu:614-711 reassociated; no reference counterpart for the layout. */
/* The order-3 residual MTTKRP of cptc_mttkrp_sparse3 (sparse.cu:614-711)
 * over a blocked copy of one mode's view, even R in (64, 128], 16-byte
 * aligned factors, dims below 2^15: elements re-sorted by (target-row block
 * of 32, run-level block of 16) with the (target, o1, o0) order kept inside
 * a block pair; spans (block pairs, staged when span_kb's top bit is set) and
 * chunks (spans of one target-row block, one workgroup each) as built by the
 * driver's layout step.  Same sum up to the order of FP64 additions. */
int cptc_mttkrp_sparse3_blk(int mode, const uint64_t* d_coords, const double* d_vals,
                            const uint32_t* d_span_start, const uint32_t* d_span_cnt,
                            const uint32_t* d_span_kb, const uint32_t* d_chunk_span0,
                            const uint32_t* d_chunk_nspan, const uint32_t* d_chunk_tb,
                            size_t nchunk, const double* d_F1, const double* d_F2, double* d_FtV,
                            int R, uint64_t dim_target, uint64_t dim_f2, void* stream);

/* Measurement probe, no reference counterpart: the element-level row
 * gathers of cptc_mttkrp_sparse3_blk alone (the same chunks, spans, per-wave
 * element ranges, rows in flight and resident waves; no run-level rows, LDS
 * accumulation or atomics), i.e. the floor those gathers set on the same
 * blocked view.  d_F1 is the mode's element-level factor (F_j for mode 0,
 * F_i otherwise); d_sink (one double) is written only if the row sums hit a
 * sentinel no finite factor produces. */
int cptc_gather_probe3_blk(int mode, const uint64_t* d_coords, const uint32_t* d_span_start,
                           const uint32_t* d_span_cnt, const uint32_t* d_chunk_span0,
                           const uint32_t* d_chunk_nspan, size_t nchunk, const double* d_F1,
                           int R, double* d_sink, void* stream);

/* One launch for both halves of an order-3 mode's MTTKRP: the MFMA dense
 * tiles (as cptc_mttkrp_dense_tiles3; grouped when d_order / d_group_off are
 * given) and the FP64 residual segments (as cptc_mttkrp_sparse3) in one grid
 * whose workgroups interleave the two kinds of work.  Replaces
 * compute_mttkrp_merged_async / mttkrp_merged_kernel (dense.cu:1914-2058,
 * 2258-2511), the reference's ALS_FUSED path (als.cu:28, 529-555; R == 32
 * there).  Even R <= 128 and 16-byte aligned factors, else
 * CPTC_ERR_UNSUPPORTED.  d_FtV is accumulated into (the caller zeroes it). */
int cptc_mttkrp_merged3(int mode, const int32_t* d_tiles, const float* d_tile_f32, size_t ntiles,
                        const uint32_t* d_order, const uint32_t* d_group_off, size_t ngroups,
                        const uint64_t* d_coords, const double* d_vals, const uint32_t* d_blk_row,
                        const uint32_t* d_blk_start, const uint32_t* d_blk_cnt, size_t nblocks,
                        const double* d_A, const double* d_B, const double* d_C, double* d_FtV,
                        int R, int dimI, int dimJ, int dimK, void* stream);

/* cptc_mttkrp_merged3 with the reference's experiment switches of the merged
 * grid (dense.cu:2277-2283, 2326-2336, 2350-2381): dense_every > 0 makes
 * every dense_every-th workgroup a tile workgroup (ALS_MERGED_STRIDE; 0 =
 * spread evenly), flags bit 0 leaves the tiles out (ALS_MERGED_NO_DENSE),
 * bit 1 the residual segments (ALS_MERGED_NO_SPARSE). */
int cptc_mttkrp_merged3_ex(int mode, const int32_t* d_tiles, const float* d_tile_f32,
                           size_t ntiles, const uint32_t* d_order, const uint32_t* d_group_off,
                           size_t ngroups, const uint64_t* d_coords, const double* d_vals,
                           const uint32_t* d_blk_row, const uint32_t* d_blk_start,
                           const uint32_t* d_blk_cnt, size_t nblocks, const double* d_A,
                           const double* d_B, const double* d_C, double* d_FtV, int R, int dimI,
                           int dimJ, int dimK, int dense_every, int flags, void* stream);

/* CP-SGD on the order-3 sparse residual (sgd.cu:51-467; ALS_SGD,
 * main.cu:467-501).  cptc_sgd3_sample: d_idx[b] = SplitMix64-finalised
 * (seed + b * 0x9E3779B97F4A7C15) mod nnz (cpsgd_sample_kernel).
 * cptc_sgd3_update: every sampled element of the packed (i<<30|j<<15|k) view
 * takes one asynchronous step A[i] += g e (B[j] o C[k]), B[j] += g e (A[i] o
 * C[k]), C[k] += g e (A[i] o B[j]), e = v - sum_r lambda_r A B C
 * (cpsgd_update_kernel; atomics, so concurrent steps on a shared row land in
 * hardware order).  cptc_sgd3_loss: *d_loss = sum_b e_b^2 over the sample
 * (cpsgd_loss_kernel; deterministic reduction).  cptc_sgd3_normalize:
 * F[:, r] /= n_r and lambda_r = n_r, both 0 when n_r < 1e-14
 * (sgd_column_norms_kernel + sgd_normalize_absorb_kernel).  1 <= R <= 128;
 * the reference runs R == 32 only. */
int cptc_sgd3_sample(uint32_t* d_idx, uint32_t batch, uint64_t nnz, uint64_t seed, void* stream);
int cptc_sgd3_update(const uint64_t* d_coords, const double* d_vals, const uint32_t* d_idx,
                     uint32_t batch, double* d_A, double* d_B, double* d_C,
                     const double* d_lambda, int R, double gamma, void* stream);
int cptc_sgd3_loss(const uint64_t* d_coords, const double* d_vals, const uint32_t* d_idx,
                   uint32_t batch, const double* d_A, const double* d_B, const double* d_C,
                   const double* d_lambda, int R, double* d_loss, void* stream);
int cptc_sgd3_normalize(double* d_F, size_t rows, int R, double* d_lambda, void* stream);

/* The reference's SGD loop (execute_sgd_decomposition, sgd.cu:302-467):
 * for it in [0, iters): sample with seed + it, update, normalise A, B, C
 * when it % 5 == 0, and when it % 10 == 0 or it is the last the batch RMSE
 * sqrt(loss / batch) goes to batch_rmse[it] (-1 for the other iterations;
 * batch_rmse may be NULL).  verbose prints the reference's "[SGD]" lines.
 * dims[3] are the factor row counts; the elements are the first nnz of the
 * mode-0 residual view.  Waits for the stream before returning. */
int cptc_sgd3_run(const uint64_t* d_coords, const double* d_vals, uint64_t nnz, double* d_A,
                  double* d_B, double* d_C, const uint64_t* dims, double* d_lambda, int R,
                  int iters, double gamma, uint32_t batch, uint64_t seed, int verbose,
                  double* batch_rmse, void* stream);

/* Writes pinv(FtF) (R x R) to d_Ainv with the same rule as cptc_solve_pinv;
 * *d_path (device int, may be NULL) receives 0 = Cholesky, 1 = Jacobi. */
int cptc_pinv_sym(const double* d_FtF, double* d_Ainv, int R, int* d_path, void* stream);

/* F = FtV * Ainv (row-major dim x R), then F[:, r] /= div[r] when d_div !=
 * NULL: the second half of cptc_solve_pinv, for callers that compute
 * pinv(FtF) with cptc_pinv_sym on another stream while FtV is still being
 * accumulated.  Same split of the reference's solve + lambda divide
 * (the factor gemm at solver.cu:985-997; als.cu:345-360). */
int cptc_apply_pinv(const double* d_FtV, const double* d_Ainv, double* d_F, size_t dim, int R,
                    const double* d_div, void* stream);

/* norms[r] = ||F[:, r]||_2.  Replaces column_norms_kernel2 (als.cu:258-303). */
int cptc_colnorms(const double* d_F, size_t rows, int R, double* d_norms, void* stream);

/* F[:, r] /= n_r (0 if n_r < 1e-14); lambda[r] *= n_r (0 if n_r < 1e-14).
 * Replaces normalize_absorb_lambda_kernel (als.cu:308-342). */
int cptc_normalize_absorb(double* d_F, size_t rows, int R, const double* d_norms,
                          double* d_lambda, void* stream);

/* x[i] = min(max(x[i], lo), hi) over n doubles.  Backs clamp_factor_thrust
 * (common.cu:160-190). */
int cptc_clamp(double* d_x, size_t n, double lo, double hi, void* stream);

/* Gram fit scalars: out[0] = iprod = sum_r lambda_r <F[:, r], M[:, r]>,
 * out[1] = model^2 = sum_{r,s} lambda_r lambda_s prod_m G_m[r, s]
 * over the `ngram` Grams in d_grams (consecutive R x R blocks).
 * Replaces the Gram fit of als.cu:659-715 and generic.cu:2174-2214. */
int cptc_fit_gram(const double* d_F, const double* d_M, size_t rows, const double* d_lambda,
                  const double* d_grams, int ngram, int R, double* d_out2, void* stream);

/* Exact residual over one row-sorted order-3 view (any mode's view):
 * out[0] += sum (v - sum_r lambda_r A B C)^2, out[1] += sum v^2.
 * d_lambda NULL = no weights.  Replaces residual_sparse_view_kernel +
 * sumsq_sparse_view_kernel (common.cu:251-342, 442-474). */
int cptc_residual3_view(const uint64_t* d_coords, const double* d_vals, size_t nnz,
                        const double* d_A, const double* d_B, const double* d_C,
                        const double* d_lambda, int R, double* d_out2, void* stream);

/* The same over dense-tile pools (entries, duplicates included).
 * Replaces residual_dense_tiles_kernel + sumsq_dense_tiles_kernel
 * (common.cu:345-439, 477-505). */
int cptc_residual3_tiles(const int32_t* d_tiles, const uint64_t* d_pool_off,
                         const int32_t* d_pool_lid, const double* d_pool_val, size_t ntiles,
                         const double* d_A, const double* d_B, const double* d_C,
                         const double* d_lambda, int R, double* d_out2, void* stream);

/* ========================================================================
 * Order-3 CP-ALS driver (main.cu:136-672 + als.cu:362-821).
 * ======================================================================== */

typedef struct cptc_als3_opts {
    int R;               /* rank (main.cu:37: default 32) */
    double threshold;    /* dense cutoff fraction (main.cu:44: 0.03); <= 0 auto-balance */
    int path;            /* -1 env/auto, 0 auto, 1 force MFMA tiles, 2 force FP64 */
    double fill_min;     /* < 0: env ALS_FILL_MIN or the CU-scaled default */
    int skip_dense;      /* -1 env ALS_NO_DENSE, 0/1 */
    int skip_sparse;     /* -1 env ALS_NO_SPARSE, 0/1 */
    int cadr;            /* 1 = CADR relabel (the reference always does) */
    uint64_t seed;       /* factor-init seed (common.cu:83: 42) */
    int verbose;         /* 1 = reference-style stdout lines */
    int fused;           /* -1 env ALS_FUSED, 0/1: one merged launch per mode
                            (cptc_mttkrp_merged3) when MFMA tiles and the
                            residual view are both present, R even and <= 128 */
} cptc_als3_opts;

void cptc_als3_default_opts(cptc_als3_opts* o);

/* Builds CADR relabel, factor init, partition, row-sorted views and path
 * selection from a host order-3 COO.  *handle owns all device memory. */
int cptc_als3_create(const cptc_coo* coo, const cptc_als3_opts* opts, void** handle);

/* Layout and selection summary. */
typedef struct cptc_als3_info {
    uint64_t dims[3];
    uint64_t nnz;
    uint64_t sparse_nnz;      /* residual (FP64 kernel) */
    uint64_t dense_nnz;       /* dense pool entries */
    int64_t num_dense_tiles;
    int dense_cutoff;
    double avg_fill;
    double fill_min;
    int use_mfma;             /* 1 = dense tiles on MFMA, 0 = FP64 dense view */
    uint64_t segments[3];     /* residual view segments per mode */
    uint64_t dense_view_segments[3];
    int num_cus;
    int fused;                /* 1 = the merged single-grid MTTKRP is in use */
    int sparse_blocked;       /* 1 = the residual runs over the blocked layout */
    int tile_bf16x3;          /* 1 = dense tiles on the split-bf16 kernel, 0 = FP32 MFMA */
    int tiles_beside;         /* 1 = tile kernel on a side stream beside the FP64 kernel */
    int tile_compact;         /* 1 = the split-bf16 kernel reads the compacted tile images */
    uint64_t tile_segments[3];  /* 16-byte segments of mode m's compacted split image (0: none) */
    int graph_mode;           /* 1 = quiet runs replay one captured iteration (HIP graph) */
    int graph_captures;       /* iterations captured so far (a capture is redone after the
                                 library's scratch buffers were reallocated) */
    int fp64_merged;          /* 1 = FP64-only path with residual and dense-pool nonzeros in
                                 one row-sorted view: one FP64 launch per mode, and the
                                 per-mode sparse kernel time covers every nonzero */
    uint64_t merged_segments[3];  /* segments of that view per mode (0: none) */
    int small_update;         /* bit m: mode m's update runs as one launch
                                 (cptc_update_small3; R <= 32, at most 4096 rows); bit 3:
                                 mode C's launch also forms the Gram fit scalars */
} cptc_als3_info;
int cptc_als3_info_get(void* handle, cptc_als3_info* info);

/* Runs `iters` ALS iterations (continuing from the current state).  Arrays
 * of length iters (may be NULL): fit, ms per iteration (hipEvent span of
 * als.cu:613, 722-726), ms of MTTKRP per iteration (sum over modes).  With
 * opts.verbose the host waits after every iteration and prints the
 * reference's "[ALS] iter" line; otherwise every iteration is queued and the
 * host waits once at the end.  In graph mode (cptc_als3_info.graph_mode:
 * ALS_GRAPH=1, or automatically when nnz x R < 2^30) a queued run replays
 * one captured steady-state iteration for every iteration except every 8th
 * and the last (those run eagerly with their events): the same launches and
 * results, one graph launch instead of ~40 queue operations; a replayed
 * iteration's MTTKRP time is NaN. */
int cptc_als3_run(void* handle, int iters, double* fit, float* ms_iter, float* ms_mttkrp);

/* Kernel times accumulated over cptc_als3_run iterations (hipEvents on the
 * driver's stream): out6[m] = ms of the FP64 residual-view sparse MTTKRP
 * kernel of mode m (of the merged tiles + residual kernel when the fused
 * path is active), out6[3 + m] = ms of all MTTKRP launches of mode m;
 * *iters = iterations accumulated.  reset != 0 zeroes the sums after reading.
 * A queued (quiet) run times every 8th iteration and its last one; a verbose
 * run times every iteration.
 * No reference counterpart (measurement plumbing; ALS_PROFILE's
 * per-phase events, als.cu:642-651, are the closest). */
int cptc_als3_kernel_times(void* handle, double* out6, int* iters, int reset);
/* ms of the MFMA tile kernel per mode (hipEvents on the tile stream),
 * accumulated over the same iterations as cptc_als3_kernel_times and reset
 * with it; 0 for modes whose tiles ran in the merged grid or not at all.
 * Measurement helper, no reference counterpart. */
int cptc_als3_tile_times(void* handle, double* out3);
/* ms per launch of cptc_gather_probe3_blk on the handle's blocked residual
 * view and current factors, per mode (mean of `reps` launches between
 * hipEvents on the driver's stream; waits for them).  CPTC_ERR_STATE without
 * a blocked view.  Measurement helper, no reference counterpart. */
int cptc_als3_gather_probe(void* handle, int reps, double* out3);

/* CP-SGD (cptc_sgd3_run) on the handle's mode-0 residual view, factors and
 * lambda (main.cu:467-501 starts it with lambda = 1, which a fresh handle
 * has); the cached Grams are refreshed afterwards.  The handle's verbose
 * flag selects the reference's "[SGD]" lines.  CPTC_ERR_STATE when the
 * residual is empty (the reference: "[SGD] sparse views not ready."). */
int cptc_als3_sgd(void* handle, int iters, double gamma, uint32_t batch, uint64_t seed,
                  double* batch_rmse);

/* One mode's MTTKRP with the current factors into a host buffer (dim x R),
 * through the same launches as the ALS loop.  For parity tests. */
int cptc_als3_mttkrp(void* handle, int mode, double* host_out);

/* Current factor `mode` (dim x R) to host; unpermuted=1 maps rows back to
 * the input's index order (cadr.cu:84-103). */
int cptc_als3_factor(void* handle, int mode, int unpermuted, double* host_out);
int cptc_als3_set_factor(void* handle, int mode, const double* host_in);
int cptc_als3_lambda(void* handle, double* host_out);

/* Exact final fit report quantities: res^2, X^2 (common.cu:517-650). */
int cptc_als3_residual(void* handle, double* res_sq, double* x_sq);

/* Copies of the layout for bit-exactness tests.  Sizes via *_info first. */
int cptc_als3_perm(void* handle, int mode, int32_t* host_out);
int cptc_als3_view(void* handle, int which /*0 residual, 1 dense-fp64, 2 merged fp64*/, int mode,
                   uint64_t* coords, double* vals, uint32_t* blk_row, uint32_t* blk_start,
                   uint32_t* blk_cnt);
int cptc_als3_tiles(void* handle, int32_t* tiles4, uint64_t* pool_off, int32_t* pool_lid,
                    double* pool_val);

int cptc_als3_destroy(void* handle);

/* ========================================================================
 * Generic N-order path (generic.cu).  Limits of the reference
 * (generic.cu:1673-1685): 2 <= nmodes <= CPTC_MAX_MODES, 1 <= R <= 32,
 * nnz <= 0x7FFFFFFF.  Coordinates are 0-based uint32, mode-major.
 * Host factor-pointer arrays (`h_F`) hold one device pointer per mode
 * (row-major dim_m x R).
 * ======================================================================== */

/* Relabels a host COO tensor in place by the reference's rules: how =
 * "hits" | "cadr" | "none" | "auto" (NULL: "hits" when nmodes >= 4, else
 * "cadr"; anything else: "cadr"); rounds = HITS rounds (< 1 -> 1);
 * sample_budget = HITS element sample (0 -> 8000000; stride nnz / budget
 * when nnz exceeds it).  rank_out (host, sum(dims) entries, may be NULL)
 * receives new = rank[old] per mode, mode-major at offsets
 * sum(dims[0..m-1]) (identity when no relabel happened); *applied (may be
 * NULL) = 1 when the coordinates were relabelled.  Host code, bit-exact with
 * apply_reordering (generic.cu:1176-1376), auto's fill probe included. */
int cptc_gen_reorder(cptc_coo* t, const char* how, int rounds, uint64_t sample_budget,
                     uint32_t* rank_out, int* applied);

/* splitbit_hash (generic.cu:39-45), the dense-unit key hash. */
uint64_t cptc_gen_hash(uint64_t x);

/* FP64 segment MTTKRP of one mode (g_mttkrp_seg_pack_kernel,
 * generic.cu:271-343; launch 2082-2105).  For segment b of the mode's view:
 * acc_r = sum_e v_e prod_{m != mode} F_m[c_m(e), r] over the segment's
 * elements with d_skip[e] == 0 (d_skip NULL: none skipped); then
 * FtV[row_b, r] = acc_r when d_single[b] != 0, else FtV[row_b, r] += acc_r
 * (atomic, skipped when acc_r == 0).  d_scoords: (nmodes - 1) x nnz uint32;
 * row q holds the coordinates of mode level_modes[q] (host array; NULL =
 * the other modes ascending, the reference's layout).  Any element order
 * is valid; runs of equal leading coordinates inside a segment are summed
 * before their factor rows are applied.  Segments hold <= CPTC_SEG
 * elements. */
int cptc_mttkrp_seg_nd(int nmodes, int mode, const uint32_t* d_scoords, const int* level_modes,
                       const double* d_vals, const uint8_t* d_skip, uint64_t nnz,
                       const uint32_t* d_seg_row, const uint32_t* d_seg_start,
                       const uint32_t* d_seg_cnt, const uint8_t* d_single, uint64_t nseg,
                       const double* const* h_F, double* d_FtV, int R, void* stream);

/* Packed level keys for the segment MTTKRP (no reference counterpart: the
 * reference's kernel reads the SoA d_scoords, generic.cu:271-343).
 * level_bits[q] (1..32) is the width of level q's field; level 0 takes the
 * top bits: key = sum_q c_q << (bits of levels q+1 .. nlev-1).
 * cptc_level_key_bytes returns 4 (sum <= 32), 8 (sum <= 64) or 0 (no key).
 * cptc_pack_level_keys writes d_keys[e] from d_scoords (nlev x nnz uint32,
 * row q = level q). */
int cptc_level_key_bytes(int nlev, const int* level_bits);
int cptc_pack_level_keys(int nlev, const uint32_t* d_scoords, uint64_t nnz, const int* level_bits,
                         void* d_keys, int key_bytes, void* stream);

/* cptc_mttkrp_seg_nd over packed level keys (same result and the same
 * single-store / atomic rule; no skip flags).  level_modes[q] (host array)
 * is the mode of level q, level_bits its field width as packed; R even in
 * 2..32; factors 16-byte aligned.  The keys kernel streams one key and one
 * value per element and evaluates runs of equal level prefixes once. */
int cptc_mttkrp_seg_nd_keys(int nmodes, int mode, const void* d_keys, int key_bytes,
                            const int* level_modes, const int* level_bits, const double* d_vals,
                            uint64_t nnz, const uint32_t* d_seg_row, const uint32_t* d_seg_start,
                            const uint32_t* d_seg_cnt, const uint8_t* d_single, uint64_t nseg,
                            const double* const* h_F, double* d_FtV, int R, void* stream);

/* cptc_mttkrp_seg_nd_keys with the tensor's dims (host array, nmodes
 * entries; NULL = unknown).  With the dims, when the last level's factor
 * takes at most 24 KB (dim x R x 8 bytes) and there are at least 4 segments
 * per workgroup of a persistent grid (5 per CU), that factor is staged in
 * LDS once per workgroup and the per-element row gathers read LDS.  Same
 * result as cptc_mttkrp_seg_nd_keys up to the order of the atomic adds
 * (generic.cu:271-343 is the reference's segment kernel). */
int cptc_mttkrp_seg_nd_keys_dims(int nmodes, int mode, const void* d_keys, int key_bytes,
                                 const int* level_modes, const int* level_bits,
                                 const double* d_vals, uint64_t nnz, const uint32_t* d_seg_row,
                                 const uint32_t* d_seg_start, const uint32_t* d_seg_cnt,
                                 const uint8_t* d_single, uint64_t nseg,
                                 const double* const* h_F, const uint64_t* h_dims,
                                 double* d_FtV, int R, void* stream);

/* Dense units (GDUnit, generic.cu:422-427): d_unit6 = nunits x {bi, bj, bk,
 * nnz, start, outer_off}; pool lid = la * 256 + lb * 16 + lc (slot order).
 * Packs each unit's pool into a 16^3 FP32 tile (nunits x 4096 floats):
 * duplicates summed in FP64, then rounded once (the reference sums them
 * with FP32 shared-memory atomics, generic.cu:447-466). */
int cptc_units_pack_nd(const uint32_t* d_unit6, uint64_t nunits, const uint32_t* d_lid,
                       const double* d_val, float* d_tiles, void* stream);
/* The same cells kept in FP64 (nunits x 4096 doubles, d_img 16-byte
 * aligned; duplicates summed in FP64): the operand of
 * cptc_gen_unit_sums_img.  No reference counterpart. */
int cptc_units_pack_nd_f64(const uint32_t* d_unit6, uint64_t nunits, const uint32_t* d_lid,
                           const double* d_val, double* d_img, void* stream);

/* Per-unit FP64 weights W[u, r] = prod_{k < nouter} F_{outer[k]}[
 * outer_coords[outer_off(u) + k], r] (generic.cu:470-490); W = 1 when
 * nouter == 0.  outer_modes: host array of nouter mode ids. */
int cptc_units_weights_nd(const uint32_t* d_unit6, uint64_t nunits,
                          const uint32_t* d_outer_coords, int nouter, const int* outer_modes,
                          const double* const* h_F, int R, double* d_W, void* stream);

/* Dense-unit MTTKRP for tile slot `slot` (g_dense_tile_mttkrp_kernel,
 * generic.cu:429-561): FtV[b_slot + t, r] += sum over the unit's two other
 * slots of T * F_a * F_b * W[u, r], with F_slot0..2 the factors of the inner
 * modes and dim0..2 their dims.  FP32 MFMA inner products, FP64 epilogue. */
int cptc_mttkrp_units_nd(int slot, const uint32_t* d_unit6, uint64_t nunits,
                         const float* d_tiles, const double* d_W, const uint32_t* d_order,
                         const uint32_t* d_group_off, size_t ngroups, const double* d_F0,
                         const double* d_F1, const double* d_F2, int dim0, int dim1, int dim2,
                         double* d_FtV, int R, void* stream);

/* The same on the split-bf16 kernel of cptc_mttkrp_dense_tiles3_ws (same
 * workspace rule, max_dim = max(dim0, dim1, dim2)); the generic driver's
 * choice under the same rule (GEN_TILE_KERNEL=fp32 / bf16x3 forces it). */
int cptc_mttkrp_units_nd_ws(int slot, const uint32_t* d_unit6, uint64_t nunits,
                            const float* d_tiles, const double* d_W, const uint32_t* d_order,
                            const uint32_t* d_group_off, size_t ngroups, const double* d_F0,
                            const double* d_F1, const double* d_F2, int dim0, int dim1, int dim2,
                            double* d_FtV, int R, void* d_ws, size_t ws_bytes, void* stream);

/* cptc_mttkrp_units_nd_ws over the units' compacted split image of `slot`
 * (cptc_dense_tiles_compact3_mask / _fill over the unit tiles, same slot). */
int cptc_mttkrp_units_nd_cws(int slot, const uint32_t* d_unit6, uint64_t nunits,
                             const uint32_t* d_cmask, const uint32_t* d_segoff, const void* d_seg,
                             uint64_t nseg, const double* d_W, const uint32_t* d_order,
                             const uint32_t* d_group_off, size_t ngroups, const double* d_F0,
                             const double* d_F1, const double* d_F2, int dim0, int dim1, int dim2,
                             double* d_FtV, int R, void* d_ws, size_t ws_bytes, void* stream);

/* A small factor's update tail in one launch (rows x R <= 65536, R <= 32):
 * cptc_gen_normalize, then the Gram of the normalised factor into
 * d_grams + mode * R * R (cptc_gram), then, when next >= 0, the next mode's
 * d_FtF = prod_{g != next} G_g (cptc_gram_hadamard) and d_FtV[0 .. nzero)
 * zeroed.  The same values up to the order of the sums.  The generic
 * driver's update of such factors; no reference counterpart (the reference
 * launches these steps separately: generic.cu:2040-2060 and 2139-2171). */
int cptc_gen_normalize_gram(double* d_F, size_t rows, int R, double* d_lambda, double* d_grams,
                            int ngram, int mode, int next, double* d_FtF, double* d_FtV,
                            size_t nzero, void* stream);

/* out = prod_{g != skip} G_g over `ngram` consecutive R x R Grams (all ones
 * when none remain): g_fill_kernel + g_mul_kernel, generic.cu:2044-2052. */
int cptc_gram_hadamard(const double* d_grams, int ngram, int skip, int R, double* d_out,
                       void* stream);

/* Per-unit inner sums for R <= 32: d_sums[u][r] = sum over unit u's dense
 * elements (d_lid = la 256 + lb 16 + lc, d_val) of v * Fa[16 bi + la][r] *
 * Fb[16 bj + lb][r] * Fc[16 bk + lc][r] (bi, bj, bk from d_unit6; Fa, Fb, Fc
 * the three inner modes' factors, of da, db, dc rows), FP64.  With every element in a unit, an
 * outer mode's MTTKRP is cptc_gen_unit_scatter of these sums: the same sum as
 * the segment kernel over all elements (generic.cu's path for outer modes),
 * in another order.  d_order / d_chunk_off / nchunks: the plan of
 * cptc_gen_unit_sums_plan for these units (every chunk's units share their
 * (bi, bj, bk), which the kernel relies on).  No reference counterpart. */
int cptc_gen_unit_sums(const uint32_t* d_unit6, size_t nunits, const uint32_t* d_lid,
                       const double* d_val, const uint32_t* d_order, const uint32_t* d_chunk_off,
                       size_t nchunks, const double* d_Fa, const double* d_Fb, const double* d_Fc,
                       int da, int db, int dc, int R, double* d_sums, void* stream);
/* cptc_gen_unit_sums from the units' dense FP64 images instead of their
 * pools (d_img: nunits x 4096 doubles, cell la 256 + lb 16 + lc, as
 * cptc_units_pack_nd_f64 builds them; 16-byte aligned), on the FP64 matrix
 * cores: the same sums in another order.  No reference counterpart. */
int cptc_gen_unit_sums_img(const uint32_t* d_unit6, size_t nunits, const double* d_img,
                           const uint32_t* d_order, const uint32_t* d_chunk_off, size_t nchunks,
                           const double* d_Fa, const double* d_Fb, const double* d_Fc, int da,
                           int db, int dc, int R, double* d_sums, void* stream);
/* Host: the plan of cptc_gen_unit_sums.  h_order (nunits entries) = the
 * units sorted stably by (bi, bj, bk); chunk c = h_order[h_chunk_off[c] ..
 * h_chunk_off[c + 1]), at most max_chunk units of one (bi, bj, bk);
 * h_chunk_off holds up to nunits + 1 entries; *nchunks = the chunk count. */
int cptc_gen_unit_sums_plan(const uint32_t* h_unit6, size_t nunits, int max_chunk,
                            uint32_t* h_order, uint32_t* h_chunk_off, size_t* nchunks);
/* d_FtV[i_m(u)][r] += d_sums[u][r] * prod over the other outer modes o of
 * d_Fo[o][i_o(u)][r], outer mode m = position pos of nouter; d_outer_coords
 * nunits x nouter, d_Fo a device array of nouter factor pointers, dim_m rows
 * of d_FtV.  Adds with FP64 atomics.  No reference counterpart. */
int cptc_gen_unit_scatter(const uint32_t* d_outer_coords, size_t nunits, int nouter, int pos,
                          const double* const* d_Fo, const double* d_sums, int R, size_t dim_m,
                          double* d_FtV, void* stream);

/* F = FtV (FtF + eps I)^-1 per row by Cholesky, eps = 1e-12 * tr(FtF) / R +
 * 1e-300 (tr <= 0: 1e-12 + 1e-300); a pivot s <= 0 becomes sqrt(eps).
 * g_chol_solve_kernel, generic.cu:746-819.  R <= 32.  One launch: each
 * workgroup of 64 rows factors in one wave and solves its rows, with the
 * same bits as cptc_chol_ridge_factor followed by cptc_chol_ridge_apply; no
 * scratch memory. */
int cptc_chol_ridge_solve(const double* d_FtF, const double* d_FtV, double* d_F, size_t dim,
                          int R, void* stream);

/* The two halves of cptc_chol_ridge_solve, so that the factorization can run
 * while FtV is still being computed: d_L (R x R row-major, zeros above the
 * diagonal) = the Cholesky factor of FtF + eps I (generic.cu:752-785), then
 * F = FtV (L L^T)^-1 by the per-row forward and backward substitutions
 * (generic.cu:788-818).  R <= 32. */
int cptc_chol_ridge_factor(const double* d_FtF, double* d_L, int R, void* stream);
int cptc_chol_ridge_apply(const double* d_L, const double* d_FtV, double* d_F, size_t dim, int R,
                          void* stream);

/* n_r = ||F[:, r]||_2 (non-finite or < 1e-14: 1); F[:, r] /= n_r;
 * lambda[r] = n_r.  g_col_norms2 + g_norms_finalize + g_normalize +
 * g_set_lambda, generic.cu:352-403, 867-883, 2144-2159. */
int cptc_gen_normalize(double* d_F, size_t rows, int R, double* d_lambda, void* stream);

/* out2[0] += sum_e (v_e - sum_r lambda_r prod_m F_m[c_m(e), r])^2,
 * out2[1] += sum_e v_e^2 over a device COO (nmodes x nnz uint32 coords).
 * g_exact_residual_kernel, generic.cu:936-967. */
int cptc_residual_nd(int nmodes, const uint32_t* d_coords, const double* d_vals, uint64_t nnz,
                     const double* const* h_F, const double* d_lambda, int R, double* d_out2,
                     void* stream);

/* Generic N-order CP-ALS driver (run_generic_cp, generic.cu:1639-2366). */
typedef struct cptc_gen_opts {
    int R;                   /* 1..32 */
    unsigned seed;           /* GEN_SEED (main.cu: 42) */
    char reorder[8];         /* GEN_REORDER: hits | cadr | none | auto ("" = by order) */
    int reorder_rounds;      /* GEN_REORDER_T (3) */
    uint64_t reorder_sample; /* GEN_REORDER_SAMPLE (8000000) */
    int dense;               /* GEN_DENSE (1) */
    double threshold;        /* GEN_DENSE_THRESHOLD (0.03) */
    int inner[3];            /* GEN_DENSE_INNER (0,1,2) */
    int svd;                 /* GEN_SOLVER=svd: truncated-SVD pinv instead of Cholesky */
    int profile;             /* GEN_PROFILE: per-phase events */
    int verbose;             /* reference-style [GEN] lines on stdout */
} cptc_gen_opts;

/* Defaults with the GEN_* environment switches applied. */
void cptc_gen_default_opts(cptc_gen_opts* o);

typedef struct cptc_gen_info {
    int nmodes;
    uint64_t dims[CPTC_MAX_MODES];
    uint64_t nnz;
    int R;
    char reorder[8];         /* method used */
    int reordered;           /* 1 = coordinates relabelled */
    int dense_enabled;       /* 1 = dense units present and used */
    int cutoff;
    int inner[3];
    uint64_t n_units;
    uint64_t dense_nnz;
    uint64_t nseg[CPTC_MAX_MODES];
    double prep_ms[3];       /* reorder, dense units, views */
    uint64_t kernel_nnz[CPTC_MAX_MODES];   /* elements of the MTTKRP kernel's view per mode
                                              (the inner modes' dense elements dropped) */
    int tile_bf16x3;         /* 1 = dense units on the split-bf16 kernel, 0 = FP32 MFMA */
    uint64_t unit_segments[3];  /* 16-byte segments of inner slot s's compacted split image */
    int unit_sums;           /* 1 = outer modes' MTTKRP from per-unit sums (every element in a
                                unit, R <= 32, GEN_UNIT_SUMS not 0), 0 = segment kernel */
    int unit_sums_img;       /* 1 = those sums from FP64 unit images on the matrix cores
                                (cptc_gen_unit_sums_img; GEN_UNIT_SUMS_IMG=0: from the pools) */
} cptc_gen_info;

/* Reorders a copy of `coo`, initialises the factors (mt19937(seed) U[0,1)
 * in mode order, rows permuted by the reorder map, generic.cu:1743-1782),
 * builds the dense units and the per-mode views on the device. */
int cptc_gen_create(const cptc_coo* coo, const cptc_gen_opts* opts, void** handle);
int cptc_gen_info_get(void* handle, cptc_gen_info* info);

/* Runs `iters` iterations (continuing from the current state).  Arrays of
 * length iters (may be NULL): Gram fit, iprod, model^2, ms per iteration.
 * With opts.verbose or opts.profile the host waits after every iteration
 * and prints the reference's "[GEN] iter" line (generic.cu:2030-2249);
 * ms_iter is then the host wall time of the iteration.  Otherwise all
 * iterations are queued and the host waits once; ms_iter is the GPU time
 * between consecutive iteration ends (hipEvents). */
int cptc_gen_run(void* handle, int iters, double* fit, double* iprod, double* model2,
                 double* ms_iter);

/* Per-phase ms (gram, mttkrp, solve, norm, fit) summed over the iterations
 * run with opts.profile set (generic.cu:2016-2240); *iters = iterations
 * summed; reset != 0 zeroes the sums after reading. */
int cptc_gen_profile(void* handle, double* out5, int* iters, int reset);

/* Kernel times summed over cptc_gen_run iterations (hipEvents on the
 * driver's stream): out[m] = ms of mode m's segment MTTKRP kernel,
 * out[CPTC_MAX_MODES + m] = ms of its dense-unit kernel (0 when none); an
 * outer mode on the per-unit-sum path (cptc_gen_info.unit_sums) has its
 * scatter in out[m] and the per-unit sums, when this mode formed them, in
 * out[CPTC_MAX_MODES + m];
 * *iters = iterations summed; reset != 0 zeroes the sums.  A queued
 * (quiet) run times every 8th iteration and its last one; a verbose or
 * profiled run times every iteration.  Measurement
 * plumbing (GEN_PROFILE's phase events, generic.cu:2016-2240, are the
 * closest counterpart). */
int cptc_gen_kernel_times(void* handle, double* out16, int* iters, int reset);

/* Mode `mode`'s MTTKRP with the current factors into a host buffer
 * (dim x R), through the same launches as the ALS loop. */
int cptc_gen_mttkrp(void* handle, int mode, double* host_out);
int cptc_gen_factor(void* handle, int mode, double* host_out);
int cptc_gen_set_factor(void* handle, int mode, const double* host_in);
int cptc_gen_lambda(void* handle, double* host_out);

/* Exact ||X - Xhat||^2 and ||X||^2 over all elements (generic.cu:2319-2336). */
int cptc_gen_residual(void* handle, double* res_sq, double* x_sq);

/* Layout copies for bit-exactness tests (sizes from cptc_gen_info).  Any
 * output pointer may be NULL.  rank: dims[mode] entries (new = rank[old]). */
int cptc_gen_rank(void* handle, int mode, uint32_t* host_out);
int cptc_gen_coords(void* handle, uint32_t* idx);
int cptc_gen_view(void* handle, int mode, uint32_t* scoords, double* vals, uint8_t* skip,
                  uint32_t* seg_row, uint32_t* seg_start, uint32_t* seg_cnt, uint8_t* single);
int cptc_gen_units(void* handle, uint32_t* unit6, uint32_t* outer_coords, uint32_t* lid,
                   double* val, uint8_t* is_dense);

/* GEN_DUMP text dump of factors and lambda in the reordered index space
 * (generic.cu:2253-2287) to <base>.factors.txt. */
int cptc_gen_dump(void* handle, const char* base);

/* The same dump; input_order != 0 writes row i of each factor for index i of
 * the input tensor (the reordered row rank[i]) and adds a comment line
 * saying so.  No counterpart in the reference, whose dump stays in the
 * reordered space (an external evaluator scoring it against the input file
 * would pair the wrong rows); GEN_DUMP_ORIGINAL=1 selects it in the CLI. */
int cptc_gen_dump_ex(void* handle, const char* base, int input_order);

int cptc_gen_destroy(void* handle);

/* The dense-unit known-answer test (run_dense_selftest,
 * generic.cu:1389-1637): a 40 x 24 x 36 x 3 tensor with two dense 16^3
 * blocks, R = 8, inner sets (0,1,2), (1,2,3), (0,1,3), (0,2,3), each
 * dense-only and mixed, against an FP64 host MTTKRP (relative L2 < 2e-3).
 * *failures = failing cases; prints [SELFTEST] lines when verbose. */
int cptc_gen_selftest(int verbose, int* failures);

#ifdef __cplusplus
}
#endif

#endif /* CPTC_HIP_H */
