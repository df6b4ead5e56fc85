// Order-3 CP-ALS driver: setup (CADR relabel, factor init, hybrid partition,
// row-sorted views, fill-rate path selection) and the ALS iteration.
//
// Follows main.cu:136-672 (setup and selection) and als.cu:362-821 (the
// iteration).  MI355X-native differences, none of which changes a result
// beyond floating-point reassociation:
//   * one main HIP stream per driver plus two side streams (all at the
//     default priority): within a mode the MFMA dense tiles and the
//     pseudoinverse of FtF run on the side streams while the FP64 residual
//     runs on the main one (both MTTKRP halves add into FtV atomically, the
//     pseudoinverse only reads FtF), and the main stream joins them before
//     the factor update, when the work is large enough to pay for the
//     cross-stream waits (choose_overlap).  No host synchronisation inside
//     an iteration.  ALS_SERIAL=1 queues everything on the main stream;
//   * Grams are cached per mode and refreshed right after that mode's update
//     (the reference recomputes the same matrices from the same factors);
//   * the solve is an on-device pseudoinverse (Cholesky inverse with an exact
//     Jacobi fallback) instead of cuSOLVER gesvdj.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <random>
#include <string>
#include <vector>

#include "blk3_params.hpp"
#include "cptc_hip.h"
#include "hip_util.hpp"
#include "host_util.hpp"
#include "layout.hpp"
#include "small_la.hpp"
#include "split_img.hpp"

namespace cptc {

namespace {

int env_flag(const char* name)
{
    const char* v = std::getenv(name);
    return v != nullptr ? 1 : 0;
}

struct Als3
{
    cptc_als3_opts o{};
    int R = 0;
    uint64_t dims[3] = {0, 0, 0};
    size_t nnz = 0;
    hipStream_t s = nullptr;
    hipStream_t s_pinv = nullptr, s_dense = nullptr;  // side streams, joined per mode
    hipEvent_t e_fork = nullptr, e_pinv = nullptr, e_dense = nullptr;
    bool overlap = true;
    int num_cus = 0;

    std::vector<int32_t> perm[3];
    int32_t* d_perm[3] = {nullptr, nullptr, nullptr};
    DevPartition3 part;
    DevViews3 views, dviews;
    // FP64-only path: one row-sorted view over residual and dense-pool
    // nonzeros together (want_fp64_merge); the kernels then read it
    // instead of views + dviews, which stay for the layout getters
    DevViews3 aviews;
    DevBlk3 blk;   // blocked residual views (R in (64, 128]), for the FP64 kernel
    float* d_tile_f32 = nullptr;
    // split-bf16 tile kernel (choose_tiles) and its per-launch operand images
    bool tile_b3 = false;
    bool dense_beside = false;   // tile kernel on the side stream, beside the FP64 kernel
    void* d_tile_ws = nullptr;
    size_t tile_ws_bytes = 0;
    // compacted tile image of the split-bf16 kernel (ALS_TILE_COMPACT=0: dense)
    SplitImg timg[3];   // compacted split tile image per target mode
    // per-mode tile groups (one target row block each) for the grouped MFMA launch
    uint32_t* d_order[3] = {nullptr, nullptr, nullptr};
    uint32_t* d_goff[3] = {nullptr, nullptr, nullptr};
    size_t ngroups[3] = {0, 0, 0};
    bool use_mfma = false;
    double fill_min = 0.08, avg_fill = 0.0;
    int64_t tiles_total = 0;
    uint64_t dense_nnz_total = 0;
    bool skip_dense = false, skip_sparse = false;
    bool fused = false;   // merged single-grid MTTKRP (ALS_FUSED)
    int merged_every = 0, merged_flags = 0;   // ALS_MERGED_STRIDE / _NO_DENSE / _NO_SPARSE

    double* d_F = nullptr;  // [A | B | C]
    double* F[3] = {nullptr, nullptr, nullptr};
    double* d_lambda = nullptr;
    double* d_G = nullptr;  // 3 x R x R
    bool gram_ok[3] = {false, false, false};
    int ftf_for = -1;   // the mode whose FtF (Hadamard of the other Grams) is in d_FtF
    int ainv_for = -1;  // the mode whose pinv(FtF) is already in d_Ainv
    int ftv_zero_for = -1;   // the mode whose MTTKRP finds d_FtV already cleared
    double* d_FtF = nullptr;
    double* d_Ainv = nullptr;  // pinv(FtF) of the mode being updated
    double* d_FtV = nullptr;
    double* d_norms = nullptr;
    double* d_scal = nullptr;  // fit iprod/model2 (2) + residual (2)
    double x_sq = 0.0;
    hipEvent_t ev[9] = {};
    // around the FP64 residual-view kernel of each mode, accumulated
    hipEvent_t kev[12] = {};   // [2m, 2m+1]: FP64 (or merged) kernel; [6+2m, 7+2m]: tiles
    // the event blocks of the iteration being queued (ev / kev, or a block of
    // the pool in a queued run), the pool and the per-iteration fit scalars
    hipEvent_t* ev_cur = ev;
    hipEvent_t* kev_cur = kev;
    std::vector<hipEvent_t> ev_pool;
    double* d_fit_hist = nullptr;
    size_t fit_hist_cap = 0;
    // quiet runs of launch-bound problems replay one captured iteration
    // bit m: mode m's update is one launch (update3_small); bit 3:
    // mode C's also forms the fit scalars and clears FtV for mode A
    int small_upd = 0;
    int graph_mode = 0;                  // 1: replay untimed iterations (ALS_GRAPH / automatic)
    hipGraphExec_t gexec = nullptr;      // the captured steady-state iteration
    uint64_t g_gen = 0;                  // scratch generation it was captured at
    int n_captures = 0;                  // successful captures (cptc_als3_info.graph_captures)
    double k_sparse_ms[3] = {0, 0, 0}, k_mttkrp_ms[3] = {0, 0, 0}, k_tile_ms[3] = {0, 0, 0};
    bool tile_timed[3] = {false, false, false};
    int k_iters = 0;
    bool timing_kernels = false;   // kernel events this iteration (residual views present)
    bool timed_iter = true;        // this iteration counts in the kernel-time sums

    double* G(int m) const { return d_G + size_t(m) * R * R; }
    bool fused_active() const { return fused; }
};

// FtV = MTTKRP of `mode`; with_pinv also writes pinv(FtF) to d_Ainv (FtF
// must already hold the mode's Hadamard product) unless the previous mode's
// one-launch update formed it already.  Everything is ordered on the main
// stream when this returns.
int mttkrp_launch(Als3& h, int mode, bool with_pinv)
{
    const int R = h.R;
    const uint64_t dim = h.dims[mode];
    if (with_pinv && h.ainv_for == mode) with_pinv = false;
    // a kernel, not hipMemsetAsync: the iteration may be captured in a HIP
    // graph; skipped when the previous mode's update cleared it (TailJobs)
    if (h.ftv_zero_for != mode) CPTC_TRY(cptc_zero(h.d_FtV, dim * size_t(R), h.s));
    h.ftv_zero_for = -1;
    const double* A = h.F[0];
    const double* B = h.F[1];
    const double* C = h.F[2];
    const bool dense = h.use_mfma && !h.skip_dense && h.part.ntiles > 0;
    // ALS_FUSED: tiles and residual segments in one launch on the main stream
    const bool merged = h.fused && dense && !h.skip_sparse && h.views.ready;
    const bool dense_side = h.overlap && h.dense_beside && dense && !merged;
    const bool fork = dense_side || (h.overlap && with_pinv);
    if (fork) CPTC_HIP(hipEventRecord(h.e_fork, h.s));
    if (with_pinv)
    {
        hipStream_t ps = h.overlap ? h.s_pinv : h.s;
        if (h.overlap) CPTC_HIP(hipStreamWaitEvent(ps, h.e_fork, 0));
        CPTC_TRY(cptc_pinv_sym(h.d_FtF, h.d_Ainv, R, nullptr, ps));
        if (h.overlap) CPTC_HIP(hipEventRecord(h.e_pinv, ps));
    }
    if (merged)
    {
        const DevViews3& v = h.views;
        if (h.timing_kernels) CPTC_HIP(hipEventRecord(h.kev_cur[2 * mode], h.s));
        CPTC_TRY(cptc_mttkrp_merged3_ex(
            mode, h.part.d_tiles4, h.d_tile_f32, size_t(h.part.ntiles), h.d_order[mode],
            h.d_goff[mode], h.ngroups[mode], v.d_coords[mode], v.d_vals[mode], v.d_blk_row[mode],
            v.d_blk_start[mode], v.d_blk_cnt[mode], v.nseg[mode], A, B, C, h.d_FtV, R,
            int(h.dims[0]), int(h.dims[1]), int(h.dims[2]), h.merged_every, h.merged_flags, h.s));
        if (h.timing_kernels) CPTC_HIP(hipEventRecord(h.kev_cur[2 * mode + 1], h.s));
    }
    else if (dense)
    {
        hipStream_t ds = dense_side ? h.s_dense : h.s;
        if (dense_side) CPTC_HIP(hipStreamWaitEvent(ds, h.e_fork, 0));
        if (h.timing_kernels) CPTC_HIP(hipEventRecord(h.kev_cur[6 + 2 * mode], ds));
        if (h.tile_b3 && h.timg[mode].ready())
            CPTC_TRY(cptc_mttkrp_dense_tiles3_cws(
                mode, h.part.d_tiles4, h.timg[mode].cmask, h.timg[mode].segoff,
                h.timg[mode].seg, h.timg[mode].nseg,
                size_t(h.part.ntiles), h.d_order[mode], h.d_goff[mode], h.ngroups[mode], A, B, C,
                h.d_FtV, R, int(h.dims[0]), int(h.dims[1]), int(h.dims[2]), h.d_tile_ws,
                h.tile_ws_bytes, ds));
        else if (h.tile_b3)
            CPTC_TRY(cptc_mttkrp_dense_tiles3_ws(
                mode, h.part.d_tiles4, h.d_tile_f32, size_t(h.part.ntiles), h.d_order[mode],
                h.d_goff[mode], h.ngroups[mode], A, B, C, h.d_FtV, R, int(h.dims[0]),
                int(h.dims[1]), int(h.dims[2]), h.d_tile_ws, h.tile_ws_bytes, ds));
        else
            CPTC_TRY(cptc_mttkrp_dense_tiles3(
                mode, h.part.d_tiles4, h.d_tile_f32, size_t(h.part.ntiles), h.d_order[mode],
                h.d_goff[mode], h.ngroups[mode], A, B, C, h.d_FtV, R, int(h.dims[0]),
                int(h.dims[1]), int(h.dims[2]), ds));
        if (h.timing_kernels) CPTC_HIP(hipEventRecord(h.kev_cur[6 + 2 * mode + 1], ds));
        h.tile_timed[mode] = h.timing_kernels;
        if (dense_side) CPTC_HIP(hipEventRecord(h.e_dense, ds));
    }
    if (!h.skip_sparse && !merged)
    {
        const double* F1 = mode == 0 ? B : A;
        const double* F2 = mode == 2 ? B : C;
        // the merged FP64 view, when built, stands for both
        const DevViews3* first = h.aviews.ready ? &h.aviews : &h.views;
        const DevViews3* second = h.aviews.ready ? nullptr : &h.dviews;
        for (const DevViews3* v : {first, second})
        {
            if (!v || !v->ready) continue;
            const bool timed = h.timing_kernels && v == first;
            if (timed) CPTC_HIP(hipEventRecord(h.kev_cur[2 * mode], h.s));
            if (v == first && h.blk.ready)
            {
                const DevBlk3& b = h.blk;
                CPTC_TRY(cptc_mttkrp_sparse3_blk(
                    mode, b.d_coords[mode], b.d_vals[mode], b.d_span_start[mode],
                    b.d_span_cnt[mode], b.d_span_kb[mode], b.d_chunk_span0[mode],
                    b.d_chunk_nspan[mode], b.d_chunk_tb[mode], b.nchunk[mode], F1, F2, h.d_FtV, R,
                    h.dims[mode], h.dims[mode == 2 ? 1 : 2], h.s));
            }
            else
                CPTC_TRY(cptc_mttkrp_sparse3(mode, v->d_coords[mode], v->d_vals[mode],
                                             v->d_blk_row[mode], v->d_blk_start[mode],
                                             v->d_blk_cnt[mode], v->nseg[mode], F1, F2, h.d_FtV,
                                             R, h.s));
            if (timed) CPTC_HIP(hipEventRecord(h.kev_cur[2 * mode + 1], h.s));
        }
    }
    if (h.overlap && with_pinv) CPTC_HIP(hipStreamWaitEvent(h.s, h.e_pinv, 0));
    if (dense_side) CPTC_HIP(hipStreamWaitEvent(h.s, h.e_dense, 0));
    return CPTC_OK;
}

// The FP64-only path (tiles below fill_min) has two FP64 views of one
// tensor: the residual and the dense pool re-sorted by row (the reference's
// two launches per mode, partition.cu:2387-2517).  Here both are one view
// over all nonzeros, sorted by target row: one launch per mode, and each
// output row's nonzeros from the two sets accumulate in one segment instead
// of two flushes.  The same products summed in another order (FP64
// reassociation, ~1e-16 relative per row).  ALS_FP64_MERGE=0 keeps two.
bool want_fp64_merge(const Als3& h)
{
    const char* e = std::getenv("ALS_FP64_MERGE");
    if (e && std::strcmp(e, "0") == 0) return false;
    return !h.use_mfma && h.part.ntiles > 0 && h.part.sparse_nnz > 0;
}

// Side streams only pay when both sides of the fork run long: each fork /
// join costs ~20 us of cross-queue waits here.  Measured on MI355X: config 1
// (tiles only, R = 32) 0.31 ms per iteration overlapped vs 0.26 serial,
// config 2 (3 M FP64 nonzeros, R = 32) equal, config 3 (37.8 M FP64
// nonzeros + 82 k tiles, R = 128) 11.7 vs 15.5.  Overlap when the FP64
// MTTKRP streams at least 2^28 nonzero-ranks or the pseudoinverse takes the
// blocked Cholesky (R > 64, >= 0.1 ms); ALS_SERIAL=1 forces one stream.
// ALS_FUSED (als.cu:28, 529-555): the merged single-grid launch when both
// halves exist; the reference also requires R == 32, here any even R <= 128
// (16-byte factor rows, the grouped tile role's LDS).
void choose_fused(Als3& h, int opt)
{
    const bool want = opt < 0 ? env_flag("ALS_FUSED") != 0 : opt != 0;
    h.fused = want && h.use_mfma && h.part.ntiles > 0 && h.views.ready && !h.dviews.ready &&
              h.R <= 128 && h.R % 2 == 0;
    cptc::merged_switches(h.merged_every, h.merged_flags);
}

// Dense tile kernel: the split-bf16 one unless R <= 16 (half of its 32-rank
// block would idle; the FP32 kernel's 16-rank blocks measured faster there),
// fewer than TILE_B3_MIN_ITEMS tile x 32-rank-block items (its operand-image
// launch then costs more than it saves: config 1, 4096 tiles at R = 32,
// 0.248 against 0.236 ms per iteration) or the merged grid (which keeps the
// FP32 tile body) is in use; ALS_TILE_KERNEL=fp32 / bf16x3 forces it.  Where it runs: beside
// the FP64 residual kernel on the side stream for the FP32 kernel (config
// 3: 1.1 ms alone, the two sharing the GPU take 3.8 ms per mode against
// 4.1 back to back), on the main stream before it for the split-bf16 kernel
// (0.45 ms alone; beside the FP64 kernel both slow down: 3.7 ms per mode
// against 3.45 back to back).  ALS_TILES_BESIDE=1 / 0 forces the choice.
void choose_tiles(Als3& h)
{
    const size_t nt = size_t(std::max<int64_t>(h.part.ntiles, 0));
    const int sw = cptc::tile_kernel_switch("ALS_TILE_KERNEL");
    h.tile_b3 = h.use_mfma && nt > 0 && !h.fused && (sw < 0 ? cptc::tile_b3_auto(nt, h.R) : sw == 1);
    const char* e = std::getenv("ALS_TILES_BESIDE");
    const bool beside = e ? std::strcmp(e, "0") != 0 : !h.tile_b3;
    h.dense_beside = h.overlap && beside;
}

// Blocked residual views for R in (64, 128] (the one-element-per-wave
// kernels): 32 target rows x 16 run-level rows per block pair, 1024 elements
// per workgroup, run-level rows staged from 64 elements of a block pair on
// (blk3_params.hpp; config 3, per launch, with the chunks in run-level order:
// chunks of 512 / 768 / 1024 / 1536 / 2048 / 4096 elements 2.19-2.26 /
// 2.16-2.21 / 2.12-2.20 / 2.15-2.19 / 2.20-2.25 / 2.27-2.37 ms; 16-row target
// blocks 2.19-2.27; staging from 32 / 96 / 128 elements 2.26-2.31 / equal /
// equal; before that, in target-block order: 16 x 8 blocks 2.45-2.71, 32 x 8
// 2.46-2.52, 32 x 32 2.93-3.00).  Used when the FP64
// residual kernel runs without the MFMA tile kernel beside it: alone it is
// faster than the row-segment kernel (config 3: 2.45 against 3.1-3.4 ms per
// launch), beside the FP32 tile kernel it is not (its LDS keeps tile
// workgroups off the CUs: 11.9-13.0 against 11.7 ms per iteration).
// ALS_SPARSE_BLOCKED=1 / 0 forces it on / off.
int build_blk(Als3& h)
{
    // over the view the FP64 kernel reads first (mttkrp_launch)
    const DevViews3& v = h.aviews.ready ? h.aviews : h.views;
    if (!v.ready || v.nnz == 0 || h.R <= 64 || h.R > 128 || h.R % 2 != 0)
        return CPTC_OK;
    const char* e = std::getenv("ALS_SPARSE_BLOCKED");
    const bool beside_tiles = h.use_mfma && h.part.ntiles > 0 && h.dense_beside && !h.skip_dense;
    const bool want = e ? std::strcmp(e, "0") != 0 : !beside_tiles;
    if (!want) return CPTC_OK;
    return blk_views3_device(v, h.dims, CPTC_BLK3_LG_TB, CPTC_BLK3_LG_KB, CPTC_BLK3_CHUNK,
                             CPTC_BLK3_STAGE_MIN, h.blk, h.s);
}

// Quiet runs of small problems are paced by the host's ~40 queue operations
// per iteration (config 1: 0.218 ms of GPU time in a 0.245 ms iteration);
// those replay one captured iteration.  ALS_GRAPH=1 / 0 forces it.
void choose_graph(Als3& h)
{
    const char* e = std::getenv("ALS_GRAPH");
    if (e) h.graph_mode = std::strcmp(e, "0") != 0 ? 1 : 0;
    else h.graph_mode = double(h.nnz) * double(h.R) < double(1u << 30) ? 1 : 0;
}

// Small factors (R <= 32, at most UPDATE3_SMALL_MAX_ROWS rows): a mode's
// apply, Gram, norms, normalisation, scaling and the next mode's FtF in one
// launch instead of five, and mode C's with the Gram fit and the
// clearing of FtV for mode A (two launches fewer again).  Config 1 (256^3,
// R = 32): 0.198 ms per iteration with the separate launches.  The ALS_DEBUG
// dump reads mode C's MTTKRP after the iteration, so it keeps the separate
// fit.  ALS_SMALL_UPDATE=0 keeps the separate launches.
void choose_small_update(Als3& h)
{
    h.small_upd = 0;
    const char* e = std::getenv("ALS_SMALL_UPDATE");
    if ((e && std::strcmp(e, "0") == 0) || h.R > 32) return;
    for (int m = 0; m < 3; ++m)
        if (h.dims[m] >= 1 && h.dims[m] <= UPDATE3_SMALL_MAX_ROWS) h.small_upd |= 1 << m;
    if ((h.small_upd & 4) && !(h.o.verbose && std::getenv("ALS_DEBUG"))) h.small_upd |= 8;
}

void choose_overlap(Als3& h)
{
    const double work = double(h.views.nnz + h.dviews.nnz) * double(h.R);
    h.overlap = env_flag("ALS_SERIAL") == 0 && (h.R > 64 || work >= double(1u << 28));
}

// The main stream, the two side streams and the driver's events.
int init_streams(Als3& h)
{
    h.overlap = env_flag("ALS_SERIAL") == 0;
    for (hipStream_t* p : {&h.s, &h.s_pinv, &h.s_dense})
        CPTC_HIP(hipStreamCreateWithFlags(p, hipStreamNonBlocking));
    for (auto& e : h.ev) CPTC_HIP(hipEventCreate(&e));
    for (auto& e : h.kev) CPTC_HIP(hipEventCreate(&e));
    for (hipEvent_t* p : {&h.e_fork, &h.e_pinv, &h.e_dense})
        CPTC_HIP(hipEventCreateWithFlags(p, hipEventDisableTiming));
    return CPTC_OK;
}

// ||X - Xhat||^2 and ||X||^2 over every stored element into d_scal[2..3]
int residual_launch(Als3& h, bool with_lambda)
{
    double* out = h.d_scal + 2;
    CPTC_HIP(hipMemsetAsync(out, 0, 2 * sizeof(double), h.s));
    const double* lam = with_lambda ? h.d_lambda : nullptr;
    const bool all = h.aviews.ready;
    for (const DevViews3* v : {all ? &h.aviews : &h.views, all ? nullptr : &h.dviews})
        if (v && v->ready)
            CPTC_TRY(cptc_residual3_view(v->d_coords[0], v->d_vals[0], v->nnz, h.F[0], h.F[1],
                                         h.F[2], lam, h.R, out, h.s));
    if (h.use_mfma && h.part.ntiles > 0)
        CPTC_TRY(cptc_residual3_tiles(h.part.d_tiles4, h.part.d_pool_off, h.part.d_pool_lid,
                                      h.part.d_pool_val, size_t(h.part.ntiles), h.F[0], h.F[1],
                                      h.F[2], lam, h.R, out, h.s));
    return CPTC_OK;
}

void destroy(Als3* h)
{
    if (!h) return;
    for (hipStream_t st : {h->s, h->s_pinv, h->s_dense})
        if (st) (void)hipStreamSynchronize(st);
    free_partition(h->part);
    free_views(h->views);
    free_views(h->dviews);
    free_views(h->aviews);
    free_blk(h->blk);
    for (auto& p : h->d_perm)
        if (p) (void)hipFree(p);
    for (int m = 0; m < 3; ++m)
        for (void* p : {(void*)h->d_order[m], (void*)h->d_goff[m]})
            if (p) (void)hipFree(p);
    for (SplitImg& g : h->timg) free_split_img(g);
    for (void* p : {(void*)h->d_tile_f32, (void*)h->d_tile_ws, (void*)h->d_F, (void*)h->d_lambda, (void*)h->d_G,
                    (void*)h->d_FtF, (void*)h->d_Ainv, (void*)h->d_FtV, (void*)h->d_norms,
                    (void*)h->d_scal, (void*)h->d_fit_hist})
        if (p) (void)hipFree(p);
    for (auto& e : h->ev)
        if (e) (void)hipEventDestroy(e);
    for (auto& e : h->kev)
        if (e) (void)hipEventDestroy(e);
    for (hipEvent_t e : {h->e_fork, h->e_pinv, h->e_dense})
        if (e) (void)hipEventDestroy(e);
    for (hipEvent_t e : h->ev_pool) (void)hipEventDestroy(e);
    if (h->gexec) (void)hipGraphExecDestroy(h->gexec);
    for (hipStream_t st : {h->s, h->s_pinv, h->s_dense})
        if (st) (void)hipStreamDestroy(st);
    delete h;
}

int alloc_buffers(Als3& h);

// Tiles of each mode grouped by target row block (at most TILE_GROUP per
// wave, fewer when the tiles are few); only for the MFMA path at R <= 128
// (the grouped kernel's LDS limit).  Config 3 (split-bf16 tiles, LDS
// atomic flushes): groups of 4 / 8 / 12 / 16 / 24 measured 0.41-0.42 /
// 0.35-0.37 / 0.33-0.34 / 0.33-0.34 / 0.32-0.35 ms per launch.
constexpr int TILE_GROUP = 16;

int build_groups(Als3& h)
{
    if (!h.use_mfma || h.part.ntiles <= 0 || h.R > 128) return CPTC_OK;
    const size_t nt = size_t(h.part.ntiles);
    CPTC_REQUIRE(h.part.h_tiles4.size() == 4 * nt, CPTC_ERR_STATE, "tile groups: no host headers");
    std::vector<uint32_t> order(nt), goff(nt + 1);
    for (int m = 0; m < 3; ++m)
    {
        size_t ng = 0;
        const int cap = cptc::tile_group_cap(nt, h.R, h.num_cus, TILE_GROUP, h.tile_b3 ? 32 : 16);
        CPTC_TRY(cptc_dense_groups(h.part.h_tiles4.data(), 4, nt, m, cap, order.data(),
                                   goff.data(), &ng));
        CPTC_HIP(hipMalloc(&h.d_order[m], nt * sizeof(uint32_t)));
        CPTC_HIP(hipMalloc(&h.d_goff[m], (ng + 1) * sizeof(uint32_t)));
        CPTC_HIP(hipMemcpyAsync(h.d_order[m], order.data(), nt * sizeof(uint32_t),
                                hipMemcpyHostToDevice, h.s));
        CPTC_HIP(hipMemcpyAsync(h.d_goff[m], goff.data(), (ng + 1) * sizeof(uint32_t),
                                hipMemcpyHostToDevice, h.s));
        CPTC_HIP(hipStreamSynchronize(h.s));
        h.ngroups[m] = ng;
    }
    return CPTC_OK;
}

int create(const cptc_coo* coo, const cptc_als3_opts* opts, Als3* h)
{
    cptc_als3_opts o;
    cptc_als3_default_opts(&o);
    if (opts) o = *opts;
    h->o = o;
    CPTC_REQUIRE(coo && coo->nmodes == 3, CPTC_ERR_ARG, "cptc_als3_create: order-3 COO expected");
    CPTC_REQUIRE(o.R >= 1 && o.R <= 512, CPTC_ERR_ARG, "cptc_als3_create: R %d not in 1..512", o.R);
    h->R = o.R;
    for (int m = 0; m < 3; ++m) h->dims[m] = coo->dims[m];
    h->nnz = coo->nnz;
    for (int m = 0; m < 3; ++m)
        CPTC_REQUIRE(h->dims[m] >= 1 && h->dims[m] < (uint64_t(1) << 31), CPTC_ERR_ARG,
                     "cptc_als3_create: dim %d = %llu", m, (unsigned long long)h->dims[m]);
    CPTC_REQUIRE(coo->nnz <= size_t(UINT32_MAX), CPTC_ERR_UNSUPPORTED,
                 "cptc_als3_create: nnz %llu exceeds uint32 range", (unsigned long long)coo->nnz);
    CPTC_REQUIRE(coo->nnz == 0 || (coo->idx && coo->val), CPTC_ERR_ARG,
                 "cptc_als3_create: null COO arrays");
    // every index must lie inside its mode (the device layout kernels index by it)
    for (int m = 0; m < 3; ++m)
    {
        const uint32_t* c = coo->idx + size_t(m) * coo->nnz;
        uint64_t mx = 0;
        #pragma omp parallel for reduction(max : mx) schedule(static)
        for (int64_t e = 0; e < int64_t(coo->nnz); ++e) mx = std::max<uint64_t>(mx, c[e]);
        CPTC_REQUIRE(coo->nnz == 0 || mx < h->dims[m], CPTC_ERR_ARG,
                     "cptc_als3_create: mode %d index %llu >= dim %llu", m,
                     (unsigned long long)mx, (unsigned long long)h->dims[m]);
    }
    CPTC_TRY(init_streams(*h));
    int dev = 0;
    CPTC_HIP(hipGetDevice(&dev));
    hipDeviceProp_t prop{};
    CPTC_HIP(hipGetDeviceProperties(&prop, dev));
    h->num_cus = prop.multiProcessorCount;

    // 1. COO -> device, CADR (main.cu:176-192)
    DevCoo3 c;
    // released once the FP64 views are built, or on any early return
    struct CooGuard
    {
        DevCoo3& c;
        ~CooGuard() { free_coo(c); }
    } c_guard{c};
    CPTC_TRY(upload_coo3(coo->idx, coo->val, coo->nnz, coo->dims, c, h->s));
    if (o.cadr)
        CPTC_TRY(cadr3_device(c, h->perm, h->d_perm, 1, h->s));
    else
    {
        for (int m = 0; m < 3; ++m)
        {
            h->perm[m].resize(h->dims[m]);
            for (uint64_t x = 0; x < h->dims[m]; ++x) h->perm[m][x] = int32_t(x);
            CPTC_HIP(hipMalloc(&h->d_perm[m], h->dims[m] * sizeof(int32_t)));
            CPTC_HIP(hipMemcpyAsync(h->d_perm[m], h->perm[m].data(), h->dims[m] * sizeof(int32_t),
                                    hipMemcpyHostToDevice, h->s));
        }
    }

    // 2. factors in the relabelled space (common.cu:66-123, main.cu:228-264)
    const int R = h->R;
    const size_t tot = (h->dims[0] + h->dims[1] + h->dims[2]) * size_t(R);
    {
        std::vector<double> hf(tot);
        std::mt19937 gen(unsigned(o.seed));
        std::uniform_real_distribution<double> dis(0.0, 1.0);
        for (size_t x = 0; x < tot; ++x) hf[x] = dis(gen);
        CPTC_HIP(hipMalloc(&h->d_F, tot * sizeof(double)));
        CPTC_HIP(hipMemcpy(h->d_F, hf.data(), tot * sizeof(double), hipMemcpyHostToDevice));
        h->F[0] = h->d_F;
        h->F[1] = h->F[0] + h->dims[0] * R;
        h->F[2] = h->F[1] + h->dims[1] * R;
    }

    // 3. hybrid partition, then the COO is released (main.cu:268-301)
    CPTC_TRY(partition3_device(c, o.threshold, h->num_cus, h->part, h->s));
    h->tiles_total = h->part.ntiles;
    h->dense_nnz_total = h->part.dense_nnz;

    // 4. residual views (main.cu:304-314)
    if (h->part.sparse_nnz > 0)
        CPTC_TRY(views3_device(h->part.d_sp[0], h->part.d_sp[1], h->part.d_sp[2],
                               h->part.d_sp_val, h->part.sparse_nnz, h->dims, h->views, h->s));
    for (int m = 0; m < 3; ++m)
        if (h->part.d_sp[m])
        {
            CPTC_HIP(hipFree(h->part.d_sp[m]));
            h->part.d_sp[m] = nullptr;
        }
    if (h->part.d_sp_val)
    {
        CPTC_HIP(hipFree(h->part.d_sp_val));
        h->part.d_sp_val = nullptr;
    }

    // 5. fill-rate path selection (main.cu:334-426): the SM-count scaling
    // becomes a CU-count scaling, 0.11 / sqrt(CUs / 24) floored at 0.08
    h->avg_fill = h->part.ntiles > 0
                      ? double(h->part.dense_nnz) / (double(h->part.ntiles) * 4096.0)
                      : 0.0;
    if (o.fill_min >= 0.0)
        h->fill_min = o.fill_min;
    else if (const char* fm = std::getenv("ALS_FILL_MIN"))
        h->fill_min = std::atof(fm);
    else
    {
        h->fill_min = 0.11 / std::sqrt(double(h->num_cus) / 24.0);
        if (h->fill_min < 0.08) h->fill_min = 0.08;
    }
    int path = o.path;
    if (path < 0) path = env_flag("ALS_FORCE_WMMA") ? 1 : env_flag("ALS_FORCE_CUDA") ? 2 : 0;
    h->use_mfma = (path == 1) ? true : (path == 2) ? false : (h->avg_fill >= h->fill_min);
    // the FP64-only path reads every nonzero from one view (want_fp64_merge)
    if (want_fp64_merge(*h))
        CPTC_TRY(views3_device(reinterpret_cast<const uint32_t*>(c.d_m[0]),
                               reinterpret_cast<const uint32_t*>(c.d_m[1]),
                               reinterpret_cast<const uint32_t*>(c.d_m[2]), c.d_val, c.nnz,
                               h->dims, h->aviews, h->s));
    free_coo(c);
    h->skip_dense = o.skip_dense < 0 ? env_flag("ALS_NO_DENSE") != 0 : o.skip_dense != 0;
    h->skip_sparse = o.skip_sparse < 0 ? env_flag("ALS_NO_SPARSE") != 0 : o.skip_sparse != 0;
    if (h->part.ntiles > 0)
    {
        if (h->use_mfma)
        {
            CPTC_HIP(hipMalloc(&h->d_tile_f32, size_t(h->part.ntiles) * 4096 * sizeof(float)));
            CPTC_TRY(cptc_dense_tiles_pack3(h->part.d_pool_lid, h->part.d_pool_val,
                                            h->part.d_pool_off, size_t(h->part.ntiles),
                                            h->d_tile_f32, h->s));
        }
        else
        {
            // FP64 dense views of the pool (partition.cu:2387-2517); the pool
            // stays allocated for the layout getters but no kernel reads it
            CPTC_TRY(dense_views3_device(h->part, h->dims, h->dviews, h->s));
        }
    }

    choose_overlap(*h);
    choose_fused(*h, o.fused);
    choose_tiles(*h);
    CPTC_TRY(build_groups(*h));
    CPTC_TRY(build_blk(*h));
    CPTC_TRY(alloc_buffers(*h));
    choose_graph(*h);
    choose_small_update(*h);
    if (o.verbose && h->fused)
        std::printf("[ALS] FUSED path active: one load-balanced grid (dense MFMA + sparse FP64, "
                    "R=%d)\n", h->R);
    if (o.verbose)
        std::printf("[Main] dense_nnz=%llu sparse_nnz=%zu tiles=%lld avg_fill=%g (threshold %g) "
                    "-> %s\n",
                    (unsigned long long)h->dense_nnz_total, h->part.sparse_nnz,
                    (long long)h->tiles_total, h->avg_fill, h->fill_min,
                    h->use_mfma ? "MFMA tiles + FP64 residual" : "FP64 only");
    return CPTC_OK;
}

// ALS buffers (als.cu:389-430) and ||X||^2 (als.cu:439-450)
int alloc_buffers(Als3& hr)
{
    Als3* h = &hr;
    const int R = h->R;
    const size_t RR = size_t(R) * R;
    const uint64_t maxdim = std::max({h->dims[0], h->dims[1], h->dims[2]});
    if (h->tile_b3)
    {
        h->tile_ws_bytes = cptc_tile_operands_bytes(maxdim, R);
        CPTC_HIP(hipMalloc(&h->d_tile_ws, h->tile_ws_bytes));
        // compacted split images, one per target mode: the kernel's A operand
        // halves of every 8-cell segment with a nonzero bit, read instead of
        // splitting the dense image on every launch
        const char* e = std::getenv("ALS_TILE_COMPACT");
        if (!(e && std::strcmp(e, "0") == 0) && h->d_tile_f32)
            for (int m = 0; m < 3; ++m)
                CPTC_TRY(build_split_img(h->d_tile_f32, size_t(h->part.ntiles), m, h->timg[m], h->s));
    }
    CPTC_HIP(hipMalloc(&h->d_lambda, size_t(R) * sizeof(double)));
    CPTC_HIP(hipMalloc(&h->d_G, 3 * RR * sizeof(double)));
    CPTC_HIP(hipMalloc(&h->d_FtF, RR * sizeof(double)));
    CPTC_HIP(hipMalloc(&h->d_Ainv, RR * sizeof(double)));
    CPTC_HIP(hipMalloc(&h->d_FtV, maxdim * size_t(R) * sizeof(double)));
    CPTC_HIP(hipMalloc(&h->d_norms, size_t(R) * sizeof(double)));
    CPTC_HIP(hipMalloc(&h->d_scal, 4 * sizeof(double)));
    {
        std::vector<double> ones(size_t(R), 1.0);
        CPTC_HIP(hipMemcpyAsync(h->d_lambda, ones.data(), size_t(R) * sizeof(double),
                                hipMemcpyHostToDevice, h->s));
    }
    // ||X||^2 once (als.cu:439-450)
    CPTC_TRY(residual_launch(*h, false));
    double r2[2] = {0, 0};
    CPTC_HIP(hipMemcpyAsync(r2, h->d_scal + 2, 2 * sizeof(double), hipMemcpyDeviceToHost, h->s));
    CPTC_HIP(hipStreamSynchronize(h->s));
    h->x_sq = r2[1];
    return CPTC_OK;
}

// d_fit: where the iteration's fit scalars go; *fit_done is set when this
// update formed them (mode C on the one-launch path).
int update_mode(Als3& h, int mode, double* d_fit = nullptr, bool* fit_done = nullptr)
{
    const int R = h.R;
    const uint64_t dim = h.dims[mode];
    const int next = (mode + 1) % 3, other = 3 - next - mode;
    if (h.small_upd & (1 << mode))
    {
        // one launch: apply, Gram, norms, normalisation, scaling, the next
        // FtF, the next MTTKRP's cleared FtV and, for mode C, the fit
        const bool fuse = h.gram_ok[other];
        const bool fit = mode == 2 && d_fit && (h.small_upd & 8);
        const size_t nz = (mode < 2 || fit) ? h.dims[next] * size_t(R) : 0;
        CPTC_TRY(update3_small(h.d_FtV, h.d_Ainv, h.F[mode], dim, R, h.G(mode), h.d_norms,
                               h.d_lambda, fuse ? h.G(other) : nullptr, fuse ? h.d_FtF : nullptr,
                               nz, fit ? h.d_G : nullptr, fit ? d_fit : nullptr, fuse ? 1 : 0,
                               h.s));
        h.ftf_for = fuse ? next : -1;
        h.ainv_for = fuse ? next : -1;   // the launch also formed pinv(FtF)
        h.ftv_zero_for = nz ? next : -1;
        h.gram_ok[mode] = true;
        if (fit_done) *fit_done = fit;
        return CPTC_OK;
    }
    // F = FtV * pinv(FtF) (pinv computed beside the MTTKRP) and divide by
    // lambda; column norms, normalise + absorb and this mode's Gram refresh
    // from one Gram of the unnormalised factor (als.cu:480-517)
    CPTC_TRY(cptc_apply_pinv(h.d_FtV, h.d_Ainv, h.F[mode], dim, R, h.d_lambda, h.s));
    // The update's last launch (the column scaling) also clears FtV for the
    // next mode of the iteration (the apply above was its last reader; after
    // mode C the fit still reads it) and, above R = 32, forms the next
    // mode's FtF when its other Gram is current: two launches fewer per mode.
    // R <= 32: the Gram's sums, norms and normalisation in one workgroup, with
    // the next mode's FtF from the same launch.
    h.ainv_for = -1;
    TailJobs tj;
    if (mode < 2)
    {
        tj.zero = h.d_FtV;
        tj.nzero = h.dims[next] * size_t(R);
    }
    if (R <= 32 && dim >= 1)
    {
        const bool fuse = h.gram_ok[other];
        CPTC_TRY(gram_normalize_absorb_next_tail(h.F[mode], dim, R, h.G(mode), h.d_norms,
                                                 h.d_lambda, fuse ? h.G(other) : nullptr,
                                                 fuse ? h.d_FtF : nullptr, &tj, h.s));
        h.ftf_for = fuse ? next : -1;
    }
    else
    {
        const bool fuse = h.gram_ok[other];
        if (fuse)
        {
            tj.ga = h.G(mode);   // normalised by the launch before the scaling
            tj.gb = h.G(other);
            tj.ftf = h.d_FtF;
        }
        CPTC_TRY(gram_normalize_absorb_tail(h.F[mode], dim, R, h.G(mode), h.d_norms, h.d_lambda,
                                            &tj, h.s));
        h.ftf_for = fuse ? next : -1;
    }
    h.ftv_zero_for = mode < 2 ? next : -1;
    h.gram_ok[mode] = true;
    return CPTC_OK;
}

// One iteration's updates and the Gram fit scalars into d_out, recording the
// events of h.ev_cur / h.kev_cur; no host wait.
int enqueue_iteration(Als3& h, double* d_out, bool events = true)
{
    const int R = h.R;
    const size_t RR = size_t(R) * R;
    if (events) CPTC_HIP(hipEventRecord(h.ev_cur[0], h.s));
    bool fit_done = false;
    for (int mode = 0; mode < 3; ++mode)
    {
        const int p = mode == 0 ? 1 : 0, q = mode == 2 ? 1 : 2;
        for (int g : {p, q})
            if (!h.gram_ok[g])
            {
                CPTC_TRY(cptc_gram(h.F[g], h.dims[g], R, h.G(g), h.s));
                h.gram_ok[g] = true;
            }
        if (h.ftf_for != mode)
        {
            CPTC_TRY(cptc_hadamard(h.G(p), h.G(q), h.d_FtF, RR, h.s));
            h.ainv_for = -1;
        }
        h.ftf_for = -1;
        if (events) CPTC_HIP(hipEventRecord(h.ev_cur[1 + 2 * mode], h.s));
        CPTC_TRY(mttkrp_launch(h, mode, true));
        if (events) CPTC_HIP(hipEventRecord(h.ev_cur[2 + 2 * mode], h.s));
        CPTC_TRY(update_mode(h, mode, d_out, &fit_done));
    }
    // Gram fit (als.cu:659-715); FtV holds mode C's MTTKRP.  ev_cur[8]:
    // mode C's update done (als.cu's t_solve), for the ALS_PROFILE line
    if (events) CPTC_HIP(hipEventRecord(h.ev_cur[8], h.s));
    if (!fit_done)
        CPTC_TRY(cptc_fit_gram(h.F[2], h.d_FtV, h.dims[2], h.d_lambda, h.d_G, 3, R, d_out, h.s));
    if (events) CPTC_HIP(hipEventRecord(h.ev_cur[7], h.s));
    return CPTC_OK;
}

// The state an iteration leaves behind and finds: every Gram current, mode
// 0's FtF formed by mode 2's update and FtV not yet cleared for mode 0 (the
// fit reads it), or already cleared when mode C's one-launch update formed
// the fit, and mode 0's pinv formed by that launch too.  Only an iteration
// that starts there has the captured iteration's launches.
bool steady(const Als3& h)
{
    return h.gram_ok[0] && h.gram_ok[1] && h.gram_ok[2] && h.ftf_for == 0 &&
           h.ftv_zero_for == ((h.small_upd & 8) ? 0 : -1) &&
           h.ainv_for == ((h.small_upd & 4) ? 0 : -1);
}

// Captures one steady-state iteration (no events, kernel timing off, the
// fit scalars into d_out) into h.gexec.  Capture mode global: an allocation
// or a synchronisation inside would fail the capture instead of running.
int capture_iteration(Als3& h, double* d_out)
{
    if (h.gexec) CPTC_HIP(hipGraphExecDestroy(h.gexec));
    h.gexec = nullptr;
    const bool tk = h.timing_kernels;
    h.timing_kernels = false;
    hipGraph_t g = nullptr;
    CPTC_HIP(hipStreamBeginCapture(h.s, hipStreamCaptureModeGlobal));
    const int rc = enqueue_iteration(h, d_out, false);
    const hipError_t ee = hipStreamEndCapture(h.s, &g);
    h.timing_kernels = tk;
    if (rc != CPTC_OK)
    {
        if (g) (void)hipGraphDestroy(g);
        h.ftf_for = -1;   // nothing ran: the next iteration forms its FtF itself
        h.ainv_for = -1;
        h.ftv_zero_for = -1;
        return rc;
    }
    CPTC_HIP(ee);
    const hipError_t ie = hipGraphInstantiate(&h.gexec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    CPTC_HIP(ie);
    h.g_gen = scratch_generation();
    ++h.n_captures;
    return CPTC_OK;
}

// Fit and timings of a finished iteration (its events in h.ev_cur / h.kev_cur).
int collect_iteration(Als3& h, int it, int iters, const double sc[2], double* fit_out,
                      float* ms_out, float* mtt_out, bool replayed = false)
{
    const double Xn = std::sqrt(h.x_sq);
    const double res = std::max(h.x_sq - 2.0 * sc[0] + sc[1], 0.0);
    const double fit = Xn > 0.0 ? 1.0 - std::sqrt(res) / Xn : 0.0;
    float ms = 0.0f, mt = 0.0f;
    CPTC_HIP(hipEventElapsedTime(&ms, h.ev_cur[0], h.ev_cur[7]));
    // a replayed iteration has no per-mode events: its MTTKRP time is NaN
    if (replayed) mt = std::numeric_limits<float>::quiet_NaN();
    for (int m = 0; m < 3 && !replayed; ++m)
    {
        float x = 0.0f;
        CPTC_HIP(hipEventElapsedTime(&x, h.ev_cur[1 + 2 * m], h.ev_cur[2 + 2 * m]));
        mt += x;
        if (h.timed_iter) h.k_mttkrp_ms[m] += x;
        if (h.timing_kernels)
        {
            float k = 0.0f;
            CPTC_HIP(hipEventElapsedTime(&k, h.kev_cur[2 * m], h.kev_cur[2 * m + 1]));
            h.k_sparse_ms[m] += k;
            if (h.tile_timed[m])
            {
                float tk = 0.0f;
                CPTC_HIP(hipEventElapsedTime(&tk, h.kev_cur[6 + 2 * m], h.kev_cur[7 + 2 * m]));
                h.k_tile_ms[m] += tk;
            }
        }
    }
    if (h.timed_iter) h.k_iters++;
    if (fit_out) fit_out[it] = fit;
    if (ms_out) ms_out[it] = ms;
    if (mtt_out) mtt_out[it] = mt;
    if (h.o.verbose) std::printf("[ALS] iter %d/%d time=%g ms fit=%.10g\n", it + 1, iters, ms, fit);
    // ALS_PROFILE (als.cu:748-760), eager iterations: gram = iteration start
    // to mode C's FtF (modes A and B whole, mode C's Grams), mttkrp = mode
    // C's MTTKRP, solve = mode C's update, fit = the Gram fit
    if (h.o.verbose && std::getenv("ALS_PROFILE") && !replayed)
    {
        float ph[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        CPTC_HIP(hipEventElapsedTime(&ph[0], h.ev_cur[0], h.ev_cur[5]));
        CPTC_HIP(hipEventElapsedTime(&ph[1], h.ev_cur[5], h.ev_cur[6]));
        CPTC_HIP(hipEventElapsedTime(&ph[2], h.ev_cur[6], h.ev_cur[8]));
        CPTC_HIP(hipEventElapsedTime(&ph[3], h.ev_cur[8], h.ev_cur[7]));
        std::printf("[ALS][profile] iter %d gram=%g mttkrp=%g solve=%g fit=%g (iter=%g)\n",
                    it + 1, double(ph[0]), double(ph[1]), double(ph[2]), double(ph[3]),
                    double(ms));
    }
    return CPTC_OK;
}

// ALS_DEBUG (als.cu:595-603, 731-746), verbose runs only: the mode-C
// MTTKRP time of the iteration, then after its log line lambda[0..3],
// A[0..3], the Gram-fit scalars X^2, iprod and model^2, the first four
// per-rank terms lambda_r <C[:, r], M_C[:, r]> of iprod, FtV[0..3] (mode C's
// MTTKRP) and the exact RMSE.  Values print with the reference's default
// stream format (%g); with R < 4 only R values are printed.
int debug_mode_c(Als3& h)
{
    float ms = 0.0f;
    CPTC_HIP(hipEventElapsedTime(&ms, h.ev_cur[5], h.ev_cur[6]));
    std::printf("[DBG] modeC mttkrp wall = %g ms %s\n", double(ms),
                h.fused_active() ? "(fused)" : "(dual)");
    return CPTC_OK;
}

int debug_state(Als3& h, const double sc[2])
{
    const int R = h.R;
    const int n = R < 4 ? R : 4;
    const size_t K = h.dims[2];
    std::vector<double> lam(static_cast<size_t>(R)), a(static_cast<size_t>(n));
    std::vector<double> c(K * static_cast<size_t>(R)), m(K * static_cast<size_t>(R));
    CPTC_HIP(hipMemcpyAsync(lam.data(), h.d_lambda, lam.size() * sizeof(double),
                            hipMemcpyDeviceToHost, h.s));
    CPTC_HIP(hipMemcpyAsync(a.data(), h.F[0], a.size() * sizeof(double), hipMemcpyDeviceToHost,
                            h.s));
    CPTC_HIP(hipMemcpyAsync(c.data(), h.F[2], c.size() * sizeof(double), hipMemcpyDeviceToHost,
                            h.s));
    CPTC_HIP(hipMemcpyAsync(m.data(), h.d_FtV, m.size() * sizeof(double), hipMemcpyDeviceToHost,
                            h.s));
    CPTC_TRY(residual_launch(h, true));
    double r2[2] = {0, 0};
    CPTC_HIP(hipMemcpyAsync(r2, h.d_scal + 2, 2 * sizeof(double), hipMemcpyDeviceToHost, h.s));
    CPTC_HIP(hipStreamSynchronize(h.s));
    auto list = [&](const char* tag, auto get) {
        std::printf(" %s[0..3]=", tag);
        for (int r = 0; r < n; ++r) std::printf(r ? " %g" : "%g", get(r));
    };
    std::printf("[DBG]");
    list("lambda", [&](int r) { return lam[size_t(r)]; });
    list("A", [&](int r) { return a[size_t(r)]; });
    std::printf(" X2=%g iprod=%g model2=%g", h.x_sq, sc[0], sc[1]);
    list("work_r", [&](int r) {
        double d = 0.0;
        for (size_t k = 0; k < K; ++k) d += c[k * size_t(R) + size_t(r)] * m[k * size_t(R) + size_t(r)];
        return lam[size_t(r)] * d;
    });
    list("FtV", [&](int r) { return m[size_t(r)]; });
    std::printf("\n");
    const double res = std::max(r2[0], 0.0);
    std::printf("[DBG] exact RMSE=%g\n", h.nnz ? std::sqrt(res / double(h.nnz)) : 0.0);
    return CPTC_OK;
}

// Verbose runs wait after every iteration and print the reference's line
// (als.cu:722-735); quiet runs queue every iteration and wait once.
int run(Als3& h, int iters, double* fit_out, float* ms_out, float* mtt_out)
{
    h.timing_kernels = h.views.ready;
    h.timed_iter = true;
    if (iters <= 0) return CPTC_OK;
    struct Reset
    {
        Als3& h;
        ~Reset()
        {
            h.ev_cur = h.ev;
            h.kev_cur = h.kev;
        }
    } reset{h};
    if (h.o.verbose)
    {
        for (int it = 0; it < iters; ++it)
        {
            CPTC_TRY(enqueue_iteration(h, h.d_scal));
            double sc[2] = {0, 0};
            CPTC_HIP(hipMemcpyAsync(sc, h.d_scal, 2 * sizeof(double), hipMemcpyDeviceToHost,
                                    h.s));
            CPTC_HIP(hipStreamSynchronize(h.s));
            const bool dbg = std::getenv("ALS_DEBUG") != nullptr;
            if (dbg) CPTC_TRY(debug_mode_c(h));
            CPTC_TRY(collect_iteration(h, it, iters, sc, fit_out, ms_out, mtt_out));
            if (dbg) CPTC_TRY(debug_state(h, sc));
        }
        return CPTC_OK;
    }
    constexpr size_t PER = 21;   // ev (9) + kev (12) per iteration
    while (h.ev_pool.size() < PER * size_t(iters))
    {
        hipEvent_t e = nullptr;
        CPTC_HIP(hipEventCreate(&e));
        h.ev_pool.push_back(e);
    }
    if (h.fit_hist_cap < size_t(iters))
    {
        if (h.d_fit_hist) CPTC_HIP(hipFree(h.d_fit_hist));
        h.d_fit_hist = nullptr;
        CPTC_HIP(hipMalloc(&h.d_fit_hist, size_t(2) * iters * sizeof(double)));
        h.fit_hist_cap = size_t(iters);
    }
    // kernel events (a few microseconds of idle GPU each) on every 8th
    // iteration and the last one
    const bool views = h.views.ready;
    auto timed = [&](int it) {
        h.timed_iter = it % 8 == 0 || it == iters - 1;
        return views && h.timed_iter;
    };
    // graph mode: the other iterations replay the captured steady-state
    // iteration (one launch instead of ~40 queue operations), bracketed by the
    // iteration's first and last events; its fit scalars land in d_scal + 2
    std::vector<char> replayed(size_t(iters), 0);
    for (int it = 0; it < iters; ++it)
    {
        h.ev_cur = h.ev_pool.data() + PER * size_t(it);
        h.kev_cur = h.ev_cur + 9;
        h.timing_kernels = timed(it);
        if (h.graph_mode && !h.timed_iter && steady(h))
        {
            if (!h.gexec || h.g_gen != scratch_generation())
                if (capture_iteration(h, h.d_scal + 2) != CPTC_OK)
                {
                    h.graph_mode = 0;   // the eager path from here on
                    (void)hipGetLastError();
                }
            if (h.graph_mode)
            {
                CPTC_HIP(hipEventRecord(h.ev_cur[0], h.s));
                CPTC_HIP(hipGraphLaunch(h.gexec, h.s));
                CPTC_HIP(hipEventRecord(h.ev_cur[7], h.s));
                CPTC_HIP(hipMemcpyAsync(h.d_fit_hist + 2 * it, h.d_scal + 2, 2 * sizeof(double),
                                        hipMemcpyDeviceToDevice, h.s));
                replayed[size_t(it)] = 1;
                continue;
            }
        }
        CPTC_TRY(enqueue_iteration(h, h.d_fit_hist + 2 * it));
    }
    std::vector<double> sc(size_t(2) * iters);
    CPTC_HIP(hipMemcpyAsync(sc.data(), h.d_fit_hist, sc.size() * sizeof(double),
                            hipMemcpyDeviceToHost, h.s));
    CPTC_HIP(hipStreamSynchronize(h.s));
    for (int it = 0; it < iters; ++it)
    {
        h.ev_cur = h.ev_pool.data() + PER * size_t(it);
        h.kev_cur = h.ev_cur + 9;
        h.timing_kernels = timed(it);
        CPTC_TRY(collect_iteration(h, it, iters, sc.data() + 2 * it, fit_out, ms_out, mtt_out,
                                   replayed[size_t(it)] != 0));
    }
    h.timing_kernels = views;
    h.timed_iter = true;
    return CPTC_OK;
}

Als3* as_h(void* p) { return static_cast<Als3*>(p); }

}  // namespace

// The iteration on a caller-owned layout and caller-owned factors (the
// contract of execute_als_decomposition, als.cu:362-821).  The layout and
// the factor buffers are borrowed: they are detached before the driver's
// own buffers are released.
int als3_execute(const uint64_t dims[3], const DevPartition3& part, const DevViews3& views,
                 const DevViews3& dviews, float* tile_f32, bool use_mfma, double* A, double* B,
                 double* C, double* lambda_out, int R, int iters, bool verbose, double* fit_last)
{
    CPTC_REQUIRE(A && B && C && lambda_out && R >= 1 && R <= 512 && iters >= 0, CPTC_ERR_ARG,
                 "als3_execute: bad arguments");
    Als3* h = new Als3();
    cptc_als3_default_opts(&h->o);
    h->o.R = R;
    h->o.verbose = verbose ? 1 : 0;
    h->R = R;
    for (int m = 0; m < 3; ++m) h->dims[m] = dims[m];
    h->part = part;
    h->views = views;
    h->dviews = dviews;
    h->d_tile_f32 = tile_f32;
    h->use_mfma = use_mfma && part.ntiles > 0 && tile_f32 != nullptr;
    h->skip_dense = env_flag("ALS_NO_DENSE") != 0;
    h->skip_sparse = env_flag("ALS_NO_SPARSE") != 0;
    h->nnz = views.nnz + part.dense_nnz;
    h->F[0] = A;
    h->F[1] = B;
    h->F[2] = C;
    int rc = CPTC_OK;
    auto step = [&](int r) {
        if (rc == CPTC_OK) rc = r;
    };
    step(init_streams(*h));
    choose_overlap(*h);
    choose_fused(*h, -1);
    choose_tiles(*h);
    if (rc == CPTC_OK) step(build_groups(*h));
    if (rc == CPTC_OK) step(build_blk(*h));
    if (verbose && h->fused)
        std::printf("[ALS] FUSED path active: one load-balanced grid (dense MFMA + sparse FP64, "
                    "R=%d)\n", R);
    if (rc == CPTC_OK) step(alloc_buffers(*h));
    choose_graph(*h);
    choose_small_update(*h);
    std::vector<double> fits(static_cast<size_t>(iters > 0 ? iters : 1), 0.0);
    if (rc == CPTC_OK) step(run(*h, iters, fits.data(), nullptr, nullptr));
    if (rc == CPTC_OK)
    {
        step(hipMemcpyAsync(lambda_out, h->d_lambda, size_t(R) * sizeof(double),
                            hipMemcpyDeviceToDevice, h->s) == hipSuccess
                 ? CPTC_OK
                 : CPTC_ERR_HIP);
        step(hipStreamSynchronize(h->s) == hipSuccess ? CPTC_OK : CPTC_ERR_HIP);
        if (fit_last && iters > 0) *fit_last = fits[size_t(iters) - 1];
    }
    h->part = DevPartition3{};
    h->views = DevViews3{};
    h->dviews = DevViews3{};
    h->d_tile_f32 = nullptr;
    destroy(h);
    return rc;
}

}  // namespace cptc

using cptc::Als3;

extern "C" void cptc_als3_default_opts(cptc_als3_opts* o)
{
    if (!o) return;
    o->R = 32;
    o->threshold = 0.03;
    o->path = -1;
    o->fill_min = -1.0;
    o->skip_dense = -1;
    o->skip_sparse = -1;
    o->cadr = 1;
    o->seed = 42;
    o->verbose = 0;
    o->fused = -1;
}

extern "C" int cptc_als3_create(const cptc_coo* coo, const cptc_als3_opts* opts, void** handle)
{
    CPTC_REQUIRE(handle, CPTC_ERR_ARG, "cptc_als3_create: null handle");
    *handle = nullptr;
    Als3* h = new Als3();
    const int rc = cptc::create(coo, opts, h);
    if (rc != CPTC_OK)
    {
        cptc::destroy(h);
        return rc;
    }
    *handle = h;
    return CPTC_OK;
}

extern "C" int cptc_als3_destroy(void* handle)
{
    cptc::destroy(cptc::as_h(handle));
    return CPTC_OK;
}

extern "C" int cptc_als3_info_get(void* handle, cptc_als3_info* info)
{
    Als3* h = cptc::as_h(handle);
    CPTC_REQUIRE(h && info, CPTC_ERR_ARG, "cptc_als3_info_get: null argument");
    std::memset(info, 0, sizeof(*info));
    for (int m = 0; m < 3; ++m)
    {
        info->dims[m] = h->dims[m];
        info->segments[m] = h->views.ready ? h->views.nseg[m] : 0;
        info->dense_view_segments[m] = h->dviews.ready ? h->dviews.nseg[m] : 0;
    }
    info->nnz = h->nnz;
    info->sparse_nnz = h->part.sparse_nnz;
    info->dense_nnz = h->dense_nnz_total;
    info->num_dense_tiles = h->tiles_total;
    info->dense_cutoff = h->part.cutoff;
    info->avg_fill = h->avg_fill;
    info->fill_min = h->fill_min;
    info->use_mfma = h->use_mfma ? 1 : 0;
    info->num_cus = h->num_cus;
    info->fused = h->fused ? 1 : 0;
    info->sparse_blocked = h->blk.ready ? 1 : 0;
    info->tile_bf16x3 = h->tile_b3 ? 1 : 0;
    info->tile_compact =
        (h->tile_b3 && h->timg[0].ready() && h->timg[1].ready() && h->timg[2].ready()) ? 1 : 0;
    for (int m = 0; m < 3; ++m) info->tile_segments[m] = h->timg[m].ready() ? h->timg[m].nseg : 0;
    info->graph_mode = h->graph_mode;
    info->graph_captures = h->n_captures;
    info->fp64_merged = h->aviews.ready ? 1 : 0;
    for (int m = 0; m < 3; ++m) info->merged_segments[m] = h->aviews.ready ? h->aviews.nseg[m] : 0;
    info->small_update = h->small_upd;
    info->tiles_beside = (h->dense_beside && h->use_mfma && h->part.ntiles > 0 && !h->fused) ? 1 : 0;
    return CPTC_OK;
}

extern "C" int cptc_als3_run(void* handle, int iters, double* fit, float* ms_iter,
                             float* ms_mttkrp)
{
    Als3* h = cptc::as_h(handle);
    CPTC_REQUIRE(h && iters >= 0, CPTC_ERR_ARG, "cptc_als3_run: bad arguments");
    return cptc::run(*h, iters, fit, ms_iter, ms_mttkrp);
}

extern "C" int cptc_als3_kernel_times(void* handle, double* out6, int* iters, int reset)
{
    Als3* h = cptc::as_h(handle);
    CPTC_REQUIRE(h && out6 && iters, CPTC_ERR_ARG, "cptc_als3_kernel_times: bad arguments");
    for (int m = 0; m < 3; ++m)
    {
        out6[m] = h->k_sparse_ms[m];
        out6[3 + m] = h->k_mttkrp_ms[m];
    }
    *iters = h->k_iters;
    if (reset)
    {
        for (int m = 0; m < 3; ++m) h->k_sparse_ms[m] = h->k_mttkrp_ms[m] = h->k_tile_ms[m] = 0.0;
        h->k_iters = 0;
    }
    return CPTC_OK;
}

extern "C" int cptc_als3_sgd(void* handle, int iters, double gamma, uint32_t batch,
                             uint64_t seed, double* batch_rmse)
{
    Als3* h = cptc::as_h(handle);
    CPTC_REQUIRE(h && iters >= 0 && batch >= 1, CPTC_ERR_ARG, "cptc_als3_sgd: bad arguments");
    CPTC_REQUIRE(h->views.ready && h->views.nnz > 0, CPTC_ERR_STATE,
                 "[SGD] sparse views not ready.");
    const cptc::DevViews3& v = h->views;
    const int rc = cptc_sgd3_run(v.d_coords[0], v.d_vals[0], v.nnz, h->F[0], h->F[1], h->F[2],
                                 h->dims, h->d_lambda, h->R, iters, gamma, batch, seed,
                                 h->o.verbose, batch_rmse, h->s);
    for (bool& g : h->gram_ok) g = false;   // the factors changed
    h->ftf_for = -1;
    h->ainv_for = -1;
    h->ftv_zero_for = -1;
    return rc;
}

extern "C" int cptc_als3_tile_times(void* handle, double* out3)
{
    Als3* h = cptc::as_h(handle);
    CPTC_REQUIRE(h && out3, CPTC_ERR_ARG, "cptc_als3_tile_times: bad arguments");
    for (int m = 0; m < 3; ++m) out3[m] = h->k_tile_ms[m];
    return CPTC_OK;
}

extern "C" int cptc_als3_gather_probe(void* handle, int reps, double* out3)
{
    Als3* h = cptc::as_h(handle);
    CPTC_REQUIRE(h && out3 && reps >= 1, CPTC_ERR_ARG, "cptc_als3_gather_probe: bad arguments");
    CPTC_REQUIRE(h->blk.ready, CPTC_ERR_STATE,
                 "cptc_als3_gather_probe: no blocked residual view (R in (64, 128] with MFMA "
                 "tiles, or ALS_SPARSE_BLOCKED=1)");
    const cptc::DevBlk3& b = h->blk;
    double* sink = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int rc = CPTC_OK;
    auto fail = [&](hipError_t e) {
        cptc::set_error("cptc_als3_gather_probe: %s", hipGetErrorString(e));
        rc = CPTC_ERR_HIP;
    };
    hipError_t e = hipMalloc(&sink, sizeof(double));
    if (e == hipSuccess) e = hipEventCreate(&e0);
    if (e == hipSuccess) e = hipEventCreate(&e1);
    if (e != hipSuccess) fail(e);
    for (int m = 0; m < 3 && rc == CPTC_OK; ++m)
    {
        // the element-level factor of mttkrp_launch: F_j for mode 0, F_i otherwise
        const double* F1 = m == 0 ? h->F[1] : h->F[0];
        if ((e = hipEventRecord(e0, h->s)) != hipSuccess)
        {
            fail(e);
            break;
        }
        for (int r = 0; r < reps && rc == CPTC_OK; ++r)
            rc = cptc_gather_probe3_blk(m, b.d_coords[m], b.d_span_start[m], b.d_span_cnt[m],
                                        b.d_chunk_span0[m], b.d_chunk_nspan[m], b.nchunk[m], F1,
                                        h->R, sink, h->s);
        if (rc != CPTC_OK) break;
        float ms = 0.0f;
        if ((e = hipEventRecord(e1, h->s)) != hipSuccess || (e = hipEventSynchronize(e1)) != hipSuccess ||
            (e = hipEventElapsedTime(&ms, e0, e1)) != hipSuccess)
        {
            fail(e);
            break;
        }
        out3[m] = double(ms) / reps;
    }
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (sink)
    {
        (void)hipStreamSynchronize(h->s);
        (void)hipFree(sink);
    }
    return rc;
}

extern "C" int cptc_als3_mttkrp(void* handle, int mode, double* host_out)
{
    Als3* h = cptc::as_h(handle);
    CPTC_REQUIRE(h && host_out && mode >= 0 && mode < 3, CPTC_ERR_ARG,
                 "cptc_als3_mttkrp: bad arguments");
    h->timing_kernels = false;
    CPTC_TRY(cptc::mttkrp_launch(*h, mode, false));
    CPTC_HIP(hipMemcpyAsync(host_out, h->d_FtV, h->dims[mode] * size_t(h->R) * sizeof(double),
                            hipMemcpyDeviceToHost, h->s));
    CPTC_HIP(hipStreamSynchronize(h->s));
    return CPTC_OK;
}

extern "C" int cptc_als3_factor(void* handle, int mode, int unpermuted, double* host_out)
{
    Als3* h = cptc::as_h(handle);
    CPTC_REQUIRE(h && host_out && mode >= 0 && mode < 3, CPTC_ERR_ARG,
                 "cptc_als3_factor: bad arguments");
    const size_t n = h->dims[mode] * size_t(h->R);
    if (!unpermuted)
    {
        CPTC_HIP(hipMemcpyAsync(host_out, h->F[mode], n * sizeof(double), hipMemcpyDeviceToHost,
                                h->s));
        CPTC_HIP(hipStreamSynchronize(h->s));
        return CPTC_OK;
    }
    double* tmp = nullptr;
    CPTC_HIP(hipMalloc(&tmp, n * sizeof(double)));
    int rc = cptc_unpermute_factor(h->F[mode], tmp, h->d_perm[mode], h->dims[mode], h->R, h->s);
    if (rc == CPTC_OK)
    {
        if (hipMemcpyAsync(host_out, tmp, n * sizeof(double), hipMemcpyDeviceToHost, h->s) !=
                hipSuccess ||
            hipStreamSynchronize(h->s) != hipSuccess)
            rc = CPTC_ERR_HIP;
    }
    (void)hipFree(tmp);
    return rc;
}

extern "C" int cptc_als3_set_factor(void* handle, int mode, const double* host_in)
{
    Als3* h = cptc::as_h(handle);
    CPTC_REQUIRE(h && host_in && mode >= 0 && mode < 3, CPTC_ERR_ARG,
                 "cptc_als3_set_factor: bad arguments");
    CPTC_HIP(hipMemcpyAsync(h->F[mode], host_in, h->dims[mode] * size_t(h->R) * sizeof(double),
                            hipMemcpyHostToDevice, h->s));
    CPTC_HIP(hipStreamSynchronize(h->s));
    h->gram_ok[mode] = false;
    h->ftf_for = -1;
    h->ainv_for = -1;
    h->ftv_zero_for = -1;
    return CPTC_OK;
}

extern "C" int cptc_als3_lambda(void* handle, double* host_out)
{
    Als3* h = cptc::as_h(handle);
    CPTC_REQUIRE(h && host_out, CPTC_ERR_ARG, "cptc_als3_lambda: bad arguments");
    CPTC_HIP(hipMemcpyAsync(host_out, h->d_lambda, size_t(h->R) * sizeof(double),
                            hipMemcpyDeviceToHost, h->s));
    CPTC_HIP(hipStreamSynchronize(h->s));
    return CPTC_OK;
}

extern "C" int cptc_als3_residual(void* handle, double* res_sq, double* x_sq)
{
    Als3* h = cptc::as_h(handle);
    CPTC_REQUIRE(h && res_sq && x_sq, CPTC_ERR_ARG, "cptc_als3_residual: bad arguments");
    CPTC_TRY(cptc::residual_launch(*h, true));
    double r2[2] = {0, 0};
    CPTC_HIP(hipMemcpyAsync(r2, h->d_scal + 2, 2 * sizeof(double), hipMemcpyDeviceToHost, h->s));
    CPTC_HIP(hipStreamSynchronize(h->s));
    *res_sq = r2[0];
    *x_sq = r2[1];
    return CPTC_OK;
}

extern "C" int cptc_als3_perm(void* handle, int mode, int32_t* host_out)
{
    Als3* h = cptc::as_h(handle);
    CPTC_REQUIRE(h && host_out && mode >= 0 && mode < 3, CPTC_ERR_ARG,
                 "cptc_als3_perm: bad arguments");
    std::memcpy(host_out, h->perm[mode].data(), h->perm[mode].size() * sizeof(int32_t));
    return CPTC_OK;
}

extern "C" int cptc_als3_view(void* handle, int which, int mode, uint64_t* coords, double* vals,
                              uint32_t* blk_row, uint32_t* blk_start, uint32_t* blk_cnt)
{
    Als3* h = cptc::as_h(handle);
    CPTC_REQUIRE(h && mode >= 0 && mode < 3 && which >= 0 && which <= 2, CPTC_ERR_ARG,
                 "cptc_als3_view: bad arguments");
    const cptc::DevViews3& v = which == 0 ? h->views : which == 1 ? h->dviews : h->aviews;
    if (!v.ready) return CPTC_OK;
    auto cp = [&](void* dst, const void* src, size_t bytes) -> int {
        if (dst && src && bytes)
            CPTC_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, h->s));
        return CPTC_OK;
    };
    CPTC_TRY(cp(coords, v.d_coords[mode], v.nnz * 8));
    CPTC_TRY(cp(vals, v.d_vals[mode], v.nnz * 8));
    CPTC_TRY(cp(blk_row, v.d_blk_row[mode], v.nseg[mode] * 4));
    CPTC_TRY(cp(blk_start, v.d_blk_start[mode], v.nseg[mode] * 4));
    CPTC_TRY(cp(blk_cnt, v.d_blk_cnt[mode], v.nseg[mode] * 4));
    CPTC_HIP(hipStreamSynchronize(h->s));
    return CPTC_OK;
}

extern "C" int cptc_als3_tiles(void* handle, int32_t* tiles4, uint64_t* pool_off,
                               int32_t* pool_lid, double* pool_val)
{
    Als3* h = cptc::as_h(handle);
    CPTC_REQUIRE(h, CPTC_ERR_ARG, "cptc_als3_tiles: null handle");
    const cptc::DevPartition3& p = h->part;
    if (tiles4 && !p.h_tiles4.empty())
        std::memcpy(tiles4, p.h_tiles4.data(), p.h_tiles4.size() * sizeof(int32_t));
    if (pool_off && !p.h_pool_off.empty())
        std::memcpy(pool_off, p.h_pool_off.data(), p.h_pool_off.size() * sizeof(uint64_t));
    if (pool_lid && p.d_pool_lid && p.dense_nnz)
        CPTC_HIP(hipMemcpyAsync(pool_lid, p.d_pool_lid, p.dense_nnz * 4, hipMemcpyDeviceToHost,
                                h->s));
    if (pool_val && p.d_pool_val && p.dense_nnz)
        CPTC_HIP(hipMemcpyAsync(pool_val, p.d_pool_val, p.dense_nnz * 8, hipMemcpyDeviceToHost,
                                h->s));
    CPTC_HIP(hipStreamSynchronize(h->s));
    return CPTC_OK;
}
