/*
 * slk.h -- C ABI of libslk, an MI355X (gfx950) implementation of the DROID-SLAM
 * per-edge update path of vibekernels/slam-hands (cuda_slam, cuda_pipeline):
 * all-pairs correlation + 4-level pyramid + radius-3 lookup, SE3 reprojection
 * kernels, and Schur-complement bundle adjustment.
 *
 * Conventions (kept from the reference, cuda_slam/main.cu and ba.cuh):
 *  - every tensor argument is a caller-owned DEVICE pointer unless its name
 *    ends in `_host`; sizes are element counts;
 *  - fmaps [nframes][C][h][w]; coords [B][2][h*w] (x plane, then y plane);
 *    lookup output [B][levels*(2r+1)^2][h*w], channel l*49 + a*7 + b with a the
 *    x offset and b the y offset; poses [N][7] = [tx,ty,tz,qx,qy,qz,qw]
 *    (world->camera); disps [N][h*w]; intrinsics [4] = fx,fy,cx,cy at 1/8 res;
 *    target/weight [M][2][h*w]; eta [N][h*w] indexed by absolute keyframe;
 *  - every call is stream-ordered on `stream` (0 = legacy default stream) and
 *    returns an slk_status; work already enqueued when an error is returned is
 *    not rolled back. The reference instead exit(1)s on any CUDA error
 *    (nn.cuh:17-41); the C++ adapters in slam-hands_amd/adapters keep that.
 *
 * Each entry point cites the reference interface it replaces.
 */
#ifndef SLK_H
#define SLK_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct slk_ctx slk_ctx;

typedef enum {
    SLK_OK = 0,
    SLK_E_ARG = 1,     /* invalid argument or unsupported shape */
    SLK_E_HIP = 2,     /* HIP runtime error (message in slk_last_error) */
    SLK_E_NOT_SPD = 3, /* BA system not positive definite; poses/disps untouched
                          (the reference produces NaN here, ba.cuh:422) */
    SLK_E_STATE = 4    /* call order violated (e.g. sample before build) */
} slk_status;

typedef enum { SLK_F32 = 0, SLK_F16 = 1 } slk_dtype;

/* Contraction used for the features:
 *  SLK_PREC_F16X3 (default)  -- batched path: every pixel's features scaled
 *                               by one power of two (its largest magnitude
 *                               over the channels into [2^14, 2^15)) and split
 *                               into fp16 hi + lo (22 significant bits), three
 *                               fp16 MFMA passes hi.hi + hi.lo + lo.hi with
 *                               fp32 accumulation, ~1e-6 relative to the two
 *                               pixels' scales. fp16 features
 *                               are their own hi (lo = 0): a level-0 target
 *                               tile takes the one pass hi.hi, the exact fp16
 *                               products of the reference's cublasGemmEx on
 *                               its fp16 fmaps (main.cu:1508-1515,1573-1581),
 *                               a pooled-level tile two.
 *  SLK_PREC_BF16X3           -- hi/lo bf16 split without a scale, three bf16
 *                               MFMA passes, ~5e-5 relative to the row scale.
 *  SLK_PREC_FP32             -- fp32 MFMA (v_mfma_f32_32x32x2f32) for fp32
 *                               features.
 * The single-edge path (slk_corr_build) splits fp32 features into bf16 hi/lo
 * under either split precision, and multiplies fp16 features as fp16 MFMA
 * products with fp32 accumulation. The split precisions need C a multiple of
 * 16 and at most 128 in the batched path; other C take fp32 MFMA. */
typedef enum {
    SLK_PREC_BF16X3 = 0,
    SLK_PREC_FP32 = 1,
    SLK_PREC_F16X3 = 2
} slk_corr_precision;

/* ---------------------------------------------------------------- context */

/* Creates a context on the current HIP device for h x w feature maps with C
 * channels. corr_scale is alpha of the correlation GEMM (1/16 in the
 * reference: cublasGemmEx alpha, cuda_slam/main.cu:1506,1572). Allocates the
 * batched scratch for max_batch edges (the reference's [B,hw,hw] volumes +
 * levels, main.cu:1413-1418, become 8x8 lookup windows per pixel and level
 * plus the split features of the frames in flight) and the single-edge volume
 * and pyramid (main.cu:1400-1405). h, w <= 65536 and h*w < 2^21 (the
 * batched path's per-slot window offsets are 32-bit).
 * Replaces CorrBlock::init (cuda_slam/corr.cuh:75) and
 * BundleAdjustment::init(h, w) (cuda_slam/ba.cuh:408). levels <= 4, radius == 3. */
int slk_create(slk_ctx** ctx, int h, int w, int C, int max_batch, int levels,
               int radius, float corr_scale);

/* Releases every buffer (BundleAdjustment::destroy ba.cuh:815,
 * CorrBlock::destroy corr.cuh:259). */
int slk_destroy(slk_ctx* ctx);

/* Text of the last failure on this thread ("" if none). */
const char* slk_last_error(void);

/* Per-kernel timing of the launches this context makes (hipEvents recorded on
 * the launch stream around each kernel). Enabling (or disabling) clears the
 * totals. Replaces the reference's CudaTimer totals (cuda_slam/main.cu:41-59,
 * print_timing :2493-2507) and BundleAdjustment::print_profile (ba.cuh:805). */
int slk_profile_enable(slk_ctx* ctx, int on);

/* Totals of the idx-th distinct kernel name (synchronises on the recorded
 * events); SLK_E_ARG once idx runs past the last name. */
int slk_profile_kernel(slk_ctx* ctx, int idx, const char** name, double* total_ms,
                       int* launches);

/* ------------------------------------------------------------ correlation */

/* Selects the contraction for fp32 features (slk_corr_precision). The
 * reference has no such switch: it always contracts fp16 fmaps. */
int slk_set_corr_precision(slk_ctx* ctx, int precision);

/* CudaDroid::batch_build_and_sample_correlation(batch_size, edge_start,
 * coords_2hw, corr_out_196hw), cuda_slam/main.cu:1555-1613 (copy in
 * cuda_pipeline/slam.cuh:2851-2909). For each edge e < B: volume
 * alpha * fmaps[ii_host[e]]^T fmaps[jj_host[e]], its 2x2 avg-pool pyramid, and
 * the radius-3 bilinear lookup at coords[e] into out[e]. fmap_stride is the
 * element distance between consecutive keyframes (C*h*w for a dense buffer).
 * ii_host/jj_host are read before the call returns. B is not capped:
 * batches above max_batch run in max_batch chunks. */
int slk_corr_batch_build_and_sample(slk_ctx* ctx, const void* fmaps, int dtype,
                                    long fmap_stride, const int* ii_host,
                                    const int* jj_host, int B, const float* coords,
                                    float* out, hipStream_t stream);

/* Same with device-resident edge indices ii_dev/jj_dev [B]. */
int slk_corr_batch_build_and_sample_dev(slk_ctx* ctx, const void* fmaps, int dtype,
                                        long fmap_stride, const int* ii_dev,
                                        const int* jj_dev, int B,
                                        const float* coords, float* out,
                                        hipStream_t stream);
/* The same batched correlation over frames split once per pass: the
 * reference's backend update (run_update_pass over batches of 48 edges,
 * main.cu:2197-2203) rebuilds each frame's operands in every batch that
 * touches it. slk_corr_prepare_frames splits frames [0, nframes) of fmaps
 * (all levels, hi/lo; ~2*C*(h*w*85/64) bytes per frame, held by the
 * context until the next call or slk_destroy); the _prepared calls then
 * take ii_host/jj_host as frame indices into them and compute the batches
 * without that step. Call it again whenever fmaps change. Results are
 * bitwise those of slk_corr_batch_build_and_sample on the same fmaps. Needs
 * the split contraction (C a multiple of 16; fp16 fmaps, or fp32
 * with SLK_PREC_F16X3 or SLK_PREC_BF16X3), and the precision of the calls
 * that follow is the one in force at slk_corr_prepare_frames. */
int slk_corr_prepare_frames(slk_ctx* ctx, const void* fmaps, int dtype, long fmap_stride,
                            int nframes, hipStream_t stream);
int slk_corr_batch_build_and_sample_prepared(slk_ctx* ctx, const int* ii_host,
                                             const int* jj_host, int B, const float* coords,
                                             float* out, hipStream_t stream);

/* No counterpart in the reference. The batched correlation with
 * device-resident edge indices, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): it takes no context and calls no allocator. Its scratch
 * (feature slots, tile lists and counters, lookup windows) is one static
 * 64 MiB device array per GPU, held until the process ends; batches run in
 * launches of as many edges as fit in it (9 at 48x64, 5 at 54x96). Map sizes
 * whose one-edge scratch exceeds 64 MiB are rejected with SLK_E_ARG (e.g.
 * 256x256). Needs C a positive multiple of 16, 8 <= h, w and h*w < 2^21;
 * fp32 features take the bf16x3 split. Results are bitwise those of
 * slk_corr_batch_build_and_sample_dev. Every call on a GPU shares that
 * GPU's array: calls that overlap on one GPU (other streams or threads)
 * race and must be serialised by the caller. */
int slk_corr_batch_build_and_sample_dev_noalloc(const void* fmaps, int dtype, long fmap_stride,
                                                const int* ii_dev, const int* jj_dev, int B,
                                                const float* coords, float* out, int h, int w,
                                                int C, float corr_scale, hipStream_t stream);

/* CudaDroid::build_correlation(i, j), main.cu:1500-1526 (and
 * CorrBlock::build for one edge, corr.cuh:84): volume of (f_i, f_j) and its
 * pyramid into the context's persistent single-edge buffers. */
int slk_corr_build(slk_ctx* ctx, const void* f_i, const void* f_j, int dtype,
                   hipStream_t stream);

/* CudaDroid::sample_correlation(coords_2hw, corr_out), main.cu:1529-1552
 * (CorrBlock::sample_single, corr.cuh:234): lookup of the last built volume. */
int slk_corr_sample(slk_ctx* ctx, const float* coords, float* out,
                    hipStream_t stream);

/* Device pointer and shape of single-edge level l ([h*w][h2][w2]); the
 * reference exposes these as corr_volume / corr_pyramid[l] (main.cu:1324-1326)
 * for its debug dump (main.cu:2859-2871). */
int slk_corr_level(slk_ctx* ctx, int level, const float** ptr, int* h2, int* w2);

/* Standalone kernels with the reference's argument lists: */
/* avg_pool_2x2_kernel(in, out, N, H, W), main.cu:1150-1170 */
int slk_avg_pool_2x2(const float* in, float* out, long N, int H, int W,
                     hipStream_t stream);
/* batch_corr_sample_kernel(volumes, coords, corr_out, M, r, H1, W1, H2, W2, hw,
 * coord_scale, level_idx), main.cu:1175-1217: writes channels
 * level_idx*49 .. +48 of corr_out (overwrite; the reference adds into a
 * zeroed buffer). r must be 3. */
int slk_corr_sample_level(const float* volumes, const float* coords, float* corr_out,
                          int M, int r, int H1, int W1, int H2, int W2, int hw,
                          float coord_scale, int level_idx, hipStream_t stream);
/* batch_coords_hw2_to_2hw(hw2, chw, M, HW), main.cu:1135-1146 */
int slk_coords_hw2_to_2hw(const float* hw2, float* chw, int M, int HW,
                          hipStream_t stream);

/* -------------------------------------------------------------------- SE3 */

/* projmap_kernel(poses, disps, intrinsics, ii, jj, coords, valid, M, H, W),
 * cuda_slam/se3.cuh:118-177: coords [M][H][W][2], valid [M][H][W]. */
int slk_projmap(const float* poses, const float* disps, const float* intrinsics,
                const int* ii, const int* jj, float* coords, float* valid, int M,
                int H, int W, hipStream_t stream);
/* pose_retr_kernel(poses, dx, t0, t1), se3.cuh:179-193 */
int slk_pose_retr(float* poses, const float* dx, int t0, int t1, hipStream_t stream);
/* disp_retr_kernel(disps, dz, inds, HW) over num_inds rows, se3.cuh:195-206 */
int slk_disp_retr(float* disps, const float* dz, const int* inds, int num_inds,
                  int HW, hipStream_t stream);
/* frame_distance_kernel(poses, disps, intrinsics, ii, jj, dist, M, H, W, beta),
 * se3.cuh:209-277 */
int slk_frame_distance(const float* poses, const float* disps,
                       const float* intrinsics, const int* ii, const int* jj,
                       float* dist, int M, int H, int W, float beta,
                       hipStream_t stream);
/* clamp_disps_kernel(disps, n, min_val), main.cu (caller :2392-2397) */
int slk_clamp_disps(float* disps, int n, float min_val, hipStream_t stream);

/* --------------------------------------------------------------------- BA */

/* BundleAdjustment::iterate(poses, disps, intrinsics, target, weight, eta,
 * ii_gpu, jj_gpu, ii_host, jj_host, num_edges, t0, t1, lm, ep, motion_only),
 * cuda_slam/ba.cuh:476-803; with motion_only=1 also the pipeline variant
 * slam::BundleAdjustment::iterate (cuda_pipeline/slam.cuh:1475-1592).
 * One Gauss-Newton step: linearization, Schur complement over the depths of
 * the keyframes in ii (unless motion_only), LM damping S_ii += ep + lm*S_ii,
 * fp64 Cholesky on the GPU, pose retraction of [t0,t1), depth
 * back-substitution. Stream-ordered and asynchronous (the reference is
 * synchronous); the index structures built from ii_host/jj_host are cached
 * while the edge set is unchanged. An indefinite system leaves poses/disps
 * untouched and is reported by slk_ba_status(). */
int slk_ba_iterate(slk_ctx* ctx, float* poses, float* disps, const float* intrinsics,
                   const float* target, const float* weight, const float* eta,
                   const int* ii_gpu, const int* jj_gpu, const int* ii_host,
                   const int* jj_host, int num_edges, int t0, int t1, float lm,
                   float ep, int motion_only, hipStream_t stream);

/* `iters` iterations of slk_ba_iterate on the same edge set: the loop of
 * run_update_pass over BundleAdjustment::iterate (cuda_slam/main.cu:2371-2389,
 * cuda_pipeline/slam.cuh:3178-3186). Same results as `iters` calls; a window
 * whose keyframes each have at most 7 E rows (own pose + other free poses)
 * runs each iteration as linearization with Schur partials, assembly and
 * solve, with the back-substitution of one step folded into the next
 * linearization. */
int slk_ba_iterate_n(slk_ctx* ctx, float* poses, float* disps, const float* intrinsics,
                     const float* target, const float* weight, const float* eta,
                     const int* ii_gpu, const int* jj_gpu, const int* ii_host,
                     const int* jj_host, int num_edges, int t0, int t1, float lm,
                     float ep, int motion_only, int iters, hipStream_t stream);

/* Synchronises `stream` and returns SLK_E_NOT_SPD if any iterate since the
 * last call met an indefinite system, SLK_E_HIP if a workgroup of an
 * overlapped fused step stopped waiting for its solve (see
 * slk_ba_set_wait_limit), else SLK_OK; clears the flags.
 * After SLK_E_HIP the state is not a whole number of steps: the poses hold
 * every step solved up to and including the one whose wait gave up, the
 * inverse depths of the pixel chunks that stopped waiting miss that step's
 * update (the other chunks have it), and every later step of that call
 * changed neither. Restore poses and disps from a copy before iterating on. */
int slk_ba_status(slk_ctx* ctx, hipStream_t stream);

/* No counterpart in the reference: the bound of the wait inside an
 * overlapped fused BA step launch (slk_ba_iterate_n), where the linearization
 * workgroups wait for the solve of the same launch. After `polls` polls (at
 * once for polls = 0) a waiting workgroup gives up: its pixel chunk skips
 * that step's depth update and the next linearization, the call's later
 * steps take no step at all, and the next slk_ba_status reports SLK_E_HIP
 * (the state left behind is described there); polls < 0 restores the
 * default (2^18, far above the ~40 a step takes). A diagnostic, used by the
 * tests to run the give-up path; production callers leave the default. */
int slk_ba_set_wait_limit(slk_ctx* ctx, int polls);

/* Debug copy of the last iterate's system (synchronising): S_host [(6P)^2]
 * after Schur + damping, b_host [6P], dx_host [6P]; any may be NULL. *n gets
 * 6P. Replaces the reference's stale S/b dumps read by
 * compare_ba_hessian.py:215-221. */
int slk_ba_last_system(slk_ctx* ctx, double* S_host, double* b_host, double* dx_host,
                       int* n, hipStream_t stream);

/* Stage kernels with the reference's argument lists (fp64 arithmetic inside,
 * fp32 storage as in the reference): */
/* projective_transform_kernel, ba.cuh:39-221: Hs [4][M][36], vs [2][M][6],
 * Eii/Eij [M][6][H*W], Cii/bz [M][H*W] */
int slk_ba_projective_transform(const float* target, const float* weight,
                                const float* poses, const float* disps,
                                const float* intrinsics, const int* ii, const int* jj,
                                float* Hs, float* vs, float* Eii, float* Eij,
                                float* Cii, float* bz, int M, int H, int W,
                                hipStream_t stream);
/* accum_kernel / accum_add_kernel(inps, ptrs, idxs, outs, D) over N_out rows,
 * ba.cuh:226-263 (add != 0 selects accum_add) */
int slk_ba_accum(const float* inps, const int* ptrs, const int* idxs, float* outs,
                 int N_out, int D, int add, hipStream_t stream);
/* damping_Q_kernel(C, eta, kf_map, Q, N_kf, HW, ep), ba.cuh:266-281 */
int slk_ba_damping_q(float* C, const float* eta, const int* kf_map, float* Q,
                     int N_kf, int HW, float ep, hipStream_t stream);
/* EEt6x6_kernel(E, Q, idx, S, D, N_pairs), ba.cuh:303-342 */
int slk_ba_eet6x6(const float* E, const float* Q, const int* idx, float* S, int D,
                  int N_pairs, hipStream_t stream);
/* Ev6x1_kernel(E, Q, w, idx, v, D, N_v), ba.cuh:346-372 (v += ...) */
int slk_ba_ev6x1(const float* E, const float* Q, const float* w, const int* idx,
                 float* v, int D, int N_v, hipStream_t stream);
/* EvT6x1_kernel(E, x, idx, w, D, N_E, P), ba.cuh:376-393 */
int slk_ba_evt6x1(const float* E, const float* x, const int* idx, float* w, int D,
                  int N_E, int P, hipStream_t stream);
/* depth_update_kernel(Q, w, dw, disps, kf_map, N_kf, HW), ba.cuh:284-299 */
int slk_ba_depth_update(const float* Q, const float* w, const float* dw, float* disps,
                        const int* kf_map, int N_kf, int HW, hipStream_t stream);

/* ------------------------------------------------------ update-pass glue */
/* The steps of CudaDroid::run_update_pass around correlation and BA
 * (cuda_slam/main.cu:2186-2400, cuda_pipeline/slam.cuh:3090-3170). Rows are
 * `row` consecutive floats; index arrays without `_host` are on the device. */

/* compute_motion_kernel(motion, coords1, coords0, target, batch, HW),
 * main.cu:1250-1273: motion [batch][4][h*w] = clamp(coords1 - coords0,
 * target - coords1 to [-64, 64]). coords0 == NULL takes the identity grid
 * that alloc_coords0 (main.cu:2150-2163) uploads, without reading it. */
int slk_compute_motion(float* motion, const float* coords1, const float* coords0,
                       const float* target, int batch, int h, int w, hipStream_t stream);
/* alloc_coords0 (main.cu:2150-2163) written on the device: coords0
 * [batch][2][h*w], x = column, y = row. */
int slk_fill_coords0(float* coords0, int batch, int h, int w, hipStream_t stream);
/* compute_target_kernel(target, weight_out, coords, delta, wt_raw, num_edges,
 * HW), main.cu:1282-1301: delta and wt_raw are [num_edges][3][hw]. */
int slk_compute_target(float* target, float* weight_out, const float* coords,
                       const float* delta, const float* wt_raw, int num_edges, int hw,
                       hipStream_t stream);
/* dst row e = src row idx[e] (idx == NULL: row e), e < n <= 65535: one launch
 * for the per-edge cudaMemcpy loops that load hidden states and inps
 * (main.cu:2216-2224: batch_nets from edge_nets + bs, idx NULL; batch_inps
 * from inps with idx = ii + bs). */
int slk_gather_rows(float* dst, const float* src, const int* idx, int n, long row,
                    hipStream_t stream);
/* dst row idx[e] = src row e (idx == NULL: row e), idx entries distinct: the
 * loops that save hidden states and conv1 features (main.cu:2245-2252) and
 * eta of the active keyframes (main.cu:2303-2309, idx = the active list of
 * slk_scatter_mean). */
int slk_scatter_rows(float* dst, const float* src, const int* idx, int n, long row,
                     hipStream_t stream);
/* GraphAgg scatter_mean, main.cu:2258-2296: the active keyframes are the
 * distinct ii_host values ascending (num_active_host of them, optionally
 * written to active_kf on the device and to active_kf_host); dst row a is the
 * sum of src rows e with ii_host[e] == active[a], taken in edge order from
 * zero, then, for more than one row, S + (1/count - 1) * S as one fused
 * multiply-add (scale_add_kernel under --use_fast_math). Bitwise equal to the
 * reference's sequence. n <= 65535. */
int slk_scatter_mean(slk_ctx* ctx, float* dst, const float* src, const int* ii_host, int n,
                     long row, int* active_kf, int* active_kf_host, int* num_active_host,
                     hipStream_t stream);
/* The BA edge set of run_update_pass, main.cu:2312-2390: t0 = forced_t0 if
 * >= 0, else max(1, min(ii_host) + 1) (num_keyframes + 1 without edges);
 * the active edges, followed, when use_inactive and n_inac > 0, by the
 * inactive edges with ii >= t0 - 3 and jj >= t0 - 3 in their order. Writes
 * the indices to ba_ii_host/ba_jj_host (capacity n + n_inac) and ba_ii/ba_jj,
 * the target and weight rows [count][2][hw] to ba_target/ba_weight (one
 * launch), *count and *t0. The BA then runs on (ba_*, count, t0,
 * num_keyframes) as in the reference. */
int slk_ba_edge_set(slk_ctx* ctx, const int* ii_host, const int* jj_host, int n,
                    const int* ii_inac_host, const int* jj_inac_host, int n_inac,
                    const float* target, const float* weight, const float* target_inac,
                    const float* weight_inac, int hw, int num_keyframes, int forced_t0,
                    int use_inactive, int* ba_ii_host, int* ba_jj_host, int* ba_ii,
                    int* ba_jj, float* ba_target, float* ba_weight, int* count, int* t0,
                    hipStream_t stream);

/* ----------------------------------------------------------- factor graph */
/* CudaDroid::add_proximity_factors(t0, t1, rad, nms, thresh, remove_old)
 * (cuda_slam/main.cu:1679-1779) up to the edge-state update, with the
 * frame distances of compute_frame_distances_batch (main.cu:1655-1676) in
 * one launch and one read-back for all pairs i in [t0, t), j in [t1, t)
 * (t = num_keyframes; poses/disps/intrinsics on the device, the context's
 * h x w maps). The existing edges are the active (ii_host/jj_host) and
 * inactive (ii_inac_host/jj_inac_host) lists. Writes the edges the update
 * appends (main.cu:1773-1781: the chosen edges not present yet, each once,
 * in the reference's order) to new_ii_host/new_jj_host (capacity
 * `capacity`; 2*(t - t0)*(t - t1 + rad + 1) always suffices), their number
 * to *n_new and the greedy step's edge count (es.size(), which the caller's
 * age-based removal compares with max_factors, main.cu:1758-1771) to *n_es;
 * dists_host, if not NULL, receives the (t - t0)*(t - t1) raw distances.
 * Equal distances are taken in pair order (the reference's std::sort leaves
 * their order unspecified). Synchronises `stream` once. */
int slk_proximity_factors(slk_ctx* ctx, const float* poses, const float* disps,
                          const float* intrinsics, int num_keyframes, int t0, int t1, int rad,
                          int nms, float thresh, float beta, const int* ii_host,
                          const int* jj_host, int n_edges, const int* ii_inac_host,
                          const int* jj_inac_host, int n_inac, int max_factors,
                          int* new_ii_host, int* new_jj_host, int capacity, int* n_new,
                          int* n_es, float* dists_host, hipStream_t stream);

/* The edge-state update that follows the selection (main.cu:1757-1796).
 * slk_oldest_edges_mask: mask_host[e] = 1 for the to_remove oldest active
 * edges (largest age first; equal ages in edge order, where the reference's
 * std::sort leaves them unspecified), the selection of add_proximity_factors'
 * step 5 (main.cu:1758-1770). Host only. */
void slk_oldest_edges_mask(const int* age_host, int n, int to_remove, unsigned char* mask_host);
/* CudaDroid::store_and_remove_edges (main.cu:795-836): each masked edge,
 * while the inactive list holds fewer than max_inac, is appended to it
 * (ii_inac_host/jj_inac_host at *num_inac, its target and weight rows copied
 * to target_inac/weight_inac); masked edges beyond that are dropped. Kept
 * edges close up in order: ii_host/jj_host/age_host (age may be NULL) are
 * compacted in place, and so are their rows of edge_nets (net_row floats,
 * 128*h*w in the reference), target and weight (tw_row floats, 2*h*w).
 * *num_inac and *n_kept are updated. The reference issues a cudaMemcpy per
 * row; here each array's rows move in one gather and one scatter launch
 * through a staging buffer (a destination row can be the source of an
 * earlier move). */
int slk_store_and_remove_edges(slk_ctx* ctx, const unsigned char* mask_host, int n,
                               int* ii_host, int* jj_host, int* age_host, int* ii_inac_host,
                               int* jj_inac_host, int* num_inac, int max_inac, float* edge_nets,
                               long net_row, float* target, float* weight, float* target_inac,
                               float* weight_inac, long tw_row, int* n_kept,
                               hipStream_t stream);
/* Hidden states of newly added edges (main.cu:1786-1796): edge_nets row e =
 * nets row ii_host[e] and weight row e = 0 for e in [first, first + count). */
int slk_init_new_edges(slk_ctx* ctx, const float* nets, float* edge_nets, float* weight,
                       const int* ii_host, int first, int count, long net_row, long tw_row,
                       hipStream_t stream);
/* CudaDroid::rm_keyframe(ix) (main.cu:866-941), for 0 <= ix < num_keyframes
 * (otherwise nothing changes): keyframe rows ix+1 .. t-1 of poses (7 floats),
 * disps (h*w), fmaps (C*h*w of fmap_dtype), nets and inps (net_row floats)
 * move down by one; active edges touching ix are removed, indices above ix
 * drop by one, and the others close up in order (ii/jj/age host lists in
 * place, *n_kept) with their rows of edge_nets (net_row), target and weight
 * (2*h*w); the inactive edges likewise (*n_inac_kept) with target_inac and
 * weight_inac. A null array pointer skips that array. Every array's rows move
 * in one gather and one scatter launch in place of the reference's per-row
 * copies; the caller drops its own timestamp and decrements num_keyframes. */
int slk_rm_keyframe(slk_ctx* ctx, int ix, int num_keyframes, float* poses, float* disps,
                    void* fmaps, int fmap_dtype, float* nets, float* inps, long net_row,
                    int* ii_host, int* jj_host, int* age_host, int n, int* n_kept,
                    int* ii_inac_host, int* jj_inac_host, int n_inac, int* n_inac_kept,
                    float* edge_nets, float* target, float* weight, float* target_inac,
                    float* weight_inac, hipStream_t stream);

/* -------------------------------------------------------- update operator */
/* UpdateModule with its ConvGRU (cuda_slam/main.cu:385-667): the network that
 * turns the 196-channel correlation lookup into delta / weight for the BA,
 * the new hidden state and the GraphAgg features. Tensors are NCHW fp32 like
 * the reference's buffers; the convolutions run as fp16-operand MFMA GEMMs
 * with fp32 accumulation (the reference's tensor-op convolutions of fp32
 * data, nn.cuh:146, round the operands to the same 10-bit mantissa), and
 * every activation the reference rounds to fp16 is rounded where it does. */
typedef struct slk_update slk_update;

/* UpdateModule::init (main.cu:552-603) for batches of up to max_batch edges
 * of h x w maps: allocates the activations. Weights are set separately. */
int slk_update_create(slk_update** um, int max_batch, int h, int w);
int slk_update_destroy(slk_update* um);

/* The 18 convolutions the forward pass uses, in a fixed order: layer i has
 * the reference's weight-file name (update_corr_encoder_0, ...;
 * WeightStore::load_conv, main.cu:81-86) and shape [co][ci][k][k]. */
int slk_update_num_layers(void);
const char* slk_update_layer_name(int layer);
int slk_update_layer_shape(int layer, int* co, int* ci, int* k);

/* Weights of one layer as host fp32 arrays in the reference's layout
 * (weight [co][ci][k][k], bias [co]; ConvLayer::init, nn.cuh:124-139). They
 * are repacked for the GPU before the next forward. */
int slk_update_set_conv(slk_update* um, int layer, const float* weight_host,
                        const float* bias_host);

/* Every layer from the reference's exported tensor files
 * <dir>/<name>_weight.bin and <name>_bias.bin (int32 ndim, int32 dims,
 * float32 data; export_weights.py:14-22, load_tensor nn.cuh:91-107). */
int slk_update_load_dir(slk_update* um, const char* dir);

/* UpdateModule::forward(corr_features, motion, net, inp, delta_out,
 * weight_out, agg_conv1_out, ..., batch, h, w), main.cu:606-650: corr
 * [B][196][hw], motion [B][4][hw], net [B][128][hw] (updated in place: the
 * GRU state, fp16-valued), inp [B][128][hw] -> delta_out [B][3][hw],
 * weight_out [B][3][hw], agg_conv1_out [B][128][hw]. B <= max_batch.
 * The flow encoder and the gate run on two streams of the module, forked
 * from `stream` and joined back to it within the call; the outputs are
 * ordered on `stream` as usual. Calls on one module must not overlap on
 * different caller streams (they share the module's buffers). */
int slk_update_forward(slk_update* um, const float* corr, const float* motion, float* net,
                       const float* inp, float* delta_out, float* weight_out,
                       float* agg_conv1_out, int batch, hipStream_t stream);

/* UpdateModule::compute_eta(agg_features, eta_out, ..., num_kf, h, w),
 * main.cu:654-667: agg_features [K][128][hw] (rounded to fp16 in place, as
 * the reference does) -> eta_out [K][hw] = 0.01 * softplus(eta conv). */
int slk_update_compute_eta(slk_update* um, float* agg_features, float* eta_out, int num_kf,
                           hipStream_t stream);

/* CudaDroid::compute_motion_gru(last_kf_idx), main.cu:1934-1983: the
 * frontend's motion filter. Builds the single-edge correlation of
 * (f_last, f_cur) in ctx (as build_correlation(last_kf, temp_slot)), samples
 * it at the identity grid, runs one update step (batch 1, zero motion) from
 * copies of the keyframe's hidden state net_kf and context inp_kf (both
 * [128][h*w], left unchanged), and writes the mean over pixels of the
 * magnitude of delta's flow channels to *mean_flow (summed on the host in
 * pixel order, like the reference). ctx and um must have the same h, w and
 * ctx 4 levels. Synchronises `stream`. */
int slk_motion_filter(slk_ctx* ctx, slk_update* um, const void* f_last, const void* f_cur,
                      int dtype, const float* net_kf, const float* inp_kf, float* mean_flow,
                      hipStream_t stream);

/* ------------------------------------------------------------- encoders */
/* HalfBasicEncoder (cuda_slam/main.cu:306-381) with its HalfResBlocks
 * (:236-303): the fp16 feature (fnet: output_dim 128, instance norm) and
 * context (cnet: 256, no norm) networks of DROID-SLAM. conv1 7x7 stride 2,
 * three stages of two residual blocks (32, 64 stride 2, 128 stride 2), conv2
 * 1x1: [3][H][W] -> [output_dim][H/8][W/8]. Every convolution is an fp16
 * MFMA GEMM with fp32 accumulation; outputs are rounded to fp16 before and
 * after the fp32 bias as the reference's cuDNN call + bias_add_half_kernel
 * do (nn.cuh:657-791), and instance norm (nn.cuh:609-654) has eps 1e-5. */
typedef struct slk_encoder slk_encoder;

/* HalfBasicEncoder::init(cudnn, ws, prefix, batch, inH, inW, out_dim,
 * use_norm), main.cu:316-353, without the weights (set separately).
 * in_h, in_w multiples of 8; out_dim a multiple of 16, at most 256. */
int slk_encoder_create(slk_encoder** enc, int in_h, int in_w, int out_dim, int use_norm,
                       int max_batch);
int slk_encoder_destroy(slk_encoder* enc);

/* The 16 convolutions in a fixed order; layer i's weight files are
 * <prefix>_<suffix>_weight.bin / _bias.bin (conv1, layer1_0_conv1, ...,
 * layer2_0_downsample_0, ..., conv2; WeightStore::load_conv, main.cu:81-86). */
int slk_encoder_num_layers(void);
const char* slk_encoder_layer_suffix(int layer);
int slk_encoder_layer_shape(const slk_encoder* enc, int layer, int* co, int* ci, int* k,
                            int* stride);

/* Weights of one layer as host fp32 arrays (weight [co][ci][k][k], bias
 * [co]); rounded to fp16 and repacked before the next forward
 * (HalfConvLayer::init converts them with float_to_half, nn.cuh:683-690). */
int slk_encoder_set_conv(slk_encoder* enc, int layer, const float* weight_host,
                         const float* bias_host);
int slk_encoder_load_dir(slk_encoder* enc, const char* dir, const char* prefix);

/* HalfBasicEncoder::forward(cudnn, input, output, ...), main.cu:357-380:
 * input [B][3][H][W] fp32 (converted to fp16 like float_to_half) ->
 * output [B][out_dim][H/8][W/8] fp16. 1 <= B <= max_batch. */
int slk_encoder_forward(slk_encoder* enc, const float* input, void* output_f16, int batch,
                        hipStream_t stream);

/* CudaDroid::encode_frame(bgr_hwc), main.cu:1465-1497: preprocess the BGR
 * frame [H][W][3] (0..255; preprocess_image_kernel, main.cu:1062-1075), run
 * fnet -> fmap [128][H/8][W/8] fp16 and cnet -> net = tanh(cmap[0:128]),
 * inp = relu(cmap[128:256]) as fp32 [128][H/8][W/8]. fnet must have out_dim
 * 128, cnet 256, both max_batch >= 1 and the same image size. cnet runs on a
 * stream of the cnet object (created on the first call) forked from `stream`
 * and joined back to it by events, so the outputs are ordered on `stream`
 * as if both encoders had run there; calls that share a cnet object must not
 * overlap. */
int slk_encode_frame(slk_encoder* fnet, slk_encoder* cnet, const float* bgr_hwc, void* fmap_f16,
                     float* net, float* inp, hipStream_t stream);

/* ------------------------------------------------------ front of the pipe */
/* nv12_to_bgr_resize_kernel, main.cu:947-985: an NV12 frame (Y plane and
 * interleaved half-resolution UV plane, strides in bytes) -> float BGR
 * [dst_h][dst_w][3] in 0..255, bilinear Y, nearest UV, BT.709. */
int slk_nv12_to_bgr(const uint8_t* y_plane, const uint8_t* uv_plane, float* bgr_out, int src_w,
                    int src_h, int y_stride, int uv_stride, int dst_w, int dst_h,
                    hipStream_t stream);
/* p010_to_bgr_resize_kernel, main.cu:988-1027: the same from P010 (10 bits
 * in the top of each 16-bit sample, scaled to the 8-bit range); strides in
 * bytes. */
int slk_p010_to_bgr(const uint16_t* y_plane, const uint16_t* uv_plane, float* bgr_out, int src_w,
                    int src_h, int y_stride_bytes, int uv_stride_bytes, int dst_w, int dst_h,
                    hipStream_t stream);
/* bgr8_to_bgrf_resize_kernel, main.cu:1030-1058: 8-bit BGR (row stride in
 * bytes) -> float BGR with bilinear resize. */
int slk_bgr8_to_bgrf(const uint8_t* bgr_in, float* bgr_out, int src_w, int src_h, int src_stride,
                     int dst_w, int dst_h, hipStream_t stream);
/* preprocess_image_kernel, main.cu:1062-1075: BGR HWC (0..255) -> RGB NCHW,
 * (x/255 - mean) / std with the ImageNet mean and std. */
int slk_preprocess_image(const float* bgr_hwc, float* rgb_nchw, int H, int W, hipStream_t stream);

/* The pose file of main.cu:2924-2937 ([num_keyframes: i32]
 * [timestamps: i32 x nk] [poses: f32 x nk x 7]); with cam_to_world the
 * world->camera poses are inverted first in the reference's float
 * arithmetic (main.cu:2896-2914). poses are host memory. */
int slk_write_poses_bin(const char* path, int num_keyframes, const int* timestamps,
                        const float* poses, int cam_to_world);

#ifdef __cplusplus
}
#endif

#endif /* SLK_H */
