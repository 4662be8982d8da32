/*
 * oracle.h -- CPU restatement of the DROID-SLAM per-edge update path of
 * vibekernels/slam-hands (cuda_slam), used ONLY as a test checker.
 *
 * TEST INFRASTRUCTURE. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library. The product library
 * (slam-hands_amd/, libslk.so) never links or calls it.
 *
 * Arithmetic: inputs and outputs are fp32 like the reference; every sum and
 * product inside is carried in fp64 (the reference accumulates in fp32 on the
 * GPU and solves in fp64 on the host, cuda_slam/ba.cuh:416-445).
 *
 * Each function cites the reference file:line it restates. How each one is
 * pinned (closed forms, finite differences, brute-force solves, scipy) is
 * listed in tests/test_oracle_*.py.
 */
#ifndef SLK_ORACLE_H
#define SLK_ORACLE_H

#ifdef __cplusplus
extern "C" {
#endif

/* OpenMP threads the oracle's parallel loops use. */
int orc_num_threads(void);

/* ---------------- correlation (cuda_slam/main.cu:1077-1217, 1500-1613) ---- */

/* vol[p][q] = alpha * sum_c fi[c][p] * fj[c][q]; fi, fj are [C][HW]
 * (main.cu:1508-1515: cublasGemmEx(N,T,hw,hw,128, alpha=1/16, A=f_j, B=f_i)). */
void orc_corr_volume(const float* fi, const float* fj, int C, int HW,
                     double alpha, float* vol);

/* Same, with fmaps given as IEEE binary16 bit patterns (DroidState::fmaps is a
 * GpuHalfBuf, main.cu:677). */
void orc_corr_volume_f16(const unsigned short* fi, const unsigned short* fj,
                         int C, int HW, double alpha, float* vol);

/* out[n][oy][ox] = 0.25f*(in[2oy][2ox]+in[2oy][2ox+1]+in[2oy+1][2ox]+in[2oy+1][2ox+1]),
 * oH = H/2, oW = W/2 (floor); fp32, left-to-right, as main.cu:1150-1170. */
void orc_avg_pool_2x2(const float* in, float* out, long N, int H, int W);

/* Radius-r bilinear lookup of one pyramid level for one edge
 * (main.cu:1175-1217 batch_corr_sample_kernel, single-edge main.cu:1079-1114).
 * level: [HW1][H2][W2]; coords: [2][HW1] (x plane then y plane);
 * out: [levels*D*D][HW1]; writes channels level_idx*D*D .. +D*D-1.
 * Channel (a,b) = a*D+b with a the x offset, b the y offset. Corners outside
 * [0,W2)x[0,H2) contribute nothing; a non-finite coordinate contributes
 * nothing to any channel. */
void orc_corr_lookup_level(const float* level, const float* coords, float* out,
                           int r, int H1, int W1, int H2, int W2,
                           float coord_scale, int level_idx);

/* Full batched path (main.cu:1555-1613): for each edge e, volume of
 * (fmaps[ii[e]], fmaps[jj[e]]), pyramid of `levels` levels, lookup of radius r
 * at coords[e] ([B][2][HW]) into out[e] ([B][levels*(2r+1)^2][HW]).
 * fmaps: [nframes][C][h][w] fp32. */
void orc_corr_batch(const float* fmaps, int C, int h, int w,
                    const int* ii, const int* jj, int B,
                    const float* coords, float* out,
                    int levels, int r, double alpha);

/* ---------------- SE3 (cuda_slam/se3.cuh:8-114) --------------------------- */
/* Pose = [tx,ty,tz,qx,qy,qz,qw]; tangent xi = [tau(3), phi(3)]. */
void orc_act_se3(const double* t, const double* q, const double* X, double* Y);
void orc_adj_se3(const double* t, const double* q, const double* X, double* Y);
void orc_rel_se3(const double* ti, const double* qi, const double* tj,
                 const double* qj, double* tij, double* qij);
void orc_exp_se3(const double* xi, double* t, double* q);
void orc_retr_se3(const double* xi, const double* t, const double* q,
                  double* t1, double* q1);

/* projmap_kernel (se3.cuh:118-177): coords [M][H][W][2], valid [M][H][W]. */
void orc_projmap(const float* poses, const float* disps, const float* intr,
                 const int* ii, const int* jj, float* coords, float* valid,
                 int M, int H, int W);

/* pose_retr_kernel (se3.cuh:179-193). */
void orc_pose_retr(float* poses, const float* dx, int t0, int t1);

/* disp_retr_kernel (se3.cuh:195-206). */
void orc_disp_retr(float* disps, const float* dz, const int* inds, int num_inds,
                   int HW);

/* frame_distance_kernel (se3.cuh:209-277). */
void orc_frame_distance(const float* poses, const float* disps, const float* intr,
                        const int* ii, const int* jj, float* dist,
                        int M, int H, int W, float beta);

/* ---------------- bundle adjustment (cuda_slam/ba.cuh) -------------------- */

/* projective_transform_kernel (ba.cuh:39-221), fp64 inside.
 * Hs [4][M][36], vs [2][M][6], Eii/Eij [M][6][HW], Cii/bz [M][HW]. */
void orc_ba_linearize(const float* target, const float* weight,
                      const float* poses, const float* disps, const float* intr,
                      const int* ii, const int* jj,
                      double* Hs, double* vs, double* Eii, double* Eij,
                      double* Cii, double* bz, int M, int H, int W);

/* One BundleAdjustment::iterate (ba.cuh:476-803), fp64 inside.
 * Updates poses [nframes][7] for k in [t0,t1) and, unless motion_only,
 * disps [nframes][HW] of every keyframe in ii. eta: [nframes][HW].
 * Debug outputs (any may be NULL): S_out [(6P)^2] (after Schur + LM damping,
 * before factorisation), b_out [6P], dx_out [6P], dz_out [nframes][HW]
 * (zero where untouched).
 * Returns 0, or 3 when S is not positive definite (poses/disps untouched). */
int orc_ba_iterate(float* poses, float* disps, const float* intr,
                   const float* target, const float* weight, const float* eta,
                   const int* ii, const int* jj, int M, int nframes,
                   int H, int W, int t0, int t1, float lm, float ep,
                   int motion_only,
                   double* S_out, double* b_out, double* dx_out, double* dz_out);

/* cholesky_solve_double (ba.cuh:416-445) on a dense SPD n x n system, fp64.
 * Returns 0, or 3 if a pivot is not positive. S is overwritten with L. */
int orc_cholesky_solve(double* S, double* b, int n);

/* ---------------- update-pass glue (cuda_slam/main.cu:1246-1301, 2186-2400) */

/* compute_motion_kernel (main.cu:1250-1273): motion [batch][4][h*w] =
 * clamp([coords1 - coords0, target - coords1], -64, 64) per plane; coords0
 * NULL is the identity grid of alloc_coords0 (main.cu:2150-2163). */
void orc_compute_motion(float* motion, const float* coords1, const float* coords0,
                        const float* target, int batch, int h, int w);

/* compute_target_kernel (main.cu:1282-1301): target = coords + delta[:, :2],
 * weight_out = wt_raw[:, :2]; delta and wt_raw are [n][3][hw]. */
void orc_compute_target(float* target, float* weight_out, const float* coords,
                        const float* delta, const float* wt_raw, int n, int hw);

/* The per-edge cudaMemcpy loops of run_update_pass (main.cu:2216-2224,
 * 2245-2252, 2305-2309): gather dst[e] = src[idx[e]], scatter dst[idx[e]] =
 * src[e]; idx NULL is the identity; rows of `row` floats. */
void orc_gather_rows(float* dst, const float* src, const int* idx, int n, long row);
void orc_scatter_rows(float* dst, const float* src, const int* idx, int n, long row);

/* GraphAgg scatter_mean (main.cu:2258-2296): active = ascending distinct ii
 * (capacity n); dst row a = rows e with ii[e] == active[a] summed in edge
 * order from zero (scale_add_kernel with scale 1, nn.cuh:382-385), then for a
 * count above one dst = fma(1/count - 1, dst, dst) (scale_add_kernel with
 * src == dst, built with --use_fast_math, so a fused multiply-add).
 * Returns the number of active keyframes. */
int orc_scatter_mean(float* dst, const float* src, const int* ii, int n, long row,
                     int* active);

/* BA edge set of run_update_pass (main.cu:2312-2390): t0 = forced_t0 if
 * >= 0, else max(1, min(ii) + 1); with use_inactive and n_inac > 0 the edges
 * are the active ones followed by the inactive ones with ii >= t0 - 3 and
 * jj >= t0 - 3, in order, and their target/weight rows [2][hw]; otherwise
 * the active edges alone. Returns the edge count; *t0_out = t0. */
int orc_ba_edge_set(const int* ii, const int* jj, int n, const int* ii_inac,
                    const int* jj_inac, int n_inac, const float* target,
                    const float* weight, const float* target_inac,
                    const float* weight_inac, int hw, int num_keyframes, int forced_t0,
                    int use_inactive, int* ba_ii, int* ba_jj, float* ba_target,
                    float* ba_weight, int* t0_out);

/* ---------------- factor graph (cuda_slam/main.cu:1655-1781) ------------- */

/* add_proximity_factors (main.cu:1679-1779) from the raw frame distances of
 * the pairs i in [t0, t), j in [t1, t) (d[(i-t0)*(t-t1) + j-t1], t =
 * num_keyframes): invalidation, NMS around the active and inactive edges,
 * mandatory neighbour edges, greedy best-distance edges (ascending distance,
 * ties in pair order), then the edges not present yet, each once, written
 * to new_ii/new_jj (up to cap). Returns the number of edges the greedy step
 * produced (both directions counted), *n_new the number of new edges. */
int orc_proximity_select(const float* d, int t, int t0, int t1, int rad, int nms,
                         float thresh, const int* ii, const int* jj, int n,
                         const int* ii_inac, const int* jj_inac, int n_inac,
                         int max_factors, int* new_ii, int* new_jj, int cap, int* n_new);

/* factor-graph edge state: step 5's age selection, store_and_remove_edges
   and the new edges' hidden states (main.cu:795-836, 1757-1796) */
void orc_oldest_mask(const int* age, int n, int to_remove, unsigned char* mask);
int orc_store_and_remove_edges(const unsigned char* mask, int n, int* ii, int* jj, int* age,
                               int* ii_inac, int* jj_inac, int* num_inac, int max_inac,
                               float* nets, long net_row, float* target, float* weight,
                               float* target_inac, float* weight_inac, long tw_row);
void orc_init_new_edges(const float* nets, float* edge_nets, float* weight, const int* ii,
                        int first, int count, long net_row, long tw_row);
/* CudaDroid::rm_keyframe (main.cu:866-941) */
void orc_rm_keyframe(int ix, int t, float* poses, float* disps, float* fmaps, long fmap_row,
                     float* nets, float* inps, long net_row, long hw, int* ii, int* jj,
                     int* age, int n, int* n_kept, int* ii_inac, int* jj_inac, int n_inac,
                     int* n_inac_kept, float* edge_nets, float* target, float* weight,
                     float* target_inac, float* weight_inac);

#ifdef __cplusplus
}
#endif
#endif
