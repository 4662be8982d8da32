// Bundle adjustment for gfx950: linearization, Schur complement over the
// depths, fp64 Cholesky pose solve and depth back-substitution, entirely on
// the GPU with no host round trip inside an iteration.
//
// Reference semantics: cuda_slam/ba.cuh:39-803 (projective_transform_kernel,
// accum, damping_Q, EEt6x6, Ev6x1, EvT6x1, depth_update, and the host
// orchestration BundleAdjustment::iterate) with se3.cuh for the geometry.
//
// Iteration = 5 kernels on one stream:
//   k_ba_lin_*    grid (pixel chunk, keyframe): every edge whose depth owner
//                 (ii) is that keyframe is linearized for the chunk's pixels in
//                 fp64. Per edge and chunk only Hjj (21) and vj (6) are
//                 reduced, since Ji = -Adj(Tij) Jj gives Hii = Adj Hjj Adj^T,
//                 Hij = -Adj Hjj and vi = -Adj vj; the depth terms (C, w),
//                 Q = 1/(C + 0.2 eta + 1e-7) and the E rows of the keyframe
//                 are accumulated in place, so the per-edge Eii/Eij/Cii/bz
//                 arrays of the reference never exist.
//   k_ba_schur    one workgroup per item over all pixels: E_r1 Q E_r2^T for
//                 the upper pairs of E rows sharing a keyframe, E_r Q w per
//                 row; then one workgroup per edge sums its chunk partials and
//                 expands them to the four blocks with the edge's Adj.
//   k_ba_assemble one workgroup per 6x6 block of S and per 6 entries of b:
//                 sums the totals listed for the block (lists built on the
//                 host; fixed order, no atomics), then S_ii += ep + lm*S_ii.
//   k_ba_solve_*  fp64 factorization and solve, dx rounded to fp32,
//                 retraction of the poses [t0, t1): Cholesky in one
//                 wavefront with S in registers up to 10 free poses, LDL^T in
//                 one workgroup with S in LDS up to 120x120, else Cholesky
//                 blocked over many workgroups in global memory.
//   k_ba_backsub  grid (pixel chunk, keyframe): dz = Q (w - E^T dx),
//                 disps += dz.
// Host work per iteration is limited to comparing the edge list with the
// cached one; index structures are rebuilt and uploaded only when it changes.
#include <algorithm>
#include <cstring>
#include <map>
#include <utility>

#include "reduce.hpp"
#include "se3.hpp"
#include "slk_internal.hpp"

namespace slk {

namespace {

constexpr int kLinWG = 256;
constexpr int kLinPx = 256;  // pixels per linearization workgroup (<= kLinWG, a multiple of 64)
constexpr int kSchWG = 256;
constexpr int kNH = 90;      // 78 upper-triangle Hessian entries + vi(6) + vj(6)
// Per (edge, pixel chunk) the linearization reduces only Hjj = sum w Jj Jj^T
// (21 upper entries) and vj = sum w r Jj (6): Ji = -Adj(Tij) Jj per pixel
// (ba.cuh:139-140, 167-168) with one 6x6 matrix Adj per edge, so
// Hii = Adj Hjj Adj^T, Hij = -Adj Hjj, Hji = Hij^T and vi = -Adj vj follow
// from the edge totals.
constexpr int kNJ = 27;
// per-edge totals: Hii (36), Hij (36), Hjj (36), vi (6), vj (6)
constexpr int kNT = 120;
constexpr int kTotHii = 0, kTotHij = 36, kTotHjj = 72, kTotVi = 108, kTotVj = 114;
constexpr double kMinDepth = 0.25;  // se3.cuh:6

__host__ __device__ __forceinline__ int tri(int n, int m) { return n * (n + 1) / 2 + m; }

// Offsets of the packed int plan (device copy of the host-built index data).
struct PlanDev {
    const int* kf_list;   // [N_kf] absolute keyframe of compact kf
    const int* kf_eptr;   // [N_kf+1] edges of each kf (ii == kf), edge order
    const int* kf_eidx;   // [M]
    const int* edge_ri;   // [M] E row of (ii-t0, ii) or -1
    const int* edge_rj;   // [M] E row of (jj-t0, ii) or -1
    const int* row_pose;  // [N_E]
    const int* row_kf;    // [N_E] compact kf
    const int* kf_rptr;   // [N_kf+1]
    const int* kf_rows;   // [N_E]
    const int* pairs;     // [N_pu][3] = r1, r2, kc (r1 <= r2)
    const int* sblk;      // [n_blk] a*P + b
    const int* sblk_ptr;  // [n_blk+1]
    const int* sblk_src;  // contributions (see encode_*)
    const int* bv_ptr;    // [P+1]
    const int* bv_src;
    const int* blkmap;    // [P*P] block id of (a, b) in sblk, or -1
};
constexpr int kPlanParts = 16;

// contribution codes: type in bits 30..31
__host__ __device__ __forceinline__ int code(int type, int v) { return (type << 30) | v; }
__host__ __device__ __forceinline__ int code_type(int c) { return (int)((unsigned)c >> 30); }
__host__ __device__ __forceinline__ int code_val(int c) { return c & 0x3fffffff; }

struct Lin {
    double Jj[2][6], Jz[2], w[2], r[2];
};

// Per-pixel linearization of one edge (ba.cuh:104-189), fp64, without Ji
// (= -Adj Jj, applied per edge or per E row by the callers).
__device__ __forceinline__ void lin_pixel(const double* tij, const double* qij, double fx,
                                          double fy, double cx, double cy, int k, int W,
                                          double disp, double tgu, double tgv, double wtu,
                                          double wtv, Lin& L) {
    const int i = k / W, j = k - (k / W) * W;
    const double u = (double)j, v = (double)i;
    double Xi[4], Xj[4];
    Xi[0] = (u - cx) / fx;
    Xi[1] = (v - cy) / fy;
    Xi[2] = 1.0;
    Xi[3] = disp;
    act_se3(tij, qij, Xi, Xj);
    const double x = Xj[0], y = Xj[1], h = Xj[3];
    const bool bad = Xj[2] < kMinDepth;
    const double d = bad ? 0.0 : 1.0 / Xj[2];
    const double d2 = d * d;
    L.w[0] = bad ? 0.0 : 0.001 * wtu;
    L.w[1] = bad ? 0.0 : 0.001 * wtv;
    L.r[0] = tgu - (fx * d * x + cx);
    L.r[1] = tgv - (fy * d * y + cy);
    double* Jj = L.Jj[0];
    Jj[0] = fx * (h * d);
    Jj[1] = 0.0;
    Jj[2] = fx * (-x * h * d2);
    Jj[3] = fx * (-x * y * d2);
    Jj[4] = fx * (1.0 + x * x * d2);
    Jj[5] = fx * (-y * d);
    L.Jz[0] = fx * (tij[0] * d - tij[2] * (x * d2));
    Jj = L.Jj[1];
    Jj[0] = 0.0;
    Jj[1] = fy * (h * d);
    Jj[2] = fy * (-y * h * d2);
    Jj[3] = fy * (-1.0 - y * y * d2);
    Jj[4] = fy * (x * y * d2);
    Jj[5] = fy * (x * d);
    L.Jz[1] = fy * (tij[1] * d - tij[2] * (y * d2));
}

// acc[0..20] += weff Jj Jj^T (upper triangle), acc[21..26] += weff r Jj
__device__ __forceinline__ void accum_hjj(const Lin& L, bool stereo, double (&acc)[kNJ]) {
#pragma unroll
    for (int row = 0; row < 2; row++) {
        const double we = stereo ? 0.0 : L.w[row];
        const double* J = L.Jj[row];
#pragma unroll
        for (int n = 0; n < 6; n++) {
            const double wn = we * J[n];
#pragma unroll
            for (int m = 0; m <= n; m++) acc[tri(n, m)] += wn * J[m];
        }
        const double wr = we * L.r[row];
#pragma unroll
        for (int n = 0; n < 6; n++) acc[21 + n] += wr * J[n];
    }
}

__device__ __forceinline__ void edge_rel(const float* poses, int ix, int jx, double* tij,
                                         double* qij) {
    if (ix == jx) {  // stereo pair (ba.cuh:73-78)
        tij[0] = -0.1;
        tij[1] = 0.0;
        tij[2] = 0.0;
        qij[0] = 0.0;
        qij[1] = 0.0;
        qij[2] = 0.0;
        qij[3] = 1.0;
    } else {
        double ti[3], qi[4], tj[3], qj[4];
        load_pose(poses, ix, ti, qi);
        load_pose(poses, jx, tj, qj);
        rel_se3(ti, qi, tj, qj, tij, qij);
    }
}

// p[0] + p[stride] + ... + p[(n - 1) stride], added in that order, with the
// loads of sixteen terms in flight at a time (a plain loop waits for each).
template <int kB = 16>
__device__ __forceinline__ double sum_strided(const double* __restrict__ p, size_t stride, int n) {
    double t = 0.0;
    for (int c = 0; c < n; c += kB) {
        double v[kB];
#pragma unroll
        for (int u = 0; u < kB; u++) v[u] = c + u < n ? p[(size_t)(c + u) * stride] : 0.0;
#pragma unroll
        for (int u = 0; u < kB; u++) t += v[u];
    }
    return t;
}

// Totals of edge e over the nch pixel chunks (summed in chunk order),
// expanded to the four Hessian blocks and both gradients of ba.cuh:198-220
// with the edge's Adj: et[0..120) = Hii, Hij, Hjj, vi, vj. One wave; `sh`
// holds 27 + 36 + 36 doubles.
__device__ void edge_totals(int e, const float* __restrict__ poses, const int* __restrict__ ii,
                            const int* __restrict__ jj, const double* __restrict__ hpart,
                            double* __restrict__ et, int nch, double* sh) {
    const int lane = threadIdx.x & 63;
    double* tot = sh;
    double* adj = tot + kNJ;
    double* ah = adj + 36;
    if (lane < kNJ) tot[lane] = sum_strided(hpart + (size_t)e * nch * kNJ + lane, kNJ, nch);
    double tij[3], qij[4];
    edge_rel(poses, ii[e], jj[e], tij, qij);
    // Adj column by column, lane c < 6 forming column c: adj_se3 of the unit
    // vectors (se3.cuh:28-41)
    {
        double u[6], y[6];
#pragma unroll
        for (int m = 0; m < 6; m++) u[m] = m == lane ? 1.0 : 0.0;
        adj_se3(tij, qij, u, y);
        if (lane < 6)
#pragma unroll
            for (int r = 0; r < 6; r++) adj[r * 6 + lane] = y[r];
    }
    __builtin_amdgcn_wave_barrier();
    const int r = lane / 6, c = lane - (lane / 6) * 6;
    if (lane < 36) {
        double t = 0.0;  // (Adj Hjj)[r][c]
#pragma unroll
        for (int k = 0; k < 6; k++) t += adj[r * 6 + k] * tot[tri(max(k, c), min(k, c))];
        ah[lane] = t;
        et[kTotHij + lane] = -t;
        et[kTotHjj + lane] = tot[tri(max(r, c), min(r, c))];
    }
    __builtin_amdgcn_wave_barrier();
    if (lane < 36) {
        double t = 0.0;  // (Adj Hjj Adj^T)[r][c]
#pragma unroll
        for (int k = 0; k < 6; k++) t += ah[r * 6 + k] * adj[c * 6 + k];
        et[kTotHii + lane] = t;
    }
    if (lane < 6) {
        double t = 0.0;
#pragma unroll
        for (int k = 0; k < 6; k++) t += adj[lane * 6 + k] * tot[21 + k];
        et[kTotVi + lane] = -t;
        et[kTotVj + lane] = tot[21 + lane];
    }
}

// ------------------------------------------------------- k_ba_lin_kf ----
// Edge-serial linearization (a keyframe with two edges to one free pose):
// grid (pixel chunk, keyframe), the workgroup walks the keyframe's edges in
// order, accumulating E rows in place.
__global__ __launch_bounds__(kLinWG) void k_ba_lin_kf(
    PlanDev plan, const float* __restrict__ target, const float* __restrict__ weight,
    const float* __restrict__ poses, const float* __restrict__ disps,
    const float* __restrict__ intr, const int* __restrict__ ii, const int* __restrict__ jj,
    const float* __restrict__ eta, double* __restrict__ hpart, double* __restrict__ E,
    double* __restrict__ Qo, double* __restrict__ Wo, int HW, int W, int nch, int motion_only) {
    __shared__ double red[kNJ * (kLinWG / 64)];
    __shared__ double rel[7];
    const int chunk = blockIdx.x;
    const int kc = blockIdx.y;
    const int kf = plan.kf_list[kc];
    const double fx = intr[0], fy = intr[1], cx = intr[2], cy = intr[3];
    const int k = chunk * kLinPx + threadIdx.x;
    const bool vpx = (int)threadIdx.x < kLinPx && k < HW;  // threads past the chunk idle
    const int r0 = plan.kf_rptr[kc], r1 = plan.kf_rptr[kc + 1];
    if (!motion_only && vpx) {
        for (int r = r0; r < r1; r++) {
            double* er = E + (size_t)plan.kf_rows[r] * 6 * HW;
            for (int n = 0; n < 6; n++) er[(size_t)n * HW + k] = 0.0;
        }
    }
    double Cacc = 0.0, Wacc = 0.0;
    const double dsp = vpx ? (double)disps[(size_t)kf * HW + k] : 1.0;
    const int e0 = plan.kf_eptr[kc], e1 = plan.kf_eptr[kc + 1];
    for (int ei = e0; ei < e1; ei++) {
        const int e = plan.kf_eidx[ei];
        const int ix = ii[e], jx = jj[e];
        const bool stereo = ix == jx;
        __syncthreads();
        if (threadIdx.x == 0) edge_rel(poses, ix, jx, rel, rel + 3);
        __syncthreads();
        double tij[3] = {rel[0], rel[1], rel[2]};
        double qij[4] = {rel[3], rel[4], rel[5], rel[6]};
        const int ri = plan.edge_ri[e], rj = plan.edge_rj[e];
        double acc[kNJ];
#pragma unroll
        for (int n = 0; n < kNJ; n++) acc[n] = 0.0;
        if (vpx) {
            const size_t base = (size_t)e * 2 * HW + k;
            Lin L;
            lin_pixel(tij, qij, fx, fy, cx, cy, k, W, dsp, (double)target[base],
                      (double)target[base + HW], (double)weight[base], (double)weight[base + HW],
                      L);
            accum_hjj(L, stereo, acc);
            if (!motion_only) {
                Cacc += L.w[0] * L.Jz[0] * L.Jz[0];
                Cacc += L.w[1] * L.Jz[1] * L.Jz[1];
                Wacc += L.w[0] * L.r[0] * L.Jz[0];
                Wacc += L.w[1] * L.r[1] * L.Jz[1];
                const double a0 = stereo ? 0.0 : L.w[0] * L.Jz[0];
                const double a1 = stereo ? 0.0 : L.w[1] * L.Jz[1];
                double g[6];
#pragma unroll
                for (int n = 0; n < 6; n++) g[n] = a0 * L.Jj[0][n] + a1 * L.Jj[1][n];
                if (ri >= 0) {  // Ji-row contribution -Adj g (ba.cuh:139-140)
                    double gi[6];
                    adj_se3(tij, qij, g, gi);
                    double* er = E + (size_t)ri * 6 * HW + k;
#pragma unroll
                    for (int n = 0; n < 6; n++) er[(size_t)n * HW] -= gi[n];
                }
                if (rj >= 0) {
                    double* er = E + (size_t)rj * 6 * HW + k;
#pragma unroll
                    for (int n = 0; n < 6; n++) er[(size_t)n * HW] += g[n];
                }
            }
        }
        block_sum_to(acc, red, hpart + ((size_t)e * nch + chunk) * kNJ);
    }
    if (!motion_only && vpx) {
        // damping_Q_kernel with ep = 1e-7 (ba.cuh:266-281, 701-702)
        const double c = Cacc + 0.2 * (double)eta[(size_t)kf * HW + k] + 1e-7;
        Qo[(size_t)kc * HW + k] = 1.0 / c;
        Wo[(size_t)kc * HW + k] = Wacc;
    }
}

// Same linearization with one wave per edge: a workgroup (pixel chunk,
// keyframe) gives its keyframe's edges to its four waves in turn, each wave
// covering all kLinPx pixels (kLinPx / 64 per lane), so no edge waits for
// another and the per-edge reduction stays inside one wave. The cross-edge
// sums (the E row of the keyframe's own pose, and C, w per pixel) go to
// per-wave LDS slices, added in wave order at the end; the E row of an edge's
// other pose is stored directly, which needs that row to be the edge's alone
// (no two edges of a keyframe share jj; the host checks this and otherwise
// runs k_ba_lin_kf).
constexpr int kLinWaves = kLinWG / 64;
constexpr int kLinPPL = kLinPx / 64;  // pixels per lane
__global__ __launch_bounds__(kLinWG) void k_ba_lin_wv(
    PlanDev plan, const float* __restrict__ target, const float* __restrict__ weight,
    const float* __restrict__ poses, const float* __restrict__ disps,
    const float* __restrict__ intr, const int* __restrict__ ii, const int* __restrict__ jj,
    const float* __restrict__ eta, double* __restrict__ hpart, double* __restrict__ E,
    double* __restrict__ Qo, double* __restrict__ Wo, int HW, int W, int nch, int motion_only) {
    __shared__ double eri_s[kLinWaves][6][kLinPx];  // keyframe-pose E row, per wave
    __shared__ double cw_s[kLinWaves][2][kLinPx];   // C and w, per wave
    const int chunk = blockIdx.x;
    const int kc = blockIdx.y;
    const int kf = plan.kf_list[kc];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const double fx = intr[0], fy = intr[1], cx = intr[2], cy = intr[3];
    int kpx[kLinPPL];
    bool vpx[kLinPPL];
    double dsp[kLinPPL];
#pragma unroll
    for (int s = 0; s < kLinPPL; s++) {
        const int px = s * 64 + lane;
        kpx[s] = chunk * kLinPx + px;
        vpx[s] = kpx[s] < HW;
        dsp[s] = vpx[s] ? (double)disps[(size_t)kf * HW + kpx[s]] : 1.0;
        if (!motion_only) {
#pragma unroll
            for (int n = 0; n < 6; n++) eri_s[wave][n][px] = 0.0;
            cw_s[wave][0][px] = 0.0;
            cw_s[wave][1][px] = 0.0;
        }
    }
    const int e0 = plan.kf_eptr[kc], e1 = plan.kf_eptr[kc + 1];
    for (int ei = e0 + wave; ei < e1; ei += kLinWaves) {
        const int e = plan.kf_eidx[ei];
        const int ix = ii[e], jx = jj[e];
        const bool stereo = ix == jx;
        double tij[3], qij[4];
        edge_rel(poses, ix, jx, tij, qij);  // uniform: every lane computes it
        const int ri = plan.edge_ri[e], rj = plan.edge_rj[e];
        // every pixel's target and weight loads go out before any pixel waits
        float tgu[kLinPPL], tgv[kLinPPL], wtu[kLinPPL], wtv[kLinPPL];
#pragma unroll
        for (int s = 0; s < kLinPPL; s++) {
            const size_t base = (size_t)e * 2 * HW + (vpx[s] ? kpx[s] : 0);
            tgu[s] = target[base];
            tgv[s] = target[base + HW];
            wtu[s] = weight[base];
            wtv[s] = weight[base + HW];
        }
        double acc[kNJ];
#pragma unroll
        for (int n = 0; n < kNJ; n++) acc[n] = 0.0;
#pragma unroll
        for (int s = 0; s < kLinPPL; s++) {
            if (!vpx[s]) continue;
            const int k = kpx[s], px = s * 64 + lane;
            Lin L;
            lin_pixel(tij, qij, fx, fy, cx, cy, k, W, dsp[s], (double)tgu[s], (double)tgv[s],
                      (double)wtu[s], (double)wtv[s], L);
            accum_hjj(L, stereo, acc);
            if (!motion_only) {
                cw_s[wave][0][px] += L.w[0] * L.Jz[0] * L.Jz[0] + L.w[1] * L.Jz[1] * L.Jz[1];
                cw_s[wave][1][px] += L.w[0] * L.r[0] * L.Jz[0] + L.w[1] * L.r[1] * L.Jz[1];
                if (!stereo) {  // a stereo edge adds nothing to E
                    const double a0 = L.w[0] * L.Jz[0], a1 = L.w[1] * L.Jz[1];
                    double g[6];
#pragma unroll
                    for (int n = 0; n < 6; n++) g[n] = a0 * L.Jj[0][n] + a1 * L.Jj[1][n];
                    if (ri >= 0) {  // Ji-row contribution -Adj g (ba.cuh:139-140)
                        double gi[6];
                        adj_se3(tij, qij, g, gi);
#pragma unroll
                        for (int n = 0; n < 6; n++) eri_s[wave][n][px] -= gi[n];
                    }
                    if (rj >= 0) {
                        double* er = E + (size_t)rj * 6 * HW + k;
#pragma unroll
                        for (int n = 0; n < 6; n++) er[(size_t)n * HW] = g[n];
                    }
                }
            }
        }
        int rbase, rvalid;
        wave_reduce_scatter(acc, lane, rbase, rvalid);
        double* hp = hpart + ((size_t)e * nch + chunk) * kNJ;
#pragma unroll
        for (int q = 0; q < RsCounts<kNJ>::c6; q++)
            if (q < rvalid) hp[rbase + q] = acc[q];
    }
    __syncthreads();
    if (!motion_only) {
        // one pixel per thread: the per-wave slices in wave order
        const int px = threadIdx.x, k = chunk * kLinPx + px;
        if (px < kLinPx && k < HW) {
            double c = 0.0, w = 0.0;
#pragma unroll
            for (int v = 0; v < kLinWaves; v++) {
                c += cw_s[v][0][px];
                w += cw_s[v][1][px];
            }
            // damping_Q_kernel with ep = 1e-7 (ba.cuh:266-281, 701-702)
            Qo[(size_t)kc * HW + k] = 1.0 / (c + 0.2 * (double)eta[(size_t)kf * HW + k] + 1e-7);
            Wo[(size_t)kc * HW + k] = w;
            // the keyframe's own pose row
            const int ri = e1 > e0 ? plan.edge_ri[plan.kf_eidx[e0]] : -1;
            if (ri >= 0) {
                double* er = E + (size_t)ri * 6 * HW + k;
#pragma unroll
                for (int n = 0; n < 6; n++) {
                    double t = 0.0;
#pragma unroll
                    for (int v = 0; v < kLinWaves; v++) t += eri_s[v][n][px];
                    er[(size_t)n * HW] = t;
                }
            }
        }
    }
}

// -------------------------------------------------------- k_ba_schur ----
// One workgroup per item over all pixels: E_r1 Q E_r2^T for an upper pair of
// E rows sharing a keyframe (EEt6x6_kernel, ba.cuh:303-342), or E_r Q w for a
// row (Ev6x1_kernel, ba.cuh:346-372); the 36 (or 6) totals go to stot[item].
// Workgroups past the N_items Schur items each form one edge's totals
// (edge_totals, wave 0), which need only the linearization's partials.
__global__ __launch_bounds__(kSchWG) void k_ba_schur(PlanDev plan, const double* __restrict__ E,
                                                     const double* __restrict__ Q,
                                                     const double* __restrict__ Wv,
                                                     double* __restrict__ stot, int HW,
                                                     int N_pu, int N_items,
                                                     const float* __restrict__ poses,
                                                     const int* __restrict__ ii,
                                                     const int* __restrict__ jj,
                                                     const double* __restrict__ hpart,
                                                     double* __restrict__ etot, int nch) {
    __shared__ double red[36 * (kSchWG / 64)];
    const int item = blockIdx.x;
    if (item >= N_items) {
        if (threadIdx.x < 64)
            edge_totals(item - N_items, poses, ii, jj, hpart,
                        etot + (size_t)(item - N_items) * kNT, nch, red);
        return;
    }
    double acc[36];
#pragma unroll
    for (int n = 0; n < 36; n++) acc[n] = 0.0;
    if (item < N_pu) {
        const int r1 = plan.pairs[item * 3 + 0], r2 = plan.pairs[item * 3 + 1];
        const int kc = plan.pairs[item * 3 + 2];
        const double* e1 = E + (size_t)r1 * 6 * HW;
        const double* e2 = E + (size_t)r2 * 6 * HW;
        const double* qk = Q + (size_t)kc * HW;
        for (int k = threadIdx.x; k < HW; k += kSchWG) {
            const double q = qk[k];
            double a[6], b[6];
#pragma unroll
            for (int n = 0; n < 6; n++) {
                a[n] = e1[(size_t)n * HW + k] * q;
                b[n] = e2[(size_t)n * HW + k];
            }
#pragma unroll
            for (int n = 0; n < 6; n++)
#pragma unroll
                for (int m = 0; m < 6; m++) acc[n * 6 + m] += a[n] * b[m];
        }
    } else {
        const int r = item - N_pu;
        const int kc = plan.row_kf[r];
        const double* er = E + (size_t)r * 6 * HW;
        for (int k = threadIdx.x; k < HW; k += kSchWG) {
            const double qw = Q[(size_t)kc * HW + k] * Wv[(size_t)kc * HW + k];
#pragma unroll
            for (int n = 0; n < 6; n++) acc[n] += qw * er[(size_t)n * HW + k];
        }
    }
    block_sum_to(acc, red, stot + (size_t)item * 36);
}

// ----------------------------------------------------------- solve ------
// the BA status words (BaState::flags): [0] the last step was rejected, [1]
// a step was rejected (sticky), [2] a failed pivot of the blocked solve, [3]
// a wait of an overlapped step gave up (sticky), [4], [5] that give-up within
// the current call (see the overlapped step's handshake)
constexpr int kBaFlags = 8;

struct SolveArgs {
    PlanDev plan;
    const double* etot;   // [M][120] per-edge Hii, Hij, Hjj, vi, vj
    const double* stot;   // [N_pu + N_E][36] Schur pair blocks / row gradients
    int N_pu, P, n, n_blk, t0, t1;
    float lm, ep;
    double* S;      // working copy of the blocked solver [(n+1)*n]: S, then b^T
    double* S_dbg;  // [n*n] assembled system (after damping), input of the solve
    double* b_dbg;  // [n]
    double* dx_dbg; // [n]
    float* dx;      // [n] fp32 step used by retraction and back-substitution
    int* flags;     // [0] this iteration not SPD, [1] sticky
    const int* halt;  // or null: when *halt is set the step is not taken (an earlier wait gave up)
    float* poses;
    float* poses_prev;  // [P][7] poses t0..t1-1 before the step (fused path), or null
    float* poses_next;  // [P][7] poses t0..t1-1 after the step (overlapped fused path), or null
    int* publish;       // or null: set (agent-scope release) once the status and dx are out,
                        // before the retraction (the overlapped step's ready flag)
};

// One edge-block or Schur-item contribution to entry (r, c) of a 6x6 block of
// S (ba.cuh:520-548, 722-742): code cd of the block's contribution list.
__device__ __forceinline__ double s_contrib(const SolveArgs& A, int cd, int r, int c) {
    const int ty = code_type(cd), v = code_val(cd);
    if (ty == 0) {
        const double* et = A.etot + (size_t)(v >> 2) * kNT;
        const int w = v & 3;
        return w == 0 ? et[kTotHii + r * 6 + c]
             : w == 1 ? et[kTotHij + r * 6 + c]
             : w == 2 ? et[kTotHij + c * 6 + r]
                      : et[kTotHjj + r * 6 + c];
    }
    return -A.stot[(size_t)v * 36 + (ty == 1 ? r * 6 + c : c * 6 + r)];
}

// One workgroup per 6x6 block (a, b) of S (P*P of them) and per 6-entry
// segment of b (P more): S = sum of the listed edge blocks minus the Schur
// pair blocks, then the LM damping S_ii += ep + lm*S_ii after the Schur step
// (ba.cuh:749-750); b = the edges' gradients minus E Q w of the pose's rows.
// Thread (slice, entry) sums contributions slice, slice + 7, ... of the list,
// and the seven slices are added in a fixed order (deterministic, no atomics).
constexpr int kAsmSlices = 7;  // 7 x 36 = 252 of the 256 threads
__global__ __launch_bounds__(256) void k_ba_assemble(SolveArgs A) {
    __shared__ double red[kAsmSlices][36];
    const int n = A.n, P = A.P;
    const int tid = threadIdx.x;
    const int sl = tid / 36, e = tid - sl * 36;
    const int g = blockIdx.x;
    double s = 0.0;
    if (g < P * P) {
        const int a = g / P, bb = g - a * P;
        const int r = e / 6, c = e - r * 6;
        const int blk = A.plan.blkmap[g];
        if (sl < kAsmSlices && blk >= 0) {
            const int q1 = A.plan.sblk_ptr[blk + 1];
            for (int q = A.plan.sblk_ptr[blk] + sl; q < q1; q += kAsmSlices)
                s += s_contrib(A, A.plan.sblk_src[q], r, c);
        }
        if (sl < kAsmSlices) red[sl][e] = s;
        __syncthreads();
        if (tid < 36) {
            double t = red[0][tid];
#pragma unroll
            for (int k = 1; k < kAsmSlices; k++) t += red[k][tid];
            const int row = a * 6 + tid / 6, col = bb * 6 + tid % 6;
            if (row == col) t = t + (double)A.ep + (double)A.lm * t;
            A.S_dbg[(size_t)row * n + col] = t;
        }
    } else {
        const int a = g - P * P;
        const int k = e;  // entries 0..5 of segment a; threads with e >= 6 idle
        if (sl < kAsmSlices && k < 6) {
            for (int q = A.plan.bv_ptr[a] + sl; q < A.plan.bv_ptr[a + 1]; q += kAsmSlices) {
                const int cd = A.plan.bv_src[q];
                const int v = code_val(cd);
                if (code_type(cd) == 0)
                    s += A.etot[(size_t)(v >> 1) * kNT + ((v & 1) ? kTotVj : kTotVi) + k];
                else
                    s -= A.stot[(size_t)(A.N_pu + v) * 36 + k];
            }
        }
        if (sl < kAsmSlices) red[sl][e] = s;
        __syncthreads();
        if (tid < 6) {
            double t = red[0][tid];
#pragma unroll
            for (int m = 1; m < kAsmSlices; m++) t += red[m][tid];
            A.b_dbg[a * 6 + tid] = t;
        }
    }
}

__device__ __forceinline__ double bcast(double v, int src) {
    const int lo = __builtin_amdgcn_readlane(__double2loint(v), src);
    const int hi = __builtin_amdgcn_readlane(__double2hiint(v), src);
    return __hiloint2double(hi, lo);
}

// A pose after its step, as the solve stores it: the fp32 values of the fp64
// retraction (pose_retr_kernel, ba.cuh:757-760) of pose p7 by the fp32 step
// d6. The linearization workgroups of an overlapped step form the poses they
// need with this too, from the same inputs, instead of waiting for the
// solve's retraction.
__device__ __forceinline__ void step_pose(const float* p7, const float (&d6)[6], float (&out)[7]) {
    double t[3], q[4], xi[6], t1[3], q1[4];
    load_pose(p7, 0, t, q);
#pragma unroll
    for (int m = 0; m < 6; m++) xi[m] = (double)d6[m];
    retr_se3(xi, t, q, t1, q1);
#pragma unroll
    for (int m = 0; m < 3; m++) out[m] = (float)t1[m];
#pragma unroll
    for (int m = 0; m < 4; m++) out[3 + m] = (float)q1[m];
}

// A halted call takes no more steps: like a rejected step, but not reported
// as one. The flag is written by an earlier launch, so a solve reads it with
// its system's loads rather than after the factorization: an unconditional
// vector load (a zero word stands in for a missing flag) whose word is only
// tested in finish_solve. Its address carries a per-lane zero offset the
// compiler cannot fold, so the load is not turned into a scalar load that is
// waited for at once; it stays in flight beside the system's loads.
__device__ int g_no_halt = 0;
__device__ __forceinline__ int solve_halt_word(const SolveArgs& A) {
    int z;
    asm volatile("v_mov_b32 %0, 0" : "=v"(z));
    return __hip_atomic_load((A.halt ? A.halt : &g_no_halt) + z, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
}

// Outputs of a solve: the status flags, dx (fp64 and the fp32 step), and the
// retraction of poses t0..t1-1, whose current values are read from
// pose_src[(k - t0) * 7 ..] (A.poses + 7 * t0, or a copy taken earlier).
// With A.publish, the flag is set once the status and dx are out, before the
// retraction (every thread of the workgroup calls this). halt_word:
// solve_halt_word, read when the solve starts.
__device__ __forceinline__ void finish_solve(const SolveArgs& A, const double* x, bool ok,
                                             int halt_word, const float* pose_src) {
    const int n = A.n;
    const bool halted = halt_word != 0;
    if (threadIdx.x == 0) {
        A.flags[0] = ok && !halted ? 0 : 1;
        if (!ok && !halted) A.flags[1] = 1;
    }
    ok = ok && !halted;
    for (int t = threadIdx.x; t < n; t += blockDim.x) {
        A.dx_dbg[t] = ok ? x[t] : 0.0;
        A.dx[t] = ok ? (float)x[t] : 0.0f;
    }
    if (A.publish) {
        // every wave's writes (status, dx) made visible device-wide before
        // the flag
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        __syncthreads();
        if (threadIdx.x == 0)
            __hip_atomic_store(A.publish, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (!ok) {  // the poses stay; the overlapped path still needs their copy
        if (A.poses_next)
            for (int t = threadIdx.x; t < (A.t1 - A.t0) * 7; t += blockDim.x)
                A.poses_next[t] = pose_src[t];
        return;
    }
    // pose_retr_kernel on the fp32 step (ba.cuh:757-760), fp64 inside
    for (int k = A.t0 + threadIdx.x; k < A.t1; k += blockDim.x) {
        if (A.poses_prev)  // the fused path's back-substitution relinearizes at these
            for (int m = 0; m < 7; m++) A.poses_prev[(k - A.t0) * 7 + m] = pose_src[(k - A.t0) * 7 + m];
        float d6[6], pn[7];
        for (int m = 0; m < 6; m++) d6[m] = (float)x[(k - A.t0) * 6 + m];
        step_pose(pose_src + (k - A.t0) * 7, d6, pn);
        for (int m = 0; m < 7; m++) A.poses[k * 7 + m] = pn[m];
        if (A.poses_next)  // read by the next overlapped step's relinearization
            for (int m = 0; m < 7; m++) A.poses_next[(k - A.t0) * 7 + m] = pn[m];
    }
}

// 1/sqrt(d) in fp64: hardware estimate + two Newton steps
// y <- y * (1.5 - 0.5 d y^2), ~1 ulp for positive normal d.
__device__ __forceinline__ double rsqrt_f64(double d) {
    double y = __builtin_amdgcn_rsq(d);
    const double h = 0.5 * d;
    y = y * (1.5 - h * y * y);
    y = y * (1.5 - h * y * y);
    return y;
}

// Cholesky of an N x N SPD matrix in one wavefront's registers (N <= 64):
// lane i holds row i in r[] and ends with row i of L in r[0..i] (entries right
// of the diagonal receive updates too and are left unused, so no lane is ever
// predicated off). Columns go in panels of W: inside a panel, each column's
// pivot and its entries in the panel's later columns come by readlane; then
// every lane publishes its W panel entries to LDS (Lp, one 8W-byte row per
// lane) and each later column k takes the panel's W updates from one
// broadcast read of row k. Only the panel steps are sequential; the trailing
// reads go out together. The arithmetic is the unblocked right-looking order
// exactly: r[k] -= L[i][j] L[k][j] for j = 0, 1, ... Same pivot test as the
// reference (every pivot > 0 before its sqrt, ba.cuh:422). inv_diag receives
// 1/L[lane][lane].
template <int N, int W, int kAhead = 3>
__device__ __forceinline__ void wave_cholesky(double (&r)[N], double (*Lp)[W], bool& ok,
                                              double& inv_diag) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int c0 = 0; c0 < N; c0 += W) {
        const int cw = N - c0 < W ? N - c0 : W;
#pragma unroll
        for (int jj = 0; jj < W; jj++) {
            if (jj < cw) {
                const int j = c0 + jj;
                const double d = bcast(r[j], j);
                ok = ok && (d > 0.0);
                const double inv = rsqrt_f64(d);  // 1 / L_jj
                r[j] = lane == j ? d * inv : r[j] * inv;
                if (lane == j) inv_diag = inv;
#pragma unroll
                for (int kk = jj + 1; kk < W; kk++)
                    if (kk < cw) r[c0 + kk] -= r[j] * bcast(r[j], c0 + kk);
            }
        }
        if (c0 + W < N) {
#pragma unroll
            for (int m = 0; m < W; m++) Lp[lane][m] = r[c0 + m];
            // rows k of the panel read kAhead columns ahead of their use, in a
            // register ring; the scheduling barriers keep the compiler from
            // pulling each read down next to its use
            double Lk[kAhead + 1][W];
#pragma unroll
            for (int q = 0; q < kAhead; q++)
                if (c0 + W + q < N)
#pragma unroll
                    for (int m = 0; m < W; m++) Lk[q][m] = Lp[c0 + W + q][m];
#pragma unroll
            for (int k = c0 + W; k < N; k++) {
                const int q = k - c0 - W;
                if (k + kAhead < N)
#pragma unroll
                    for (int m = 0; m < W; m++) Lk[(q + kAhead) % (kAhead + 1)][m] = Lp[k + kAhead][m];
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int m = 0; m < W; m++) r[k] -= r[c0 + m] * Lk[q % (kAhead + 1)][m];
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
}

constexpr int kPanelW = 8;

// ---- one-workgroup panel solver (n <= kPanelN: the frontend's systems) ----
// LDL^T of the bordered matrix [S b; b^T *] in LDS, right-looking in panels
// of kPW columns. The system is padded to n8 = a multiple of kPW with
// identity rows and columns (b padded with zeros), so every panel is full,
// every row block of the backward solve lies on one side of row 64, and the
// latency chains below carry no bounds branches (a taken branch costs about
// as much as a dependent fp64 operation). The packed lower triangle (row i
// at tri(i)) holds rows 0..n8-1 and b^T in row n8. Per panel, two barriers:
// (1) every wave g < ng holds the panel's diagonal rows in lanes 0..kPW-1
//     and up to kPanelRows rows below the diagonal block in the other lanes,
//     their panel entries in registers, and eliminates the panel's columns
//     one at a time: pivot d_j by readlane, 1/d_j (hardware estimate + two
//     Newton steps), l_ij = u_ij / d_j, and u_ik -= l_ij u_kj for the later
//     panel columns k, u_kj being read by readlane before 1/d_j is known.
//     Every wave eliminates the diagonal block itself, with the same
//     arithmetic, so no wave waits on another inside a panel; each writes
//     back the l of its rows below the block.
// (2) after the barrier, wave 0 writes the diagonal block's l (its pivots
//     went out before the barrier), and all threads subtract the panel's products from the
//     trailing lower triangle, A[i][k] -= sum_m l_im d_m l_km, in 2 x 2
//     register blocks.
// Row n8 ends as w = D^-1 L^-1 b, so the backward solve L^T x = w (unit
// diagonal) is one readlane and one multiply-add per row, in wave 0 (lane i
// holding rows i and i + 64), with each block's entries of L read into
// registers while the previous block runs. S = L D L^T is the reference's
// S = L L^T with L_chol = L D^1/2; the pivot test is the reference's (every
// pivot > 0, ba.cuh:422), and a failed pivot ends the factorization with a
// zero step.
constexpr int kPW = 8;
constexpr int kPanelRows = 64 - kPW;  // rows below the diagonal block per wave
constexpr int kPanelN = 120;          // packed [S; b^T] of n8 = 120: 7381 doubles, 59 KB
constexpr int kPanelPoses = kPanelN / 6;
static_assert(kPanelN % kPW == 0, "the largest system is a whole number of panels");
static_assert(kPanelN + 1 - kPW <= 3 * kPanelRows, "three waves cover the rows below a panel");
static_assert(kPanelN <= 128 && 64 % kPW == 0, "the backward solve holds two rows per lane");

__host__ __device__ __forceinline__ int tri(int i) { return i * (i + 1) / 2; }
__host__ __device__ __forceinline__ int pad_panel(int n) { return (n + kPW - 1) / kPW * kPW; }

size_t panel_solve_lds_bytes(int n) {
    const int n8 = pad_panel(n);
    return ((size_t)tri(n8 + 1) + 2 * (size_t)n8) * sizeof(double);
}

// 1/d in fp64: hardware estimate + two Newton steps (~1 ulp for normal d)
__device__ __forceinline__ double rcp_f64(double d) {
    double y = __builtin_amdgcn_rcp(d);
    y = __builtin_fma(y, __builtin_fma(-d, y, 1.0), y);
    y = __builtin_fma(y, __builtin_fma(-d, y, 1.0), y);
    return y;
}

// 1/d with one Newton step: the estimate's 2^-24.4 relative error squared,
// ~2^-48.8 (4e-15), for the pivots of the small solve, where each pivot's
// reciprocal is on the factorization's dependency chain.
__device__ __forceinline__ double rcp_f64_1(double d) {
    const double y = __builtin_amdgcn_rcp(d);
    return __builtin_fma(y, __builtin_fma(-d, y, 1.0), y);
}

// LDS of the panel solver at its largest size, for a launch whose LDS is
// declared statically (sm: packed [S; b^T], pivots, solution)
struct PanelLds {
    double sm[(kPanelN + 1) * (kPanelN + 2) / 2 + 2 * kPanelN];
    int ok;
    float pose0[kPanelPoses * 7];
};

// sm: panel_solve_lds_bytes(A.n) bytes; pose0: the poses t0..t1-1 before the step
__device__ __forceinline__ void solve_panel_body(const SolveArgs& A, double* sm, int& ok_sh,
                                                 float* pose0) {
    const int n = A.n, n8 = pad_panel(n), tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    double* L = sm;                   // packed lower [S; b^T], padded
    double* piv = sm + tri(n8 + 1);   // [n8] pivots d_j
    double* xs = piv + n8;            // [n8] the solution
    const int halt_word = solve_halt_word(A);
    if (tid < (A.t1 - A.t0) * 7) pose0[tid] = A.poses[A.t0 * 7 + tid];
    // rows of [S; b^T] with the padding (identity rows, zeros elsewhere):
    // wave w takes rows w, w + 4, .., lanes the columns lane, lane + 64; the
    // loads of kLdRows rows go out before the first is stored (S comes from
    // the assembly on other CUs)
    constexpr int kLdRows = 8;
    for (int i0 = wave; i0 <= n8; i0 += 4 * kLdRows) {
        double v[kLdRows][2];
#pragma unroll
        for (int r = 0; r < kLdRows; r++)
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int i = i0 + 4 * r, k = lane + 64 * h;
                double x = k == i ? 1.0 : 0.0;
                if (k < n && i < n && k <= i) x = A.S_dbg[(size_t)i * n + k];
                if (k < n && i == n8) x = A.b_dbg[k];
                v[r][h] = x;
            }
#pragma unroll
        for (int r = 0; r < kLdRows; r++)
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int i = i0 + 4 * r, k = lane + 64 * h;
                if (i <= n8 && k <= i && k < n8) L[tri(i) + k] = v[r][h];
            }
    }
    if (tid == 0) ok_sh = 1;
    __syncthreads();
    for (int c0 = 0; c0 < n8; c0 += kPW) {
        const int r0 = c0 + kPW;
        const int ng = (n8 + 1 - r0 + kPanelRows - 1) / kPanelRows;  // >= 1
        const bool dg = lane < kPW;
        double p[kPW];
        double dj = 0.0;  // diagonal lane j: pivot j
        if (wave < ng) {  // uniform
            const int row = dg ? c0 + lane : r0 + kPanelRows * wave + lane - kPW;
            const bool live = dg || row <= n8;
            const double* src = L + tri(live ? row : n8) + c0;
#pragma unroll
            for (int m = 0; m < kPW; m++) {
                const double v = src[m];
                p[m] = live && (!dg || m <= lane) ? v : 0.0;
            }
            bool ok = true;
#pragma unroll
            for (int j = 0; j < kPW; j++) {
                double u[kPW];  // u_kj of the later diagonal rows k, before the pivot is known
#pragma unroll
                for (int k = j + 1; k < kPW; k++) u[k] = bcast(p[j], k);
                const double d = bcast(p[j], j);
                ok = ok && (d > 0.0);
                const double l = p[j] * rcp_f64(d);
                if (lane == j) dj = d;
                p[j] = l;
#pragma unroll
                for (int k = j + 1; k < kPW; k++) p[k] -= l * u[k];
            }
            if (!dg && live) {
                double* dst = L + tri(row) + c0;
#pragma unroll
                for (int m = 0; m < kPW; m++) dst[m] = p[m];
            }
            if (wave == 0 && dg) piv[c0 + lane] = dj;  // read by the trailing update
            if (!ok && lane == 0) ok_sh = 0;
        }
        __syncthreads();
        if (!ok_sh) break;  // uniform
        if (wave == 0 && dg) {
            // the diagonal block: no wave reads it again during this panel
            double* dst = L + tri(c0 + lane) + c0;
#pragma unroll
            for (int m = 0; m < kPW; m++)
                if (m < lane) dst[m] = p[m];
        }
        // trailing update, rows r0..n8 (b^T last), columns r0..n8-1, 2 x 2
        // blocks; the last block row holds b^T alone
        const int nbi = (n8 - r0) / 2 + 1;
        const int cnt = nbi * (nbi + 1) / 2;
        for (int t = tid; t < cnt; t += 256) {
            const int bi = (int)((__builtin_sqrt(8.0 * t + 1.0) - 1.0) * 0.5);
            const int bk = t - tri(bi);
            const int i0 = r0 + 2 * bi, k0 = r0 + 2 * bk;
            if (k0 >= n8) continue;  // b^T's block row has one block fewer
            const bool two = i0 < n8;  // i0 + 1 exists (not b^T's row)
            const double* a0 = L + tri(i0) + c0;
            const double* a1 = L + tri(two ? i0 + 1 : i0) + c0;
            const double* b0 = L + tri(k0) + c0;
            const double* b1 = L + tri(k0 + 1) + c0;
            const double* dp = piv + c0;
            double x0[kPW], x1[kPW], y0[kPW], y1[kPW];
#pragma unroll
            for (int m = 0; m < kPW; m++) {
                x0[m] = a0[m];
                x1[m] = a1[m];
                y0[m] = b0[m] * dp[m];
                y1[m] = b1[m] * dp[m];
            }
            double s00 = 0.0, s01 = 0.0, s10 = 0.0, s11 = 0.0;
#pragma unroll
            for (int m = 0; m < kPW; m++) {
                s00 += x0[m] * y0[m];
                s01 += x0[m] * y1[m];
                s10 += x1[m] * y0[m];
                s11 += x1[m] * y1[m];
            }
            L[tri(i0) + k0] -= s00;  // k0 <= i0
            if (k0 < i0) L[tri(i0) + k0 + 1] -= s01;
            if (two) {
                L[tri(i0 + 1) + k0] -= s10;
                L[tri(i0 + 1) + k0 + 1] -= s11;
            }
        }
        __syncthreads();
    }
    const bool ok = ok_sh != 0;
    if (ok && wave == 0 && n8 <= 64) {
        // L^T x = w, w = row n8, lane i holding row i: x_k = acc_k once the
        // rows below k are in, then acc_i -= l_ki x_k for i < k (l_ki taken
        // as zero for i >= k, so lane k keeps x_k). The whole column of L is
        // read into registers first; the 64 steps are straight-line code
        // (rows past n8 carry zeros).
        double c[64];
#pragma unroll
        for (int k = 0; k < 64; k++) {
            const int kk = min(k, n8 - 1);  // rows past n8 - 1 read row n8 - 1, discarded
            const double v = L[tri(kk) + min(lane, kk)];
            c[k] = lane < k && k < n8 ? v : 0.0;
        }
        double acc = L[tri(n8) + min(lane, n8 - 1)];
        if (lane >= n8) acc = 0.0;
#pragma unroll
        for (int k = 63; k >= 0; k--) acc -= c[k] * bcast(acc, k);
        if (lane < n8) xs[lane] = acc;
    } else if (ok && wave == 0) {
        // L^T x = w, w = row n8: x_k = acc_k once the rows below k are in;
        // then acc_i -= l_ki x_k for i < k (the prefetched l_ki is zero for
        // i >= k, so lane k keeps x_k). Blocks of kPW rows from the bottom.
        const double* w = L + tri(n8);
        double acc0 = lane < n8 ? w[lane] : 0.0;
        double acc1 = lane + 64 < n8 ? w[lane + 64] : 0.0;
        double l0[kPW], l1[kPW];
        auto fetch = [&](int kb) {  // rows kb, kb - 1, .., kb - kPW + 1
#pragma unroll
            for (int q = 0; q < kPW; q++) {
                const int k = kb - q;
                const double* Lk = L + tri(k);
                const double v0 = Lk[min(lane, k)], v1 = Lk[min(lane + 64, k)];
                l0[q] = lane < k ? v0 : 0.0;
                l1[q] = lane + 64 < k ? v1 : 0.0;
            }
        };
        fetch(n8 - 1);
        for (int kb = n8 - 1; kb >= 0; kb -= kPW) {  // uniform
            double c0v[kPW], c1v[kPW];
#pragma unroll
            for (int q = 0; q < kPW; q++) {
                c0v[q] = l0[q];
                c1v[q] = l1[q];
            }
            if (kb >= kPW) fetch(kb - kPW);
            if (kb >= 64) {  // uniform: the block's rows are all >= 64
#pragma unroll
                for (int q = 0; q < kPW; q++) {
                    const double xk = bcast(acc1, kb - 64 - q);
                    acc0 -= c0v[q] * xk;
                    acc1 -= c1v[q] * xk;
                }
            } else {
#pragma unroll
                for (int q = 0; q < kPW; q++) {
                    const double xk = bcast(acc0, kb - q);
                    acc0 -= c0v[q] * xk;
                }
            }
        }
        if (lane < n8) xs[lane] = acc0;
        if (lane + 64 < n8) xs[lane + 64] = acc1;
    }
    __syncthreads();
    finish_solve(A, xs, ok, halt_word, pose0);
}

__global__ __launch_bounds__(256) void k_ba_solve_panel(SolveArgs A) {
    extern __shared__ double sm[];
    __shared__ int ok_sh;
    __shared__ float pose0[kPanelPoses * 7];
    solve_panel_body(A, sm, ok_sh, pose0);
}

// ---- one-workgroup solver with the system in registers (n <= 64) ----
// LDL^T of the bordered matrix [S b; b^T *] padded to n8 (a multiple of
// kPW, <= 64) as in k_ba_solve_panel, but the working matrix never lives in
// LDS: its lower triangle is cut into 2 x 2 blocks (block row n8 / 2 holds
// b^T alone), each owned by one thread for the whole factorization
// (kSmallSlots register blocks per thread), and loaded from the assembled
// system once. Per panel of kPW columns, two barriers:
// (1) the owners of the panel's blocks publish them (rows c0..n8) to LDS;
// (2) every thread reads the panel's diagonal block and eliminates it
//     itself (uniform values: pivots, 1/d by estimate + two Newton steps,
//     multipliers), so every thread takes the same pivot test without a
//     shared flag; thread t then finishes row r0 + t of the panel by forward
//     substitution against the diagonal block and publishes its l and d*l;
// (3) every thread subtracts the panel's products from its own blocks right
//     of the panel, A[i][k] -= sum_m l_im (d_m l_km).
// The l of every panel also go to a full copy of L (upper part and rows
// past n8 zero), which wave 0's backward solve L^T x = w (w = D^-1 L^-1 b,
// the bordered row) reads column by column with constant offsets, every
// read unconditional (a conditional LDS read becomes a branch that waits
// for it).
constexpr int kSmallN = 64;
constexpr int kSmallSlots = 3;  // ceil(560 / 256): 2 x 2 blocks of n8 = 64 per thread
static_assert(kSmallN % kPW == 0 && kSmallN <= 64, "one row per lane in the backward solve");

// Rows of the panel buffers hold kPW + 1 doubles and rows of L 65: a lane
// per row then lands on a different pair of LDS banks for every lane (at
// kPW and 64 doubles, 16 and 64 lanes of a wave share a bank).
constexpr int kSmallPLd = kPW + 1;
constexpr int kSmallLfLd = 65;
constexpr int kSmallLfRows = (kSmallN + 1 + 7) / 8 * 8;
static_assert(kSmallLfRows * kSmallLfLd % 2 == 0, "L zeroed as 16-byte pairs");

struct SmallLds {
    double PU[kSmallN + 1][kSmallPLd];  // panel as published
    double PL[kSmallN + 1][kSmallPLd];  // l of rows >= r0
    double PD[kSmallN + 1][kSmallPLd];  // d_m * l of rows >= r0
    // L by rows, row n8 = w; zero elsewhere
    __attribute__((aligned(16))) double Lf[kSmallLfRows][kSmallLfLd];
    double xs[kSmallN];
    float pose0[(kSmallN / 6) * 7];
};

__device__ __forceinline__ void solve_small_body(const SolveArgs& A, SmallLds& sm) {
    auto& PU = sm.PU;
    auto& PL = sm.PL;
    auto& PD = sm.PD;
    auto& Lf = sm.Lf;
    auto& xs = sm.xs;
    auto& pose0 = sm.pose0;
    const int n = A.n, n8 = pad_panel(n), tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int hb = n8 / 2;                    // block rows 0..hb (hb: b^T)
    const int nblk = hb * (hb + 1) / 2 + hb;  // lower 2 x 2 blocks
    {
        constexpr int kPairs = kSmallLfRows * kSmallLfLd / 2;
#pragma unroll
        for (int u = 0; u < (kPairs + 255) / 256; u++)
            if (tid + 256 * u < kPairs)
                reinterpret_cast<double2*>(&Lf[0][0])[tid + 256 * u] = make_double2(0.0, 0.0);
    }
    // this thread's blocks: (i0, k0) of slot s, and their four entries
    // (every slot's indices first, then the loads: the index arithmetic
    // carries waits of its own that would otherwise fall between the loads)
    int bi0[kSmallSlots], bk0[kSmallSlots];
#pragma unroll
    for (int s = 0; s < kSmallSlots; s++) {
        const int b = tid + 256 * s;
        int bi = hb, bk = b - hb * (hb + 1) / 2;
        if (b < hb * (hb + 1) / 2) {
            bi = (int)((__builtin_sqrt(8.0 * b + 1.0) - 1.0) * 0.5);
            bk = b - bi * (bi + 1) / 2;
        }
        const bool live = b < nblk;
        bi0[s] = live ? 2 * bi : -2;  // -2: no block (never in a panel's rows)
        bk0[s] = live ? 2 * bk : -2;
    }
    const int halt_word = solve_halt_word(A);
    // this thread's word of the poses t0..t1-1 (clamped, unconditional: the
    // load goes out with the system's and is waited for only at its store)
    const int np7 = (A.t1 - A.t0) * 7;
    const float pose_word = A.poses[np7 > 0 ? A.t0 * 7 + min(tid, np7 - 1) : 0];
    double a[kSmallSlots][4];
#pragma unroll
    for (int s = 0; s < kSmallSlots; s++) {
        const bool live = bi0[s] >= 0;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int i = bi0[s] + (e >> 1), k = bk0[s] + (e & 1);
            double x = i == k ? 1.0 : 0.0;
            if (live && k < n && i < n && k <= i) x = A.S_dbg[(size_t)i * n + k];
            if (live && k < n && i == n8) x = A.b_dbg[k];
            a[s][e] = x;
        }
    }
    if (tid < np7) pose0[tid] = pose_word;
    bool ok = true;
    for (int c0 = 0; c0 < n8; c0 += kPW) {  // uniform
        const int r0 = c0 + kPW;
        // (1) publish the panel's columns, rows c0..n8
#pragma unroll
        for (int s = 0; s < kSmallSlots; s++) {
            const int i0 = bi0[s], k0 = bk0[s];
            if (i0 >= c0 && k0 >= c0 && k0 < r0) {
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int i = i0 + (e >> 1), k = k0 + (e & 1);
                    if (i <= n8 && k <= i) PU[i][k - c0] = a[s][e];
                }
            }
        }
        __syncthreads();
        // (2) the diagonal block, eliminated by every thread (uniform), and
        // with it, pivot by pivot, thread t's row r0 + t of rows r0..n8
        // (right-looking: l_j = u_j / d_j, then u_k -= l_j D_kj for the later
        // columns k, D_kj being the block's column j before its scaling), so
        // the rows' chains run beside the pivots' instead of after them
        const bool has_row = tid <= n8 - r0;
        const int row = has_row ? r0 + tid : n8;
        double D[kPW][kPW], Lb[kPW][kPW], rj[kPW], dj[kPW], u[kPW], l[kPW];
#pragma unroll
        for (int i = 0; i < kPW; i++)
#pragma unroll
            for (int k = 0; k <= i; k++) D[i][k] = PU[c0 + i][k];
#pragma unroll
        for (int j = 0; j < kPW; j++) u[j] = PU[row][j];
#pragma unroll
        for (int j = 0; j < kPW; j++) {
            dj[j] = D[j][j];
            ok = ok && (dj[j] > 0.0);
            rj[j] = rcp_f64_1(dj[j]);
            l[j] = u[j] * rj[j];
#pragma unroll
            for (int k = j + 1; k < kPW; k++) u[k] -= l[j] * D[k][j];
#pragma unroll
            for (int i = j + 1; i < kPW; i++) Lb[i][j] = D[i][j] * rj[j];
#pragma unroll
            for (int i = j + 1; i < kPW; i++)
#pragma unroll
                for (int k = j + 1; k <= i; k++) D[i][k] -= Lb[i][j] * D[k][j];
        }
        if (!ok) break;  // uniform: every thread took the same pivots
        if (has_row) {
#pragma unroll
            for (int j = 0; j < kPW; j++) {
                PL[row][j] = l[j];
                PD[row][j] = l[j] * dj[j];
                Lf[row][c0 + j] = l[j];
            }
        }
        if (tid == 255) {  // the diagonal block's rows of L (constant indices into Lb)
#pragma unroll
            for (int q = 1; q < kPW; q++)
#pragma unroll
                for (int m = 0; m < q; m++) Lf[c0 + q][c0 + m] = Lb[q][m];
        }
        __syncthreads();
        // (3) this thread's blocks right of the panel
#pragma unroll
        for (int s = 0; s < kSmallSlots; s++) {
            const int i0 = bi0[s], k0 = bk0[s];
            if (k0 >= r0) {  // then i0 >= k0 >= r0 (no-block slots have k0 = -2)
                const int i1 = min(i0 + 1, n8);
                double s00 = 0.0, s01 = 0.0, s10 = 0.0, s11 = 0.0;
#pragma unroll
                for (int m = 0; m < kPW; m++) {
                    const double x0 = PL[i0][m], x1 = PL[i1][m];
                    const double y0 = PD[k0][m], y1 = PD[k0 + 1][m];
                    s00 += x0 * y0;
                    s01 += x0 * y1;
                    s10 += x1 * y0;
                    s11 += x1 * y1;
                }
                a[s][0] -= s00;
                a[s][1] -= s01;
                a[s][2] -= s10;
                a[s][3] -= s11;
            }
        }
    }
    // (every thread left the loop at the same panel; the last barrier of a
    // completed factorization orders the writes of Lf before these reads)
    if (ok && wave == 0) {
        double c[64];
#pragma unroll
        for (int k = 0; k < 64; k++) c[k] = Lf[k][lane];  // zero unless lane < k < n8
        double acc = Lf[n8][lane];
#pragma unroll
        for (int k = 63; k >= 0; k--) acc -= c[k] * bcast(acc, k);
        if (lane < n8) xs[lane] = acc;
    }
    __syncthreads();
    finish_solve(A, xs, ok, halt_word, pose0);
}

__global__ __launch_bounds__(256) void k_ba_solve_small(SolveArgs A) {
    __shared__ SmallLds sm;
    solve_small_body(A, sm);
}

// ---- blocked Cholesky over many workgroups (n > kPanelN: the backend's systems) ----
// Right-looking, lower, on the row-major working copy A.S, which holds the
// system in rows 0..n-1 and b^T in row n (leading dimension n): factoring the
// bordered matrix [S b; b^T *] leaves L^-1 b in row n, so the forward solve
// costs one more panel row. In kCB-column steps: (1) k_chol_diag factors the
// kCB x kCB diagonal block in one wavefront's registers (lane = row,
// wave_cholesky); (2) k_chol_panel solves the rows below it (b's row
// included) against it, one thread per row; (3) k_chol_syrk subtracts the
// new panel's products from the trailing lower triangle in 64 x 64 tiles,
// one workgroup per tile. k_chol_finish then runs the backward solve
// L^T x = z in one workgroup (O(n^2), coalesced column reads) and the
// retraction. A failed pivot is flagged in flags[2] (cleared by k_chol_init);
// later kernels then do nothing and k_chol_finish reports the system not
// positive definite, as the one-workgroup solvers do.
constexpr int kCB = 64;

__global__ __launch_bounds__(256) void k_chol_init(SolveArgs A) {
    const size_t nn = (size_t)A.n * A.n;
    for (size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x; t < nn + A.n;
         t += (size_t)gridDim.x * blockDim.x)
        A.S[t] = t < nn ? A.S_dbg[t] : A.b_dbg[t - nn];
    if (blockIdx.x == 0 && threadIdx.x == 0) A.flags[2] = 0;
}

// The diagonal block, padded to kCB x kCB with an identity block (whose
// Cholesky is itself), so wave_cholesky runs at its compile-time size.
__global__ __launch_bounds__(64) void k_chol_diag(SolveArgs A, int j0) {
    __shared__ __attribute__((aligned(16))) double Lp[64][kPanelW];
    if (A.flags[2]) return;
    const int n = A.n, lane = threadIdx.x;
    const int nb = min(kCB, n - j0);
    double* S = A.S;
    double r[kCB];
#pragma unroll
    for (int m = 0; m < kCB; m++)
        r[m] = (lane < nb && m < nb) ? S[(size_t)(j0 + lane) * n + j0 + m]
                                     : (m == lane ? 1.0 : 0.0);
    bool ok = true;
    double invd = 0.0;
    wave_cholesky<kCB, kPanelW>(r, Lp, ok, invd);
    if (lane < nb) {
#pragma unroll
        for (int m = 0; m < kCB; m++)
            if (m <= lane) S[(size_t)(j0 + lane) * n + j0 + m] = r[m];
    }
    if (lane == 0 && !ok) A.flags[2] = 1;
}

// rows j0 + nb <= i <= n (row n is b): x L_jj^T = S[i][j0 .. j0+nb), one
// thread per row
__global__ __launch_bounds__(256) void k_chol_panel(SolveArgs A, int j0) {
    __shared__ double L[kCB][kCB + 1];
    __shared__ double invd[kCB];
    if (A.flags[2]) return;
    const int n = A.n;
    const int nb = min(kCB, n - j0);
    double* S = A.S;
    for (int t = threadIdx.x; t < kCB * kCB; t += blockDim.x) {
        const int r = t / kCB, c = t - (t / kCB) * kCB;
        L[r][c] = (r < nb && c <= r) ? S[(size_t)(j0 + r) * n + j0 + c] : 0.0;
    }
    __syncthreads();
    if (threadIdx.x < kCB)
        invd[threadIdx.x] = threadIdx.x < nb ? 1.0 / L[threadIdx.x][threadIdx.x] : 0.0;
    __syncthreads();
    const int i = j0 + nb + blockIdx.x * blockDim.x + threadIdx.x;
    if (i > n) return;
    double* row = S + (size_t)i * n + j0;
    double x[kCB];
#pragma unroll
    for (int k = 0; k < kCB; k++) {
        if (k < nb) {
            double v = row[k];
#pragma unroll
            for (int m = 0; m < k; m++) v -= x[m] * L[k][m];
            x[k] = v * invd[k];
        } else {
            x[k] = 0.0;
        }
    }
#pragma unroll
    for (int k = 0; k < kCB; k++)
        if (k < nb) row[k] = x[k];
}

// trailing S[i][k] -= sum_m L[i][j0+m] L[k][j0+m] for r0 <= k <= i <= n, k < n
// (row n is b; the upper entries of the diagonal tiles are updated too and
// never read), r0 = j0 + nb; one workgroup per lower 64 x 64 tile of the
// (n + 1 - r0)-row trailing block, 4 x 4 outputs per thread.
__global__ __launch_bounds__(256) void k_chol_syrk(SolveArgs A, int j0) {
    __shared__ double Ai[64][kCB + 1], Bk[64][kCB + 1];
    if (A.flags[2]) return;
    const int n = A.n;
    const int nb = min(kCB, n - j0);
    const int r0 = j0 + nb;
    // blockIdx.x -> lower tile (ti, tk), tk <= ti
    int ti = (int)((sqrtf(8.0f * (float)blockIdx.x + 1.0f) - 1.0f) * 0.5f);
    while (ti * (ti + 1) / 2 > (int)blockIdx.x) ti--;
    while ((ti + 1) * (ti + 2) / 2 <= (int)blockIdx.x) ti++;
    const int tk = (int)blockIdx.x - ti * (ti + 1) / 2;
    const int ri = r0 + ti * 64, rk = r0 + tk * 64;
    if (rk >= n) return;  // a column tile made only of b's row
    double* S = A.S;
    for (int t = threadIdx.x; t < 64 * kCB; t += blockDim.x) {
        const int r = t / kCB, m = t - (t / kCB) * kCB;
        Ai[r][m] = (ri + r <= n && m < nb) ? S[(size_t)(ri + r) * n + j0 + m] : 0.0;
        Bk[r][m] = (rk + r < n && m < nb) ? S[(size_t)(rk + r) * n + j0 + m] : 0.0;
    }
    __syncthreads();
    const int ty = threadIdx.x >> 4, tx = threadIdx.x & 15;
    double acc[4][4] = {};
    for (int m = 0; m < nb; m++) {
        double a[4], b[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            a[u] = Ai[ty + 16 * u][m];
            b[u] = Bk[tx + 16 * u][m];
        }
#pragma unroll
        for (int u = 0; u < 4; u++)
#pragma unroll
            for (int v = 0; v < 4; v++) acc[u][v] += a[u] * b[v];
    }
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int i = ri + ty + 16 * u;
        if (i > n) continue;
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int k = rk + tx + 16 * v;
            if (k < n) S[(size_t)i * n + k] -= acc[u][v];
        }
    }
}

// L^T x = z with L in the lower triangle of S (leading dimension n), z -> x
// in y (LDS), one workgroup, blocks of kCB rows from the bottom. Per block,
// wave 0 holds the block's columns of L in registers (loaded up front, so the
// sequential substitution only waits on readlane broadcasts), then all
// threads subtract the block's contribution from the entries above it,
// reading L by rows (coalesced over the threads).
__device__ void back_solve_blocked(const double* __restrict__ S, double* y, int n) {
    const int tid = threadIdx.x;
    for (int j0 = ((n - 1) / kCB) * kCB; j0 >= 0; j0 -= kCB) {  // backward: L^T x = z
        const int jb = min(kCB, n - j0);
        if (tid < 64) {
            // lane c holds column c of the block: L[j0+k][j0+c] for k >= c
            const int lane = tid, lc = min(lane, jb - 1);
            double d[kCB];
#pragma unroll
            for (int k = 0; k < kCB; k++) d[k] = k < jb ? S[(size_t)(j0 + k) * n + j0 + lc] : 0.0;
            double dl = 1.0;
#pragma unroll
            for (int k = 0; k < kCB; k++)
                if (k == lc) dl = d[k];
            const double invl = 1.0 / dl;
            double v = lane < jb ? y[j0 + lane] : 0.0;
#pragma unroll
            for (int k = kCB - 1; k >= 0; k--) {
                if (k < jb) {
                    const double xk = bcast(v * invl, k);
                    if (lane == k) v = xk;
                    else if (lane < k) v -= d[k] * xk;
                }
            }
            if (lane < jb) y[j0 + lane] = v;
        }
        __syncthreads();
        for (int i = tid; i < j0; i += blockDim.x) {
            double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
            int m = 0;
            for (; m + 4 <= jb; m += 4) {
                s0 += S[(size_t)(j0 + m) * n + i] * y[j0 + m];
                s1 += S[(size_t)(j0 + m + 1) * n + i] * y[j0 + m + 1];
                s2 += S[(size_t)(j0 + m + 2) * n + i] * y[j0 + m + 2];
                s3 += S[(size_t)(j0 + m + 3) * n + i] * y[j0 + m + 3];
            }
            for (; m < jb; m++) s0 += S[(size_t)(j0 + m) * n + i] * y[j0 + m];
            y[i] -= (s0 + s1) + (s2 + s3);
        }
        __syncthreads();
    }
}

constexpr int kFinishWG = 512;
__global__ __launch_bounds__(kFinishWG) void k_chol_finish(SolveArgs A) {
    extern __shared__ double smem[];
    const int n = A.n;
    double* b = smem;
    const bool ok = A.flags[2] == 0;
    const int halt_word = solve_halt_word(A);
    for (int t = threadIdx.x; t < n; t += blockDim.x) b[t] = A.S[(size_t)n * n + t];  // z
    __syncthreads();
    if (ok) back_solve_blocked(A.S, b, n);
    __syncthreads();
    finish_solve(A, b, ok, halt_word, A.poses + 7 * A.t0);
}

int solve_blocked(const SolveArgs& A, hipStream_t stream) {
    const int n = A.n;
    hipLaunchKernelGGL(k_chol_init, dim3(std::min(1024, (n * (n + 1) + 255) / 256)), dim3(256),
                       0, stream, A);
    for (int j0 = 0; j0 < n; j0 += kCB) {
        hipLaunchKernelGGL(k_chol_diag, dim3(1), dim3(64), 0, stream, A, j0);
        const int rows = n + 1 - std::min(n, j0 + kCB);  // trailing rows, b's included
        hipLaunchKernelGGL(k_chol_panel, dim3((rows + 255) / 256), dim3(256), 0, stream, A, j0);
        if (rows <= 1) break;
        const int T = (rows + 63) / 64;
        hipLaunchKernelGGL(k_chol_syrk, dim3(T * (T + 1) / 2), dim3(256), 0, stream, A, j0);
    }
    hipLaunchKernelGGL(k_chol_finish, dim3(1), dim3(kFinishWG), (size_t)n * sizeof(double),
                       stream, A);
    SLK_HIP(hipGetLastError());
    return SLK_OK;
}

// ------------------------------------------------------ k_ba_backsub ----
// EvT6x1 + accum + depth_update (ba.cuh:762-783) fused per keyframe pixel.
__global__ __launch_bounds__(256) void k_ba_backsub(PlanDev plan, const double* __restrict__ E,
                                                    const double* __restrict__ Q,
                                                    const double* __restrict__ Wv,
                                                    const float* __restrict__ dx,
                                                    const int* __restrict__ flags,
                                                    float* __restrict__ disps, int HW) {
    if (flags[0]) return;
    const int kc = blockIdx.y;
    const int k = blockIdx.x * blockDim.x + threadIdx.x;
    if (k >= HW) return;
    double dw = 0.0;
    for (int r = plan.kf_rptr[kc]; r < plan.kf_rptr[kc + 1]; r++) {
        const int row = plan.kf_rows[r];
        const double* er = E + (size_t)row * 6 * HW + k;
        const float* x = dx + plan.row_pose[row] * 6;
#pragma unroll
        for (int n = 0; n < 6; n++) dw += er[(size_t)n * HW] * (double)x[n];
    }
    const double dz = Q[(size_t)kc * HW + k] * (Wv[(size_t)kc * HW + k] - dw);
    float* d = disps + (size_t)plan.kf_list[kc] * HW + k;
    *d = (float)((double)*d + dz);
}

// ===================================================== fused iteration ====
// Systems whose keyframes have at most kFzMaxSlots E rows each (the
// frontend's windows) run an iteration in three launches, and the E rows
// never reach HBM:
//   k_ba_fz  grid (pixel chunk, keyframe). Optionally first the
//            back-substitution of the previous step (EvT6x1 + depth_update,
//            ba.cuh:762-783), by relinearizing every edge of the keyframe at
//            the poses and depths that step was taken from: dw = sum_e g_e .
//            (dx_j - Adj_e^T dx_i), g_e = w Jz Jj per pixel (the E rows of
//            ba.cuh:139-140, 167-168 regrouped by edge). Then the
//            linearization at the current state: the Hjj/vj partials of every
//            edge as in k_ba_lin_wv, and the keyframe's E rows and w for the
//            chunk's pixels in LDS as [pixel][row], from which the chunk's
//            Schur products Z = [E; w] Q [E; w]^T (EEt6x6 / Ev6x1,
//            ba.cuh:303-372) are formed on fp64 MFMA (v_mfma_f64_16x16x4),
//            each wave over 48 pixels, the four partials added in wave order.
//   k_ba_fz_assemble  one workgroup per block of S and per segment of b: the
//            chunk sums (in chunk order) of the Z entries and edge partials
//            the block needs, then the LM damping.
//   a solve kernel, which also keeps the poses before the step.
// A last k_ba_fz_bs applies the final step's back-substitution. When every
// linearization workgroup fits the CUs at once, the solve and the next
// k_ba_fz share a launch instead (k_ba_fz_step): the linearization
// workgroups rebuild the solved step's E rows while it runs and wait for its
// dx on a flag, so an iteration is two launches (assembly, step).
// E rows ("slots") of a keyframe: its own pose when free (slot 0), then one
// per non-stereo edge whose jj is free, in edge order (two edges to the same
// pose keep separate slots; the assembly adds their products). Row 6 * nslot
// holds w; the rows after it, up to 16 T, are zero.
constexpr int kFzMaxSlots = 7;
constexpr int kFzMaxT = 3;                             // 16-row tiles of [E; w]
constexpr int kFzMaxNT = kFzMaxT * (kFzMaxT + 1) / 2;  // tiles (ti <= tj) kept
constexpr int kFzLd = 16 * kFzMaxT + 9;  // doubles per pixel in LDS (odd: 2-way stores)
constexpr int kFzMaxDst = 32;            // distinct edges feeding one block of S or b
constexpr int kFzMaxCodes = 80;          // contributions to one block of S or b
// A block's assembly record: [0] contributions, [1] distinct edges, then
// (edge, ii, jj) of each edge at kFzRecEdges, then (code, Schur item) of
// each contribution, 5 ints, at kFzRecCodes
constexpr int kFzRecEdges = 2;
constexpr int kFzRecCodes = kFzRecEdges + 3 * kFzMaxDst;
constexpr int kFzRecInts = (kFzRecCodes + 5 * kFzMaxCodes + 63) / 64 * 64;
static_assert(6 * kFzMaxSlots + 1 <= 16 * kFzMaxT, "the slot rows and w fill at most T tiles");
// pixels of a fused workgroup's chunk: half its threads take one pixel each
// in the per-pixel steps, and each wave's lanes hold kFzPPL pixels
constexpr int kFzPx = 192;
constexpr int kFzPPL = kFzPx / 64;
// fused workgroups resident per CU (their LDS takes more than half of a CU's
// 160 KB)
constexpr int kFzWgPerCu = 1;
static_assert(kFzPx <= kLinWG && kFzPx % 64 == 0 && kFzPx % 16 == 0, "chunk shape");
static_assert((3 * kFzMaxNT + kFzMaxNT) * 256 <= kFzPx * kFzLd, "the waves' MFMA tiles fit in xs");

struct FzKf {
    int kf, e0, e1, info;  // edges e0..e1 of the edge table; info = nslot | ri << 8 | T << 12
};
struct FzEdge {
    int e, ix, jx, slot;  // slot of the edge's own E row, -1 for none
};

struct FzArgs {
    const FzKf* kfs;
    const FzEdge* eds;
    const float* target;
    const float* weight;
    const float* poses;
    const float* poses_prev;  // [P][7]: poses t0..t1-1 of the last step's linearization
    float* pose_copy;         // [P][7] or null: k_ba_fz<false, *> copies poses t0..t1-1 here
    const float* intr;
    const float* eta;
    const float* dx;   // [6P] the last step
    // [0]: the last step was rejected (not SPD); [3] a wait gave up (sticky,
    // reported by slk_ba_status); [4] a wait of this call gave up (cleared by
    // the call's first launch); [5] the copy of [4] the next solve reads
    int* flags;
    float* disps;
    double* hpart;  // [M][nch][27]
    double* spart;  // [N_kf][nch][kFzMaxNT][256] Z tiles in MFMA lane order
    int HW, W, nch, t0, t1;
    int npose;     // poses the call's edges and free range refer to (0..npose-1)
    int spin_max;  // polls before a waiting workgroup gives up
};

// Calls of at most this many poses keep all of them in LDS for the
// linearization at the poses after an overlapped step (fixed poses staged
// before the wait, the free ones formed after it), so that no pose is read
// from memory after the flag.
constexpr int kFzLdsPoses = 64;
static_assert(kFzLdsPoses >= kPanelPoses, "the free poses fit the LDS pose array");

__device__ __forceinline__ float ld_coherent(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Relative pose of edge (ix, jx) at the current poses, at the poses after
// this launch's step (pn, which the workgroup formed: every pose when npose
// <= kFzLdsPoses, else poses t0..t1-1, the others not moving), or (prev) at
// the poses of the last step's linearization: only t0..t1-1 moved.
__device__ __forceinline__ void fz_rel(const FzArgs& F, bool prev, int ix, int jx, double* tij,
                                       double* qij, const float* pn = nullptr) {
    if (ix == jx) {
        edge_rel(F.poses, ix, jx, tij, qij);  // stereo constants
        return;
    }
    double ti[3], qi[4], tj[3], qj[4];
    if (pn && F.npose <= kFzLdsPoses) {
        load_pose(pn, ix, ti, qi);
        load_pose(pn, jx, tj, qj);
    } else if (pn) {
        const bool si = ix >= F.t0 && ix < F.t1, sj = jx >= F.t0 && jx < F.t1;
        load_pose(si ? pn : F.poses, si ? ix - F.t0 : ix, ti, qi);
        load_pose(sj ? pn : F.poses, sj ? jx - F.t0 : jx, tj, qj);
    } else {
        const bool pi = prev && ix >= F.t0 && ix < F.t1, pj = prev && jx >= F.t0 && jx < F.t1;
        load_pose(pi ? F.poses_prev : F.poses, pi ? ix - F.t0 : ix, ti, qi);
        load_pose(pj ? F.poses_prev : F.poses, pj ? jx - F.t0 : jx, tj, qj);
    }
    rel_se3(ti, qi, tj, qj, tij, qij);
}

typedef double fz_d4 __attribute__((ext_vector_type(4)));

// Z = [E; w] Q [E; w]^T over this wave's 64 pixels of xs ([pixel][row]),
// for the T (T + 1) / 2 upper 16 x 16 tiles: operand A = rows 16 ti + (l %
// 16) of pixel l / 16 of a 4-pixel step, B = Q times rows 16 tj + (l % 16);
// then the wave's tiles go to xs as [wave][tile][256] (lane * 4 + r), which
// overwrites the rows: a barrier separates every wave's reads from the first
// write.
template <int T>
__device__ __forceinline__ void fz_schur_tiles(double* xs, const double* qs, int wave, int lane) {
    constexpr int NT = T * (T + 1) / 2;
    fz_d4 z[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) z[t] = fz_d4{0.0, 0.0, 0.0, 0.0};
    const int i16 = lane & 15, kg = lane >> 4;
#pragma unroll
    for (int ks = 0; ks < kFzPx / 16; ks++) {
        const int kp = wave * (kFzPx / 4) + ks * 4 + kg;
        const double q = qs[kp];
        const double* xr = xs + kp * kFzLd + i16;
        double a[T], b[T];
#pragma unroll
        for (int t = 0; t < T; t++) {
            a[t] = xr[16 * t];
            b[t] = a[t] * q;
        }
        int tt = 0;
#pragma unroll
        for (int tj = 0; tj < T; tj++)
#pragma unroll
            for (int ti = 0; ti <= tj; ti++, tt++)
                z[tt] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[ti], b[tj], z[tt], 0, 0, 0);
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) xs[(wave * kFzMaxNT + t) * 256 + lane * 4 + r] = z[t][r];
}

// LDS of a fused linearization workgroup.
struct FzLds {
    double xs[kFzPx * kFzLd];        // [pixel][row]; then the MFMA partials
    double cw[2][kLinWaves][kFzPx];  // per-wave sums (C, w)
    double qs[kFzPx];
    double dxr[6 * kFzMaxSlots];  // the last step's dx, by slot row
    int spose[kFzMaxSlots];       // the pose of each slot
    // the poses after the overlapped launch's step: all of them when npose <=
    // kFzLdsPoses, else poses t0..t1-1 (from index 0)
    float pnew[kFzLdsPoses * 7];
    int wait_state;
};

// What the first pass over a wave's first edge read, reused by the second:
// its targets and weights, and (rel) its relative pose at the current poses.
struct FzCache {
    bool valid, rel;
    int ix, jx;
    float tgu[kFzPPL], tgv[kFzPPL], wtu[kFzPPL], wtv[kFzPPL];
    double tn[3], qn[4];
};

// One pass over the keyframe's edges for the chunk's pixels, at the poses of
// the last step (kPrev: the rows that step's back-substitution needs) or at
// the current poses (the Hjj/vj partials of every edge to hpart as well).
// Leaves L.xs with the keyframe's E rows and w ([pixel][row]: the slots'
// rows, own row in slot 0 when the keyframe's pose is free, w at row
// 6 nslot, zeros up to 16 T) and L.qs with Q (damping_Q_kernel with
// ep = 1e-7, ba.cuh:266-281, 701-702; eta_px: eta of the thread's pixel).
// Ends with a barrier.
template <bool kPrev>
__device__ __forceinline__ void fz_pass(const FzArgs& F, const FzKf& K, FzLds& L, int chunk,
                                        const int (&kpx)[kFzPPL], const bool (&vpx)[kFzPPL],
                                        const double (&dsp)[kFzPPL], double eta_px,
                                        FzCache& cache, const float* pn = nullptr) {
    const int nslot = K.info & 0xff, ri = (K.info >> 8) & 1, T = K.info >> 12;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, tid = threadIdx.x;
    const int HW = F.HW;
    const double fx = F.intr[0], fy = F.intr[1], cx = F.intr[2], cy = F.intr[3];
    double* xs = L.xs;
    if (tid < kFzPx) {
        // rows past the slots and w (and every row of a pixel past HW) are zero
        const int k = chunk * kFzPx + tid;
        double* xr = xs + tid * kFzLd;
        for (int r = k < HW ? 6 * nslot + 1 : 0; r < 16 * T; r++) xr[r] = 0.0;
    }
    double er[kFzPPL][6];  // this lane's pixels: -sum Adj g over the wave's edges
    double cp[kFzPPL], wp[kFzPPL];
#pragma unroll
    for (int s = 0; s < kFzPPL; s++) {
        cp[s] = wp[s] = 0.0;
#pragma unroll
        for (int n = 0; n < 6; n++) er[s][n] = 0.0;
    }
    for (int ei = K.e0 + wave; ei < K.e1; ei += kLinWaves) {
        const bool first = ei == K.e0 + wave;  // uniform
        const FzEdge E = F.eds[ei];
        const bool stereo = E.ix == E.jx;
        double tij[3], qij[4];
        if (!kPrev && first && cache.rel) {
#pragma unroll
            for (int m = 0; m < 3; m++) tij[m] = cache.tn[m];
#pragma unroll
            for (int m = 0; m < 4; m++) qij[m] = cache.qn[m];
        } else {
            fz_rel(F, kPrev, E.ix, E.jx, tij, qij, pn);
        }
        float tgu[kFzPPL], tgv[kFzPPL], wtu[kFzPPL], wtv[kFzPPL];
        if (!kPrev && first && cache.valid) {
#pragma unroll
            for (int s = 0; s < kFzPPL; s++) {
                tgu[s] = cache.tgu[s];
                tgv[s] = cache.tgv[s];
                wtu[s] = cache.wtu[s];
                wtv[s] = cache.wtv[s];
            }
        } else {
#pragma unroll
            for (int s = 0; s < kFzPPL; s++) {
                const size_t base = (size_t)E.e * 2 * HW + (vpx[s] ? kpx[s] : 0);
                tgu[s] = F.target[base];
                tgv[s] = F.target[base + HW];
                wtu[s] = F.weight[base];
                wtv[s] = F.weight[base + HW];
            }
            if (kPrev && first) {
                cache.valid = true;
                cache.ix = E.ix;
                cache.jx = E.jx;
#pragma unroll
                for (int s = 0; s < kFzPPL; s++) {
                    cache.tgu[s] = tgu[s];
                    cache.tgv[s] = tgv[s];
                    cache.wtu[s] = wtu[s];
                    cache.wtv[s] = wtv[s];
                }
            }
        }
        double acc[kNJ];
#pragma unroll
        for (int n = 0; n < kNJ; n++) acc[n] = 0.0;
#pragma unroll
        for (int s = 0; s < kFzPPL; s++) {
            if (!vpx[s]) continue;
            const int px = s * 64 + lane;
            Lin Ln;
            lin_pixel(tij, qij, fx, fy, cx, cy, kpx[s], F.W, dsp[s], (double)tgu[s],
                      (double)tgv[s], (double)wtu[s], (double)wtv[s], Ln);
            if (!kPrev) accum_hjj(Ln, stereo, acc);
            cp[s] += Ln.w[0] * Ln.Jz[0] * Ln.Jz[0] + Ln.w[1] * Ln.Jz[1] * Ln.Jz[1];
            wp[s] += Ln.w[0] * Ln.r[0] * Ln.Jz[0] + Ln.w[1] * Ln.r[1] * Ln.Jz[1];
            if (!stereo) {  // a stereo edge adds nothing to E
                const double a0 = Ln.w[0] * Ln.Jz[0], a1 = Ln.w[1] * Ln.Jz[1];
                double g[6];
#pragma unroll
                for (int n = 0; n < 6; n++) g[n] = a0 * Ln.Jj[0][n] + a1 * Ln.Jj[1][n];
                if (E.slot >= 0) {
                    double* xr = xs + px * kFzLd + 6 * E.slot;
#pragma unroll
                    for (int n = 0; n < 6; n++) xr[n] = g[n];
                }
                if (ri) {  // Ji-row contribution -Adj g (ba.cuh:139-140)
                    double gi[6];
                    adj_se3(tij, qij, g, gi);
#pragma unroll
                    for (int n = 0; n < 6; n++) er[s][n] -= gi[n];
                }
            }
        }
        if (!kPrev) {
            int rbase, rvalid;
            wave_reduce_scatter(acc, lane, rbase, rvalid);
            double* hp = F.hpart + ((size_t)E.e * F.nch + chunk) * kNJ;
#pragma unroll
            for (int q = 0; q < RsCounts<kNJ>::c6; q++)
                if (q < rvalid) hp[rbase + q] = acc[q];
        }
    }
#pragma unroll
    for (int s = 0; s < kFzPPL; s++) {
        const int px = s * 64 + lane;
        L.cw[0][wave][px] = cp[s];
        L.cw[1][wave][px] = wp[s];
    }
    // the keyframe's own row (slot 0): the waves' parts added in wave order,
    // from per-wave copies in the columns past the tiles when two tiles hold
    // the rows, else one wave after another
    constexpr int kErCol = 32;
    static_assert(kErCol + 6 * kLinWaves <= kFzLd, "four 6-row copies fit past two tiles");
    const bool er_cols = T <= 2;  // uniform
    if (ri && er_cols) {
#pragma unroll
        for (int s = 0; s < kFzPPL; s++) {
            double* xr = xs + (s * 64 + lane) * kFzLd + kErCol + 6 * wave;
#pragma unroll
            for (int n = 0; n < 6; n++) xr[n] = er[s][n];
        }
    } else if (ri) {
        for (int v = 0; v < kLinWaves; v++) {
            __syncthreads();
            if (wave == v) {
#pragma unroll
                for (int s = 0; s < kFzPPL; s++) {
                    if (!vpx[s]) continue;
                    double* xr = xs + (s * 64 + lane) * kFzLd;
#pragma unroll
                    for (int n = 0; n < 6; n++) xr[n] = (v == 0 ? 0.0 : xr[n]) + er[s][n];
                }
            }
        }
    }
    __syncthreads();
    if (tid < kFzPx) {
        const int k = chunk * kFzPx + tid;
        double q = 0.0;
        double* xr = xs + tid * kFzLd;
        if (k < HW) {
            double c = 0.0, w = 0.0;
#pragma unroll
            for (int v = 0; v < kLinWaves; v++) {
                c += L.cw[0][v][tid];
                w += L.cw[1][v][tid];
            }
            q = 1.0 / (c + 0.2 * eta_px + 1e-7);
            xr[6 * nslot] = w;
            if (ri && er_cols) {
#pragma unroll
                for (int n = 0; n < 6; n++) {
                    double t = xr[kErCol + n];
#pragma unroll
                    for (int v = 1; v < kLinWaves; v++) t += xr[kErCol + 6 * v + n];
                    xr[n] = t;
                }
            }
        }
        L.qs[tid] = q;
    }
    __syncthreads();
}

// The overlapped step's handshake: the assembly launch before it clears
// *ready, the step launch's solve workgroup stores 1 there once dx, the flags
// and the poses are written, and a linearization workgroup waits for it
// (thread 0 polls, bounded: after F.spin_max polls, kFzSpinMax unless
// slk_ba_set_wait_limit set another, or at once for a limit of 0, the
// workgroup gives up: it sets flags[3] (reported by slk_ba_status) and
// flags[4], and writes nothing more, so its chunk's depths miss that step's
// update. The next assembly launch copies flags[4] to flags[5], and every
// later solve of the call then takes no step (finish_solve), so the rest of
// the call changes neither poses nor depths.)
constexpr int kFzSpinMax = 1 << 18;

struct FzWait {
    int* ready;  // null: no wait (the step's dx is known at launch)
};

// The depth update of the last step when its dx is known at launch (a
// rejected step leaves the depths as they are): per edge the step's
// projection dl = dx_j - Adj^T dx_i (lane c < 6 forms component c), then per
// pixel dw = sum_e g_e . dl_e, g_e = w Jz Jj at the last step's poses and
// depths (EvT6x1 + depth_update, ba.cuh:762-783); dsp receives the new
// depths. The first edge of each wave goes to `cache` (with its relative
// pose at the current poses when want_rel). LDS: cwd, cw0, cw1 [kLinWaves]
// [kFzPx] and qs [kFzPx] doubles; ends with a barrier.
__device__ __forceinline__ void fz_bs_direct(const FzArgs& F, const FzKf& K, int chunk,
                                             const int (&kpx)[kFzPPL],
                                             const bool (&vpx)[kFzPPL],
                                             double (&dsp)[kFzPPL], double eta_px,
                                             FzCache& cache, bool want_rel, double* cwd,
                                             double* cw0, double* cw1, double* qs) {
    const int ri = (K.info >> 8) & 1;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, tid = threadIdx.x;
    const int HW = F.HW;
    const int kown = chunk * kFzPx + tid;
    const bool mine = tid < kFzPx && kown < HW;  // this thread's pixel, if any
    double dwp[kFzPPL], cp[kFzPPL], wp[kFzPPL];
#pragma unroll
    for (int s = 0; s < kFzPPL; s++) dwp[s] = cp[s] = wp[s] = 0.0;
    const double fx = F.intr[0], fy = F.intr[1], cx = F.intr[2], cy = F.intr[3];
    for (int ei = K.e0 + wave; ei < K.e1; ei += kLinWaves) {
        const FzEdge E = F.eds[ei];
        const bool stereo = E.ix == E.jx;
        const bool first = ei == K.e0 + wave;  // uniform
        double tij[3], qij[4];
        fz_rel(F, true, E.ix, E.jx, tij, qij);
        if (want_rel && first) {  // the linearization's relative pose of this edge
            fz_rel(F, false, E.ix, E.jx, cache.tn, cache.qn);
            cache.rel = true;
        }
        double dl[6] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
        if (!stereo) {
            if (E.slot >= 0)
#pragma unroll
                for (int n = 0; n < 6; n++) dl[n] = (double)F.dx[(E.jx - F.t0) * 6 + n];
            if (ri) {  // lane c < 6: (Adj^T dx_i)[c] = adj_se3(e_c) . dx_i
                double u[6], y[6], t = 0.0;
#pragma unroll
                for (int m = 0; m < 6; m++) u[m] = m == lane ? 1.0 : 0.0;
                adj_se3(tij, qij, u, y);
#pragma unroll
                for (int m = 0; m < 6; m++) t += y[m] * (double)F.dx[(E.ix - F.t0) * 6 + m];
#pragma unroll
                for (int c = 0; c < 6; c++) dl[c] -= __shfl(t, c);
            }
        }
        float tgu[kFzPPL], tgv[kFzPPL], wtu[kFzPPL], wtv[kFzPPL];
#pragma unroll
        for (int s = 0; s < kFzPPL; s++) {
            const size_t base = (size_t)E.e * 2 * HW + (vpx[s] ? kpx[s] : 0);
            tgu[s] = F.target[base];
            tgv[s] = F.target[base + HW];
            wtu[s] = F.weight[base];
            wtv[s] = F.weight[base + HW];
        }
        if (first) {
            cache.valid = true;
            cache.ix = E.ix;
            cache.jx = E.jx;
#pragma unroll
            for (int s = 0; s < kFzPPL; s++) {
                cache.tgu[s] = tgu[s];
                cache.tgv[s] = tgv[s];
                cache.wtu[s] = wtu[s];
                cache.wtv[s] = wtv[s];
            }
        }
#pragma unroll
        for (int s = 0; s < kFzPPL; s++) {
            if (!vpx[s]) continue;
            Lin Ln;
            lin_pixel(tij, qij, fx, fy, cx, cy, kpx[s], F.W, dsp[s], (double)tgu[s],
                      (double)tgv[s], (double)wtu[s], (double)wtv[s], Ln);
            cp[s] += Ln.w[0] * Ln.Jz[0] * Ln.Jz[0] + Ln.w[1] * Ln.Jz[1] * Ln.Jz[1];
            wp[s] += Ln.w[0] * Ln.r[0] * Ln.Jz[0] + Ln.w[1] * Ln.r[1] * Ln.Jz[1];
            if (!stereo) {
                const double a0 = Ln.w[0] * Ln.Jz[0], a1 = Ln.w[1] * Ln.Jz[1];
                double t = 0.0;
#pragma unroll
                for (int n = 0; n < 6; n++)
                    t += (a0 * Ln.Jj[0][n] + a1 * Ln.Jj[1][n]) * dl[n];
                dwp[s] += t;
            }
        }
    }
#pragma unroll
    for (int s = 0; s < kFzPPL; s++) {
        const int px = s * 64 + lane;
        cwd[wave * kFzPx + px] = dwp[s];
        cw0[wave * kFzPx + px] = cp[s];
        cw1[wave * kFzPx + px] = wp[s];
    }
    __syncthreads();
    if (mine) {
        double dw = 0.0, c = 0.0, w = 0.0;
#pragma unroll
        for (int v = 0; v < kLinWaves; v++) {
            dw += cwd[v * kFzPx + tid];
            c += cw0[v * kFzPx + tid];
            w += cw1[v * kFzPx + tid];
        }
        // damping_Q_kernel (ep = 1e-7) and depth_update_kernel
        const double q = 1.0 / (c + 0.2 * eta_px + 1e-7);
        double own = dsp[0];
#pragma unroll
        for (int s = 1; s < kFzPPL; s++)
            if (s == wave) own = dsp[s];
        const float dn = (float)(own + q * (w - dw));
        F.disps[(size_t)K.kf * HW + kown] = dn;
        qs[tid] = (double)dn;
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < kFzPPL; s++)
        if (vpx[s]) dsp[s] = qs[s * 64 + lane];
    __syncthreads();  // the caller's next use of this LDS
}

// k_ba_fz's work for one (pixel chunk, keyframe): with kBs first the depth
// update of the last step, dz = Q (w - E^T dx) (EvT6x1 + depth_update,
// ba.cuh:762-783) from that step's E rows, Q and w recomputed at its poses
// and depths (with a wait for dx when `wait.ready` is set); with kLin then the
// linearization at the current state and the Schur tiles of the chunk.
template <bool kBs, bool kLin>
__device__ __forceinline__ void fz_body(const FzArgs& F, FzLds& L, int chunk, int kc,
                                        FzWait wait) {
    const FzKf K = F.kfs[kc];
    const int nslot = K.info & 0xff, ri = (K.info >> 8) & 1, T = K.info >> 12;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, tid = threadIdx.x;
    const int HW = F.HW;
    int kpx[kFzPPL];
    bool vpx[kFzPPL];
    double dsp[kFzPPL];
#pragma unroll
    for (int s = 0; s < kFzPPL; s++) {
        kpx[s] = chunk * kFzPx + s * 64 + lane;
        vpx[s] = kpx[s] < HW;
        dsp[s] = vpx[s] ? (double)F.disps[(size_t)K.kf * HW + kpx[s]] : 1.0;
    }
    FzCache cache;
    cache.valid = cache.rel = false;
    const int kown = chunk * kFzPx + tid;  // the pixel of the per-pixel steps
    const bool mine = tid < kFzPx && kown < HW;
    const double eta_px = mine ? (double)F.eta[(size_t)K.kf * HW + kown] : 0.0;
    const float* pn = nullptr;  // L.pnew once it holds the poses after this launch's step
    if (kBs && !wait.ready && F.flags[0] == 0) {  // uniform
        // (fz_bs_direct's computation, written out here: called as a
        // function, it changed this kernel's register allocation and cost
        // 2-6 us per launch)
        // dx is known at launch (a rejected step leaves the depths as they
        // are): per edge the step's projection dl = dx_j - Adj^T dx_i (lane
        // c < 6 forms component c), then per pixel dw = sum_e g_e . dl_e,
        // g_e = w Jz Jj at the last step's poses and depths
        double* cwd = L.xs;  // [kLinWaves][kFzPx] per-wave sums of dw
        double dwp[kFzPPL], cp[kFzPPL], wp[kFzPPL];
#pragma unroll
        for (int s = 0; s < kFzPPL; s++) dwp[s] = cp[s] = wp[s] = 0.0;
        const double fx = F.intr[0], fy = F.intr[1], cx = F.intr[2], cy = F.intr[3];
        for (int ei = K.e0 + wave; ei < K.e1; ei += kLinWaves) {
            const FzEdge E = F.eds[ei];
            const bool stereo = E.ix == E.jx;
            const bool first = ei == K.e0 + wave;  // uniform
            double tij[3], qij[4];
            fz_rel(F, true, E.ix, E.jx, tij, qij);
            if (kLin && first) {  // the linearization's relative pose of this edge
                fz_rel(F, false, E.ix, E.jx, cache.tn, cache.qn);
                cache.rel = true;
            }
            double dl[6] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
            if (!stereo) {
                if (E.slot >= 0)
#pragma unroll
                    for (int n = 0; n < 6; n++) dl[n] = (double)F.dx[(E.jx - F.t0) * 6 + n];
                if (ri) {  // lane c < 6: (Adj^T dx_i)[c] = adj_se3(e_c) . dx_i
                    double u[6], y[6], t = 0.0;
#pragma unroll
                    for (int m = 0; m < 6; m++) u[m] = m == lane ? 1.0 : 0.0;
                    adj_se3(tij, qij, u, y);
#pragma unroll
                    for (int m = 0; m < 6; m++) t += y[m] * (double)F.dx[(E.ix - F.t0) * 6 + m];
#pragma unroll
                    for (int c = 0; c < 6; c++) dl[c] -= __shfl(t, c);
                }
            }
            float tgu[kFzPPL], tgv[kFzPPL], wtu[kFzPPL], wtv[kFzPPL];
#pragma unroll
            for (int s = 0; s < kFzPPL; s++) {
                const size_t base = (size_t)E.e * 2 * HW + (vpx[s] ? kpx[s] : 0);
                tgu[s] = F.target[base];
                tgv[s] = F.target[base + HW];
                wtu[s] = F.weight[base];
                wtv[s] = F.weight[base + HW];
            }
            if (first) {
                cache.valid = true;
                cache.ix = E.ix;
                cache.jx = E.jx;
#pragma unroll
                for (int s = 0; s < kFzPPL; s++) {
                    cache.tgu[s] = tgu[s];
                    cache.tgv[s] = tgv[s];
                    cache.wtu[s] = wtu[s];
                    cache.wtv[s] = wtv[s];
                }
            }
#pragma unroll
            for (int s = 0; s < kFzPPL; s++) {
                if (!vpx[s]) continue;
                Lin Ln;
                lin_pixel(tij, qij, fx, fy, cx, cy, kpx[s], F.W, dsp[s], (double)tgu[s],
                          (double)tgv[s], (double)wtu[s], (double)wtv[s], Ln);
                cp[s] += Ln.w[0] * Ln.Jz[0] * Ln.Jz[0] + Ln.w[1] * Ln.Jz[1] * Ln.Jz[1];
                wp[s] += Ln.w[0] * Ln.r[0] * Ln.Jz[0] + Ln.w[1] * Ln.r[1] * Ln.Jz[1];
                if (!stereo) {
                    const double a0 = Ln.w[0] * Ln.Jz[0], a1 = Ln.w[1] * Ln.Jz[1];
                    double t = 0.0;
#pragma unroll
                    for (int n = 0; n < 6; n++)
                        t += (a0 * Ln.Jj[0][n] + a1 * Ln.Jj[1][n]) * dl[n];
                    dwp[s] += t;
                }
            }
        }
#pragma unroll
        for (int s = 0; s < kFzPPL; s++) {
            const int px = s * 64 + lane;
            cwd[wave * kFzPx + px] = dwp[s];
            L.cw[0][wave][px] = cp[s];
            L.cw[1][wave][px] = wp[s];
        }
        __syncthreads();
        if (mine) {
            double dw = 0.0, c = 0.0, w = 0.0;
#pragma unroll
            for (int v = 0; v < kLinWaves; v++) {
                dw += cwd[v * kFzPx + tid];
                c += L.cw[0][v][tid];
                w += L.cw[1][v][tid];
            }
            // damping_Q_kernel (ep = 1e-7) and depth_update_kernel
            const double q = 1.0 / (c + 0.2 * eta_px + 1e-7);
            double own = dsp[0];
#pragma unroll
            for (int s = 1; s < kFzPPL; s++)
                if (s == wave) own = dsp[s];
            const float dn = (float)(own + q * (w - dw));
            F.disps[(size_t)K.kf * HW + kown] = dn;
            L.qs[tid] = (double)dn;
        }
        __syncthreads();
#pragma unroll
        for (int s = 0; s < kFzPPL; s++)
            if (vpx[s]) dsp[s] = L.qs[s * 64 + lane];
        __syncthreads();  // qs and xs are the linearization's next
    } else if (kBs && wait.ready) {  // uniform
        // the pose of each slot: the keyframe's for slot 0 when free, else
        // the jj of the edge that owns it (ordered by the pass's barriers)
        for (int ei = K.e0 + tid; ei < K.e1; ei += kLinWG) {
            const FzEdge E = F.eds[ei];
            if (E.slot >= 0) L.spose[E.slot] = E.jx;
        }
        if (ri && tid == 0) L.spose[0] = K.kf;
        // the poses that do not move, for the linearization after the wait
        // (the free ones' entries are replaced then; the pass's barriers
        // order these writes)
        const bool lds_all = kLin && F.npose <= kFzLdsPoses;  // uniform
        if (lds_all)
            for (int i = tid; i < F.npose * 7; i += kLinWG) L.pnew[i] = F.poses[i];
        fz_pass<true>(F, K, L, chunk, kpx, vpx, dsp, eta_px, cache);
        if (wait.ready) {
            if (tid == 0) {
                int st = F.spin_max > 0 ? 1 : 0;  // a limit of 0 gives up without a poll
                for (int n = 0; st && __hip_atomic_load(wait.ready, __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_AGENT) == 0;
                     n++) {
                    if (n >= F.spin_max) {
                        st = 0;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(2);
                }
                L.wait_state = st;
            }
            __syncthreads();
            if (!L.wait_state) {  // uniform
                if (tid == 0) {
                    F.flags[3] = 1;
                    F.flags[4] = 1;
                }
                return;
            }
            // What the solve wrote (the status, dx) is read from
            // here on with device-coherent loads (agent scope, relaxed),
            // issued after the flag was seen and a workgroup barrier: the
            // solve's release fence wrote them back before its flag store,
            // and these loads bypass the caches that could hold older
            // copies, so no cache of this workgroup needs invalidating. (An
            // agent-scope acquire fence here would invalidate this XCD's L2
            // as well, and the next step's input loads measured ~4.5 us
            // slower after it.)
        }
        // the status and dx by slot row (slot poses are free poses)
        const int r6 = nslot > 0 ? min(tid, 6 * nslot - 1) : 0;
        const int dxi = nslot > 0 ? (L.spose[r6 / 6] - F.t0) * 6 + r6 % 6 : 0;
        const int okv = __hip_atomic_load(F.flags, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const float dxf = ld_coherent(F.dx + dxi);
        const bool ok = okv == 0;
        if (kLin) {
            // the free poses after the step, one thread each, formed as the
            // solve forms them (step_pose, from the poses this step started
            // at and its dx) rather than read after its retraction; a
            // rejected or halted step leaves them as they were
            for (int k = tid; k < F.t1 - F.t0; k += kLinWG) {
                const float* p7 = F.poses_prev + k * 7;
                float d6[6], out[7];
                // (loaded unconditionally, beside the status: a load under
                // `ok` would wait for the status load first)
#pragma unroll
                for (int m = 0; m < 6; m++) d6[m] = ld_coherent(F.dx + k * 6 + m);
#pragma unroll
                for (int m = 0; m < 6; m++) d6[m] = ok ? d6[m] : 0.0f;
                if (ok)
                    step_pose(p7, d6, out);
                else
#pragma unroll
                    for (int m = 0; m < 7; m++) out[m] = p7[m];
                float* dst = L.pnew + (lds_all ? (F.t0 + k) * 7 : k * 7);
#pragma unroll
                for (int m = 0; m < 7; m++) dst[m] = out[m];
            }
            pn = L.pnew;
        }
        if (tid < 6 * nslot) L.dxr[tid] = (double)dxf;
        __syncthreads();
        if (kLin && cache.valid) {  // the wave's first edge at the poses after the step
            fz_rel(F, false, cache.ix, cache.jx, cache.tn, cache.qn, pn);
            cache.rel = true;
        }
        if (ok) {  // uniform
            double own = dsp[0];  // the depth of pixel kown (lane's pixel of s = wave)
#pragma unroll
            for (int s = 1; s < kFzPPL; s++)
                if (s == wave) own = dsp[s];
            if (mine) {
                const double* xr = L.xs + tid * kFzLd;
                double dw = 0.0;
                for (int sl = 0; sl < nslot; sl++)
#pragma unroll
                    for (int m = 0; m < 6; m++) dw += xr[6 * sl + m] * L.dxr[6 * sl + m];
                const float dn = (float)(own + L.qs[tid] * (xr[6 * nslot] - dw));
                F.disps[(size_t)K.kf * HW + kown] = dn;
                L.cw[0][0][tid] = (double)dn;
            }
            __syncthreads();
#pragma unroll
            for (int s = 0; s < kFzPPL; s++)
                if (vpx[s]) dsp[s] = L.cw[0][0][s * 64 + lane];
        }
    }
    if (!kLin) return;
    fz_pass<false>(F, K, L, chunk, kpx, vpx, dsp, eta_px, cache, pn);
    if (T == 1)
        fz_schur_tiles<1>(L.xs, L.qs, wave, lane);
    else if (T == 2)
        fz_schur_tiles<2>(L.xs, L.qs, wave, lane);
    else
        fz_schur_tiles<3>(L.xs, L.qs, wave, lane);
    __syncthreads();
    const int nt = T * (T + 1) / 2;
    const double* red = L.xs;
    double* sp = F.spart + (size_t)(kc * F.nch + chunk) * kFzMaxNT * 256;
    for (int idx = tid; idx < nt * 256; idx += kLinWG) {
        double v = red[idx];
#pragma unroll
        for (int w = 1; w < kLinWaves; w++) v += red[w * kFzMaxNT * 256 + idx];
        sp[idx] = v;
    }
}

template <bool kBs, bool kLin>
__global__ __launch_bounds__(kLinWG, kFzWgPerCu) void k_ba_fz(FzArgs F) {
    __shared__ FzLds L;
    if (!kBs && F.pose_copy && blockIdx.x == 0 && blockIdx.y == 0) {
        // the first launch of an overlapped call: the poses its first step
        // starts from, and no wait of this call has given up yet
        for (int t = threadIdx.x; t < (F.t1 - F.t0) * 7; t += kLinWG)
            F.pose_copy[t] = F.poses[F.t0 * 7 + t];
        if (threadIdx.x == 0) {
            F.flags[4] = 0;
            F.flags[5] = 0;
        }
    }
    fz_body<kBs, kLin>(F, L, blockIdx.x, blockIdx.y, FzWait{nullptr});
}

// The last step's depth update alone (the launch after the final solve of a
// fused iteration that did not overlap its steps): fz_bs_direct with 26 KB
// of LDS, so several workgroups share a CU.
struct FzBsLds {
    double cwd[kLinWaves * kFzPx];
    double cw0[kLinWaves * kFzPx];
    double cw1[kLinWaves * kFzPx];
    double qs[kFzPx];
};

__global__ __launch_bounds__(kLinWG) void k_ba_fz_bs(FzArgs F) {
    __shared__ FzBsLds L;
    if (F.flags[0] != 0) return;  // uniform: a rejected step leaves the depths
    const int chunk = blockIdx.x;
    const FzKf K = F.kfs[blockIdx.y];
    const int lane = threadIdx.x & 63, HW = F.HW;
    int kpx[kFzPPL];
    bool vpx[kFzPPL];
    double dsp[kFzPPL];
#pragma unroll
    for (int s = 0; s < kFzPPL; s++) {
        kpx[s] = chunk * kFzPx + s * 64 + lane;
        vpx[s] = kpx[s] < HW;
        dsp[s] = vpx[s] ? (double)F.disps[(size_t)K.kf * HW + kpx[s]] : 1.0;
    }
    const int kown = chunk * kFzPx + threadIdx.x;
    const bool mine = threadIdx.x < kFzPx && kown < HW;
    const double eta_px = mine ? (double)F.eta[(size_t)K.kf * HW + kown] : 0.0;
    FzCache cache;
    cache.valid = cache.rel = false;
    fz_bs_direct(F, K, chunk, kpx, vpx, dsp, eta_px, cache, false, L.cwd, L.cw0, L.cw1, L.qs);
}

// One launch per step k >= 2 of the overlapped fused iteration (n <= kPanelN):
// workgroup 0 solves step k - 1 (the system the assembly just wrote), the
// others run k_ba_fz's work for their (chunk, keyframe), recomputing step
// k - 1's E rows at F.poses_prev (its poses, copied by the step before)
// while the solve runs, and waiting for its dx only for the depth update.
// Every waiter waits on workgroup 0 alone, which is dispatched first.
union FzStepLds {
    FzLds fz;
    SmallLds sv;
    PanelLds pv;
};
static_assert(kFzWgPerCu * sizeof(FzStepLds) <= 160 * 1024, "kFzWgPerCu step workgroups per CU");

// kPanel: the system is solved by the panel solver (n <= kPanelN), else by
// the register solver (n <= kSmallN)
template <bool kLin, bool kPanel>
__global__ __launch_bounds__(kLinWG, kFzWgPerCu) void k_ba_fz_step(FzArgs F, SolveArgs A, FzWait wait) {
    __shared__ FzStepLds lds;
    if (blockIdx.x == 0) {
        // the solve is the launch's spine; a linearization workgroup may share
        // its CU, so its waves issue first
        __builtin_amdgcn_s_setprio(3);
        // the solve sets wait.ready (A.publish) once the status and dx are
        // out, before it retracts the poses
        if (kPanel)
            solve_panel_body(A, lds.pv.sm, lds.pv.ok, lds.pv.pose0);
        else
            solve_small_body(A, lds.sv);
        return;
    }
    const int b = blockIdx.x - 1;
    fz_body<true, kLin>(F, lds.fz, b % F.nch, b / F.nch, wait);
}

struct FzAsmArgs {
    // [P*P + P][kFzRecInts] assembly record of each block / segment: its
    // contribution codes (with the Schur item {kc, s1, s2 or -1 (the w
    // column), w row} of each code of type 1) and its distinct edges
    const int* rec;
    const double* hpart;
    const double* spart;
    const float* poses;
    int nch, P, n;
    float lm, ep;
    double* S;  // [n][n] assembled system (after damping)
    double* b;  // [n]
    int* ready;  // or null: the overlapped step's flag, cleared here for the launch after
    int* flags;  // with ready: flags[5] = flags[4] for the solve of the launch after
};

// Chunk 0's partial of entry (row, col) of a keyframe's Z (the other chunks'
// follow at stride kFzMaxNT * 256): Z is symmetric and only its upper tiles
// are kept, in the MFMA's lane order (result register r of lane l holds entry
// (4 r + l / 16, l % 16) of a 16 x 16 tile; the A operand of lane l is
// (l % 16, l / 16), the B operand (l / 16, l % 16)).
__device__ __forceinline__ const double* fz_z(const FzAsmArgs& A, int kc, int row, int col) {
    const int lo = min(row, col), hi = max(row, col);
    const int th = hi >> 4, tl = lo >> 4;
    const int i = lo & 15, j = hi & 15;
    const size_t idx = (size_t)(th * (th + 1) / 2 + tl) * 256 + ((i & 3) * 16 + j) * 4 + (i >> 2);
    return A.spart + (size_t)kc * A.nch * kFzMaxNT * 256 + idx;
}

// One workgroup per 6x6 block (a, b) of S (P*P) and per 6-entry segment of b
// (P more), as k_ba_assemble, with the chunk sums done here. The totals of
// the block's edges (edge_totals' arithmetic) are formed by the whole
// workgroup at once: the chunk sums of all Hjj/vj partials, the Adj columns
// (one thread per edge and column), then the expansions. Thread (slice,
// entry) adds the Z entries of its slice's Schur items, then the edges' block
// entries; the seven slices are added in a fixed order (deterministic, no
// atomics).
__global__ __launch_bounds__(256) void k_ba_fz_assemble(FzAsmArgs A) {
    __shared__ double tot[kFzMaxDst][kNJ];   // chunk sums: Hjj (upper), vj
    __shared__ double adj[kFzMaxDst][36];    // Adj of each edge, [r][c]
    __shared__ double ah[kFzMaxDst][36];     // Adj Hjj
    __shared__ double et[kFzMaxDst][kNT];    // Hii, Hij, Hjj, vi, vj
    __shared__ double red[kAsmSlices][36];
    __shared__ __attribute__((aligned(16))) int rec[kFzRecInts];
    const int g = blockIdx.x, tid = threadIdx.x;
    const int sl = tid / 36, ent = tid - sl * 36;
    const int P = A.P, n = A.n;
    const bool isS = g < P * P;
    const bool act = sl < kAsmSlices && (isS || ent < 6);
    const int r = ent / 6, c = ent - (ent / 6) * 6;
    // the block's record in one round of 16-byte loads
    static_assert(kFzRecInts % 4 == 0 && kFzRecInts / 4 <= 256, "one int4 of the record a thread");
    if (tid < kFzRecInts / 4)
        reinterpret_cast<int4*>(rec)[tid] =
            reinterpret_cast<const int4*>(A.rec + (size_t)g * kFzRecInts)[tid];
    __syncthreads();
    const int nq = rec[0], nd = rec[1];
    const int* redge = rec + kFzRecEdges;  // (edge, ii, jj)
    const int* rcode = rec + kFzRecCodes;  // (code, Schur item)
    // (1) chunk sums of the edges' partials, and the Adj columns
    for (int t = tid; t < nd * kNJ; t += 256) {
        const int le = t / kNJ, v = t - (t / kNJ) * kNJ;
        tot[le][v] = sum_strided<32>(A.hpart + (size_t)redge[3 * le] * A.nch * kNJ + v, kNJ, A.nch);
    }
    for (int t = tid; t < nd * 6; t += 256) {
        const int le = t / 6, cc = t - (t / 6) * 6;
        double tij[3], qij[4], u[6], y[6];
        edge_rel(A.poses, redge[3 * le + 1], redge[3 * le + 2], tij, qij);
#pragma unroll
        for (int m = 0; m < 6; m++) u[m] = m == cc ? 1.0 : 0.0;
        adj_se3(tij, qij, u, y);  // column cc (se3.cuh:28-41)
#pragma unroll
        for (int m = 0; m < 6; m++) adj[le][m * 6 + cc] = y[m];
    }
    // the Schur items (thread-private)
    double s = 0.0;
    if (act) {
        for (int q = sl; q < nq; q += kAsmSlices) {
            const int* rc = rcode + 5 * q;
            if (code_type(rc[0]) != 1) continue;
            s -= sum_strided<32>(isS ? fz_z(A, rc[1], 6 * rc[2] + r, 6 * rc[3] + c)
                                     : fz_z(A, rc[1], 6 * rc[2] + ent, rc[4]),
                                 kFzMaxNT * 256, A.nch);
        }
    }
    __syncthreads();
    // (2) Hij = -Adj Hjj, Hjj, vi = -Adj vj, vj (ba.cuh:198-220 via Ji = -Adj^T Jj)
    for (int t = tid; t < nd * 36; t += 256) {
        const int le = t / 36, rc = t - (t / 36) * 36;
        const int rr = rc / 6, cc = rc - (rc / 6) * 6;
        double a = 0.0;
#pragma unroll
        for (int k = 0; k < 6; k++) a += adj[le][rr * 6 + k] * tot[le][tri(max(k, cc), min(k, cc))];
        ah[le][rc] = a;
        et[le][kTotHij + rc] = -a;
        et[le][kTotHjj + rc] = tot[le][tri(max(rr, cc), min(rr, cc))];
        if (rc < 6) {
            double v = 0.0;
#pragma unroll
            for (int k = 0; k < 6; k++) v += adj[le][rc * 6 + k] * tot[le][21 + k];
            et[le][kTotVi + rc] = -v;
            et[le][kTotVj + rc] = tot[le][21 + rc];
        }
    }
    __syncthreads();
    // (3) Hii = Adj Hjj Adj^T
    for (int t = tid; t < nd * 36; t += 256) {
        const int le = t / 36, rc = t - (t / 36) * 36;
        const int rr = rc / 6, cc = rc - (rc / 6) * 6;
        double h = 0.0;
#pragma unroll
        for (int k = 0; k < 6; k++) h += ah[le][rr * 6 + k] * adj[le][cc * 6 + k];
        et[le][kTotHii + rc] = h;
    }
    __syncthreads();
    if (act) {
        for (int q = sl; q < nq; q += kAsmSlices) {
            const int cd = rcode[5 * q];
            if (code_type(cd) != 0) continue;
            const int v = code_val(cd);
            if (isS) {
                const double* e = et[v >> 2];
                const int w = v & 3;
                s += w == 0 ? e[kTotHii + r * 6 + c]
                   : w == 1 ? e[kTotHij + r * 6 + c]
                   : w == 2 ? e[kTotHij + c * 6 + r]
                            : e[kTotHjj + r * 6 + c];
            } else {
                s += et[v >> 1][((v & 1) ? kTotVj : kTotVi) + ent];
            }
        }
    }
    if (sl < kAsmSlices) red[sl][ent] = s;
    __syncthreads();
    if (isS && tid < 36) {
        double t = red[0][tid];
#pragma unroll
        for (int k = 1; k < kAsmSlices; k++) t += red[k][tid];
        const int a = g / P, bb = g - (g / P) * P;
        const int row = a * 6 + tid / 6, col = bb * 6 + tid % 6;
        if (row == col) t = t + (double)A.ep + (double)A.lm * t;  // ba.cuh:749-750
        A.S[(size_t)row * n + col] = t;
    } else if (!isS && tid < 6) {
        double t = red[0][tid];
#pragma unroll
        for (int k = 1; k < kAsmSlices; k++) t += red[k][tid];
        A.b[(g - P * P) * 6 + tid] = t;
    }
    if (A.ready && g == 0 && tid == 0) {  // (last: its load is waited for at once)
        *A.ready = 0;
        A.flags[5] = A.flags[4];  // a wait of the last launch gave up: no more steps
    }
}

}  // namespace

// ----------------------------------------------------------- host side ---
struct BaState {
    // cached plan key
    bool valid = false;
    std::vector<int> key_ii, key_jj;
    int key_t0 = 0, key_t1 = 0, key_motion = 0, key_HW = 0;
    // plan sizes
    int M = 0, P = 0, n = 0, N_kf = 0, N_E = 0, N_pu = 0, n_blk = 0, nch = 1;
    int npose = 0;  // max(the edges' largest frame index + 1, t1)
    std::vector<int> host;  // packed plan
    size_t off[kPlanParts] = {0};
    DevBuf plan_dev, hpart, etot, stot, E, Q, Wv, S, S_dbg, b_dbg, dx_dbg, dx, flags;
    HostStage stage;
    bool has_system = false;
    bool lin_by_wave = false;  // no keyframe has two edges to the same free pose
    // fused path (every keyframe with at most kFzMaxSlots E rows)
    bool fz = false;
    size_t fz_off[3] = {0};  // kfs, eds, assembly records (ints into host)
    DevBuf spart, poses_prev;
    // overlapped steps: the second pose copy and the step flag
    DevBuf poses_alt, ready;
    int cus = 0;  // compute units: the overlapped step's workgroups must all be resident
    int spin_max = kFzSpinMax;  // the step launch's bounded wait
};

namespace {

PlanDev plan_ptrs(BaState* s) {
    const int* base = s->plan_dev.as<int>();
    PlanDev p;
    const int** f[kPlanParts] = {&p.kf_list, &p.kf_eptr, &p.kf_eidx, &p.edge_ri, &p.edge_rj,
                                 &p.row_pose, &p.row_kf, &p.kf_rptr, &p.kf_rows, &p.pairs,
                                 &p.sblk, &p.sblk_ptr, &p.sblk_src, &p.bv_ptr, &p.bv_src,
                                 &p.blkmap};
    for (int i = 0; i < kPlanParts; i++) *f[i] = base + s->off[i];
    return p;
}

// Tables of the fused path (k_ba_fz, k_ba_fz_assemble), appended to the
// packed plan 16-byte aligned; s->fz stays false when a keyframe has more
// than kFzMaxSlots E rows or a block of S more than kFzMaxDst edges (those
// systems take the five-kernel iteration). Slots, items and the contribution
// lists follow the E rows and the S/b scatter of ba.cuh:520-548, 577-663.
void build_fz(BaState* s, const int* ii, const int* jj, int M, int t0, int t1, int motion_only,
              const std::vector<int>& kf_list, const std::vector<int>& kf_eptr,
              const std::vector<int>& kf_eidx) {
    s->fz = false;
    if (motion_only) return;
    const int P = t1 - t0, N_kf = (int)kf_list.size();
    const int ND = P * P + P;  // destinations: blocks of S, then segments of b
    auto free_pose = [&](int f) { return f >= t0 && f < t1; };
    std::vector<int> kfs, eds, items;
    std::vector<std::vector<int>> codes(ND), dedges(ND);
    for (int kc = 0; kc < N_kf; kc++) {
        const int kf = kf_list[kc];
        const int ri = free_pose(kf) ? 1 : 0;
        std::vector<int> spose;  // pose of each slot
        if (ri) spose.push_back(kf - t0);
        for (int ei = kf_eptr[kc]; ei < kf_eptr[kc + 1]; ei++) {
            const int e = kf_eidx[ei];
            int slot = -1;
            if (ii[e] != jj[e] && free_pose(jj[e])) {
                slot = (int)spose.size();
                spose.push_back(jj[e] - t0);
            }
            eds.insert(eds.end(), {e, ii[e], jj[e], slot});
        }
        const int nslot = (int)spose.size();
        if (nslot > kFzMaxSlots) return;
        const int T = (6 * nslot + 1 + 15) / 16;
        kfs.insert(kfs.end(), {kf, kf_eptr[kc], kf_eptr[kc + 1], nslot | ri << 8 | T << 12});
        const int wrow = 6 * nslot;
        for (int s1 = 0; s1 < nslot; s1++) {
            for (int s2 = 0; s2 < nslot; s2++) {
                codes[spose[s1] * P + spose[s2]].push_back(code(1, (int)items.size() / 4));
                items.insert(items.end(), {kc, s1, s2, wrow});
            }
            codes[P * P + spose[s1]].push_back(code(1, (int)items.size() / 4));
            items.insert(items.end(), {kc, s1, -1, wrow});
        }
    }
    auto local = [&](int d, int e) {
        std::vector<int>& v = dedges[d];
        for (int k = 0; k < (int)v.size(); k++)
            if (v[k] == e) return k;
        v.push_back(e);
        return (int)v.size() - 1;
    };
    for (int e = 0; e < M; e++) {
        const int a = ii[e] - t0, b = jj[e] - t0;
        const bool va = a >= 0 && a < P, vb = b >= 0 && b < P;
        if (va) codes[a * P + a].push_back(code(0, local(a * P + a, e) * 4 + 0));
        if (va && vb) {
            codes[a * P + b].push_back(code(0, local(a * P + b, e) * 4 + 1));
            codes[b * P + a].push_back(code(0, local(b * P + a, e) * 4 + 2));
        }
        if (vb) codes[b * P + b].push_back(code(0, local(b * P + b, e) * 4 + 3));
        if (va) codes[P * P + a].push_back(code(0, local(P * P + a, e) * 2 + 0));
        if (vb) codes[P * P + b].push_back(code(0, local(P * P + b, e) * 2 + 1));
    }
    // one record of kFzRecInts per block of S / segment of b; the records of
    // every block, empty ones included, stay under 4 MB (P <= 42; frontend
    // windows have P ~ 10-20, and larger graphs exceed kFzMaxSlots anyway)
    if ((size_t)ND * kFzRecInts > ((size_t)1 << 20)) return;
    std::vector<int> rec((size_t)ND * kFzRecInts, 0);
    for (int d = 0; d < ND; d++) {
        const int nd = (int)dedges[d].size(), nq = (int)codes[d].size();
        if (nd > kFzMaxDst || nq > kFzMaxCodes) return;
        int* r = rec.data() + (size_t)d * kFzRecInts;
        r[0] = nq;
        r[1] = nd;
        for (int le = 0; le < nd; le++) {
            const int e = dedges[d][le];
            r[kFzRecEdges + 3 * le] = e;
            r[kFzRecEdges + 3 * le + 1] = ii[e];
            r[kFzRecEdges + 3 * le + 2] = jj[e];
        }
        for (int q = 0; q < nq; q++) {
            const int cd = codes[d][q];
            int* c = r + kFzRecCodes + 5 * q;
            c[0] = cd;
            if (code_type(cd) == 1)
                for (int k = 0; k < 4; k++) c[1 + k] = items[(size_t)code_val(cd) * 4 + k];
        }
    }
    const std::vector<int>* parts[3] = {&kfs, &eds, &rec};
    for (int i = 0; i < 3; i++) {
        while (s->host.size() % 4) s->host.push_back(0);
        s->fz_off[i] = s->host.size();
        s->host.insert(s->host.end(), parts[i]->begin(), parts[i]->end());
        s->host.push_back(0);
    }
    s->fz = true;
}

// Builds the index structures of ba.cuh:520-663 once per edge set: keyframes
// (unique ii, ascending), E rows keyed by (pose, kf) in order of first
// appearance, upper pairs of rows per keyframe, and the contribution lists of
// every 6x6 block of S and every 6-vector of b.
int build_plan(BaState* s, const int* ii, const int* jj, int M, int t0, int t1, int motion_only,
               int HW) {
    const int P = t1 - t0;
    s->M = M;
    s->P = P;
    s->n = 6 * P;
    int maxf = 0;
    for (int e = 0; e < M; e++) {
        if (ii[e] < 0 || jj[e] < 0) return fail(SLK_E_ARG, "ba_iterate: negative frame index");
        maxf = std::max(maxf, std::max(ii[e], jj[e]));
    }
    s->npose = std::max(maxf + 1, t1);
    std::vector<int> kf_compact(maxf + 1, -1), kf_list;
    for (int e = 0; e < M; e++) kf_compact[ii[e]] = 0;
    for (int k = 0; k <= maxf; k++)
        if (kf_compact[k] == 0) {
            kf_compact[k] = (int)kf_list.size();
            kf_list.push_back(k);
        }
    const int N_kf = (int)kf_list.size();
    std::vector<int> kf_eptr(N_kf + 1, 0), kf_eidx(M);
    for (int e = 0; e < M; e++) kf_eptr[kf_compact[ii[e]] + 1]++;
    for (int k = 0; k < N_kf; k++) kf_eptr[k + 1] += kf_eptr[k];
    {
        std::vector<int> fill(kf_eptr.begin(), kf_eptr.end() - 1);
        for (int e = 0; e < M; e++) kf_eidx[fill[kf_compact[ii[e]]]++] = e;
    }
    std::map<std::pair<int, int>, int> rowmap;
    std::vector<int> row_pose, row_kf, edge_ri(M, -1), edge_rj(M, -1);
    if (!motion_only) {
        auto get_row = [&](int p, int kfabs) {
            auto key = std::make_pair(p, kfabs);
            auto it = rowmap.find(key);
            if (it != rowmap.end()) return it->second;
            const int r = (int)row_pose.size();
            rowmap[key] = r;
            row_pose.push_back(p);
            row_kf.push_back(kf_compact[kfabs]);
            return r;
        };
        for (int e = 0; e < M; e++) {
            const int pi = ii[e] - t0, pj = jj[e] - t0;
            if (pi >= 0 && pi < P) edge_ri[e] = get_row(pi, ii[e]);
            if (pj >= 0 && pj < P) edge_rj[e] = get_row(pj, ii[e]);
        }
    }
    const int N_E = (int)row_pose.size();
    // k_ba_lin_wv stores each non-stereo edge's jj row directly: the row must
    // belong to that edge alone
    {
        std::vector<int> owner(N_E, -1);
        s->lin_by_wave = true;
        for (int e = 0; e < M && s->lin_by_wave; e++) {
            const int r = edge_rj[e];
            if (r < 0 || ii[e] == jj[e]) continue;
            if (owner[r] >= 0) s->lin_by_wave = false;
            owner[r] = e;
        }
    }
    std::vector<int> kf_rptr(N_kf + 1, 0), kf_rows(N_E);
    for (int r = 0; r < N_E; r++) kf_rptr[row_kf[r] + 1]++;
    for (int k = 0; k < N_kf; k++) kf_rptr[k + 1] += kf_rptr[k];
    {
        std::vector<int> fill(kf_rptr.begin(), kf_rptr.end() - 1);
        for (int r = 0; r < N_E; r++) kf_rows[fill[row_kf[r]]++] = r;
    }
    std::vector<int> pairs;
    for (int kc = 0; kc < N_kf; kc++)
        for (int a = kf_rptr[kc]; a < kf_rptr[kc + 1]; a++)
            for (int b = a; b < kf_rptr[kc + 1]; b++) {
                pairs.push_back(kf_rows[a]);
                pairs.push_back(kf_rows[b]);
                pairs.push_back(kc);
            }
    const int N_pu = (int)pairs.size() / 3;
    // contributions per destination block a*P+b
    std::map<int, std::vector<int>> blocks;
    for (int e = 0; e < M; e++) {
        const int a = ii[e] - t0, b = jj[e] - t0;
        const bool va = a >= 0 && a < P, vb = b >= 0 && b < P;
        if (va) blocks[a * P + a].push_back(code(0, e * 4 + 0));
        if (va && vb) {
            blocks[a * P + b].push_back(code(0, e * 4 + 1));
            blocks[b * P + a].push_back(code(0, e * 4 + 2));
        }
        if (vb) blocks[b * P + b].push_back(code(0, e * 4 + 3));
    }
    for (int p = 0; p < N_pu; p++) {
        const int r1 = pairs[3 * p], r2 = pairs[3 * p + 1];
        const int a = row_pose[r1], b = row_pose[r2];
        blocks[a * P + b].push_back(code(1, p));
        if (r1 != r2) blocks[b * P + a].push_back(code(2, p));
    }
    std::vector<int> sblk, sblk_ptr(1, 0), sblk_src;
    for (auto& kv : blocks) {
        sblk.push_back(kv.first);
        sblk_src.insert(sblk_src.end(), kv.second.begin(), kv.second.end());
        sblk_ptr.push_back((int)sblk_src.size());
    }
    std::vector<std::vector<int>> bl(P);
    for (int e = 0; e < M; e++) {
        const int a = ii[e] - t0, b = jj[e] - t0;
        if (a >= 0 && a < P) bl[a].push_back(code(0, e * 2 + 0));
        if (b >= 0 && b < P) bl[b].push_back(code(0, e * 2 + 1));
    }
    for (int r = 0; r < N_E; r++) bl[row_pose[r]].push_back(code(1, r));
    std::vector<int> bv_ptr(1, 0), bv_src;
    for (int a = 0; a < P; a++) {
        bv_src.insert(bv_src.end(), bl[a].begin(), bl[a].end());
        bv_ptr.push_back((int)bv_src.size());
    }
    s->N_kf = N_kf;
    s->N_E = N_E;
    s->N_pu = N_pu;
    s->n_blk = (int)sblk.size();
    s->nch = (HW + kLinPx - 1) / kLinPx;
    std::vector<int> blkmap((size_t)P * P, -1);
    for (size_t k = 0; k < sblk.size(); k++) blkmap[sblk[k]] = (int)k;
    const std::vector<int>* parts[kPlanParts] = {&kf_list, &kf_eptr, &kf_eidx, &edge_ri,
                                                 &edge_rj, &row_pose, &row_kf, &kf_rptr,
                                                 &kf_rows, &pairs, &sblk, &sblk_ptr,
                                                 &sblk_src, &bv_ptr, &bv_src, &blkmap};
    s->host.clear();
    for (int i = 0; i < kPlanParts; i++) {
        s->off[i] = s->host.size();
        s->host.insert(s->host.end(), parts[i]->begin(), parts[i]->end());
        s->host.push_back(0);  // keeps every array non-empty
    }
    build_fz(s, ii, jj, M, t0, t1, motion_only, kf_list, kf_eptr, kf_eidx);
    if (s->fz) s->nch = (HW + kFzPx - 1) / kFzPx;  // the fused kernels' chunks
    return SLK_OK;
}

}  // namespace

int ba_create(slk_ctx* ctx) {
    ctx->ba = new BaState();
    SLK_TRY(ctx->ba->flags.ensure(kBaFlags * sizeof(int)));
    SLK_HIP(hipMemset(ctx->ba->flags.ptr, 0, kBaFlags * sizeof(int)));
    if (hipDeviceGetAttribute(&ctx->ba->cus, hipDeviceAttributeMultiprocessorCount,
                              ctx->device) != hipSuccess)
        return fail(SLK_E_HIP, "hipDeviceGetAttribute(multiProcessorCount) failed");
    return SLK_OK;
}

void ba_destroy(slk_ctx* ctx) {
    BaState* s = ctx->ba;
    if (!s) return;
    DevBuf* bufs[] = {&s->plan_dev, &s->hpart,  &s->etot,      &s->stot,      &s->E,
                      &s->Q,        &s->Wv,     &s->S,         &s->S_dbg,     &s->b_dbg,
                      &s->dx_dbg,   &s->dx,     &s->flags,     &s->spart,     &s->poses_prev,
                      &s->poses_alt, &s->ready};
    for (DevBuf* b : bufs) b->release();
    s->stage.release();
    delete s;
    ctx->ba = nullptr;
}

}  // namespace slk

using namespace slk;

namespace {

struct IterArgs {
    float* poses;
    float* disps;
    const float* intr;
    const float* target;
    const float* weight;
    const float* eta;
    const int* ii_gpu;
    const int* jj_gpu;
    int t0, t1;
    float lm, ep;
    int motion_only;
};

// Argument checks, and the plan and buffers of the edge set (rebuilt only
// when the edge list, t0/t1 or the mode change).
int ba_prepare(slk_ctx* ctx, const IterArgs& I, const int* ii_host, const int* jj_host, int M,
               hipStream_t stream) {
    if (!ctx || !ctx->ba) return fail(SLK_E_ARG, "ba_iterate: null context");
    if (M < 1 || I.t0 < 0 || I.t1 <= I.t0)
        return fail(SLK_E_ARG, "ba_iterate: need M >= 1, 0 <= t0 < t1");
    if (!I.poses || !I.disps || !I.intr || !I.target || !I.weight || !I.ii_gpu || !I.jj_gpu ||
        !ii_host || !jj_host || (!I.motion_only && !I.eta))
        return fail(SLK_E_ARG, "ba_iterate: null argument");
    BaState* s = ctx->ba;
    const int HW = ctx->HW;
    const int t0 = I.t0, t1 = I.t1, motion_only = I.motion_only;
    const bool same = s->valid && s->key_t0 == t0 && s->key_t1 == t1 &&
                      s->key_motion == motion_only && s->key_HW == HW &&
                      (int)s->key_ii.size() == M &&
                      std::memcmp(s->key_ii.data(), ii_host, sizeof(int) * M) == 0 &&
                      std::memcmp(s->key_jj.data(), jj_host, sizeof(int) * M) == 0;
    if (same) return SLK_OK;
    s->valid = false;
    SLK_TRY(build_plan(s, ii_host, jj_host, M, t0, t1, motion_only, HW));
    if (s->n > 0x7fff) return fail(SLK_E_ARG, "ba_iterate: too many free poses");
    const size_t pbytes = s->host.size() * sizeof(int);
    SLK_TRY(s->stage.ensure(pbytes));
    std::memcpy(s->stage.ptr, s->host.data(), pbytes);
    SLK_TRY(s->plan_dev.ensure(pbytes));
    SLK_HIP(hipMemcpyAsync(s->plan_dev.ptr, s->stage.ptr, pbytes, hipMemcpyHostToDevice, stream));
    SLK_HIP(hipEventRecord(s->stage.done, stream));
    s->stage.pending = true;
    const size_t n = (size_t)s->n;
    SLK_TRY(s->hpart.ensure((size_t)M * s->nch * kNJ * sizeof(double)));
    if (s->fz) {
        SLK_TRY(s->spart.ensure((size_t)s->N_kf * s->nch * kFzMaxNT * 256 * sizeof(double)));
        SLK_TRY(s->poses_prev.ensure((size_t)s->P * 7 * sizeof(float)));
        SLK_TRY(s->poses_alt.ensure((size_t)s->P * 7 * sizeof(float)));
        SLK_TRY(s->ready.ensure(sizeof(int)));
    } else {
        SLK_TRY(s->etot.ensure((size_t)M * kNT * sizeof(double)));
        SLK_TRY(s->stot.ensure(std::max<size_t>(1, (size_t)(s->N_pu + s->N_E) * 36) *
                               sizeof(double)));
        SLK_TRY(s->E.ensure(std::max<size_t>(1, (size_t)s->N_E * 6 * HW) * sizeof(double)));
        SLK_TRY(s->Q.ensure((size_t)s->N_kf * HW * sizeof(double)));
        SLK_TRY(s->Wv.ensure((size_t)s->N_kf * HW * sizeof(double)));
    }
    if (n > (size_t)kPanelN) SLK_TRY(s->S.ensure((n + 1) * n * sizeof(double)));
    SLK_TRY(s->S_dbg.ensure(n * n * sizeof(double)));
    SLK_TRY(s->b_dbg.ensure(n * sizeof(double)));
    SLK_TRY(s->dx_dbg.ensure(n * sizeof(double)));
    SLK_TRY(s->dx.ensure(n * sizeof(float)));
    s->key_ii.assign(ii_host, ii_host + M);
    s->key_jj.assign(jj_host, jj_host + M);
    s->key_t0 = t0;
    s->key_t1 = t1;
    s->key_motion = motion_only;
    s->key_HW = HW;
    s->valid = true;
    return SLK_OK;
}

SolveArgs solve_args(BaState* s, const PlanDev& plan, const IterArgs& I) {
    SolveArgs A;
    A.plan = plan;
    A.etot = s->etot.as<double>();
    A.stot = s->stot.as<double>();
    A.N_pu = s->N_pu;
    A.P = s->P;
    A.n = s->n;
    A.n_blk = s->n_blk;
    A.t0 = I.t0;
    A.t1 = I.t1;
    A.lm = I.lm;
    A.ep = I.ep;
    A.S = s->S.as<double>();
    A.S_dbg = s->S_dbg.as<double>();
    A.b_dbg = s->b_dbg.as<double>();
    A.dx_dbg = s->dx_dbg.as<double>();
    A.dx = s->dx.as<float>();
    A.flags = s->flags.as<int>();
    A.halt = nullptr;
    A.publish = nullptr;
    A.poses = I.poses;
    A.poses_prev = s->fz ? s->poses_prev.as<float>() : nullptr;
    A.poses_next = nullptr;
    return A;
}

int launch_solve(slk_ctx* ctx, BaState* s, const SolveArgs& A, hipStream_t stream) {
    ProfScope ps(ctx, "ba_solve", stream);
    if (s->n <= kSmallN) {
        hipLaunchKernelGGL(k_ba_solve_small, dim3(1), dim3(256), 0, stream, A);
    } else if (s->n <= kPanelN) {
        // t1 - t0 = P <= kPanelPoses
        hipLaunchKernelGGL(k_ba_solve_panel, dim3(1), dim3(256), panel_solve_lds_bytes(s->n),
                           stream, A);
    } else {
        SLK_TRY(solve_blocked(A, stream));
    }
    SLK_HIP(hipGetLastError());
    return SLK_OK;
}

// The five-kernel iteration: linearization with the E rows in HBM, Schur
// items and edge totals, assembly, solve, back-substitution.
int iterate_classic(slk_ctx* ctx, BaState* s, const IterArgs& I, hipStream_t stream) {
    const int HW = ctx->HW, M = s->M;
    const PlanDev plan = plan_ptrs(s);
    {
        // one profile name per kernel: k_ba_lin_wv (one wave per edge) or
        // k_ba_lin_kf (edge by edge, when a row has two edges)
        ProfScope ps(ctx, s->lin_by_wave ? "ba_lin_wv" : "ba_lin_kf", stream);
        hipLaunchKernelGGL(s->lin_by_wave ? k_ba_lin_wv : k_ba_lin_kf, dim3(s->nch, s->N_kf),
                           dim3(kLinWG), 0, stream, plan, I.target, I.weight, I.poses, I.disps,
                           I.intr, I.ii_gpu, I.jj_gpu, I.eta, s->hpart.as<double>(),
                           s->E.as<double>(), s->Q.as<double>(), s->Wv.as<double>(), HW,
                           ctx->w, s->nch, I.motion_only);
    }
    SLK_HIP(hipGetLastError());
    {
        // the Schur items, then one workgroup per edge for its totals
        const int items = I.motion_only ? 0 : s->N_pu + s->N_E;
        ProfScope ps(ctx, "ba_schur", stream);
        hipLaunchKernelGGL(k_ba_schur, dim3(items + M), dim3(kSchWG), 0, stream, plan,
                           s->E.as<double>(), s->Q.as<double>(), s->Wv.as<double>(),
                           s->stot.as<double>(), HW, s->N_pu, items, I.poses, I.ii_gpu,
                           I.jj_gpu, s->hpart.as<double>(), s->etot.as<double>(), s->nch);
        SLK_HIP(hipGetLastError());
    }
    const SolveArgs A = solve_args(s, plan, I);
    {
        ProfScope ps(ctx, "ba_assemble", stream);
        hipLaunchKernelGGL(k_ba_assemble, dim3(s->P * s->P + s->P), dim3(256), 0, stream, A);
    }
    SLK_HIP(hipGetLastError());
    SLK_TRY(launch_solve(ctx, s, A, stream));
    if (!I.motion_only && s->N_E > 0) {
        ProfScope ps(ctx, "ba_backsub", stream);
        hipLaunchKernelGGL(k_ba_backsub, dim3((HW + 255) / 256, s->N_kf), dim3(256), 0, stream,
                           plan, s->E.as<double>(), s->Q.as<double>(), s->Wv.as<double>(),
                           s->dx.as<float>(), s->flags.as<int>(), I.disps, HW);
        SLK_HIP(hipGetLastError());
    }
    return SLK_OK;
}

// `iters` fused iterations: k_ba_fz (the previous step's back-substitution
// from the second iteration on, then the linearization and Schur partials),
// k_ba_fz_assemble and the solve each; then the last back-substitution.
int iterate_fused(slk_ctx* ctx, BaState* s, const IterArgs& I, int iters, hipStream_t stream) {
    const PlanDev plan = plan_ptrs(s);
    const int* base = s->plan_dev.as<int>();
    FzArgs F;
    F.kfs = reinterpret_cast<const FzKf*>(base + s->fz_off[0]);
    F.eds = reinterpret_cast<const FzEdge*>(base + s->fz_off[1]);
    F.target = I.target;
    F.weight = I.weight;
    F.poses = I.poses;
    F.poses_prev = s->poses_prev.as<float>();
    F.pose_copy = nullptr;
    F.spin_max = s->spin_max;
    F.intr = I.intr;
    F.eta = I.eta;
    F.dx = s->dx.as<float>();
    F.flags = s->flags.as<int>();
    F.disps = I.disps;
    F.hpart = s->hpart.as<double>();
    F.spart = s->spart.as<double>();
    F.HW = ctx->HW;
    F.W = ctx->w;
    F.nch = s->nch;
    F.t0 = I.t0;
    F.t1 = I.t1;
    F.npose = s->npose;
    FzAsmArgs G;
    G.rec = base + s->fz_off[2];
    G.hpart = s->hpart.as<double>();
    G.spart = s->spart.as<double>();
    G.poses = I.poses;
    G.nch = s->nch;
    G.P = s->P;
    G.n = s->n;
    G.lm = I.lm;
    G.ep = I.ep;
    G.S = s->S_dbg.as<double>();
    G.b = s->b_dbg.as<double>();
    G.ready = nullptr;
    G.flags = s->flags.as<int>();
    const SolveArgs A = solve_args(s, plan, I);
    const dim3 grid(s->nch, s->N_kf);
    // all workgroups resident at once (kFzWgPerCu per CU): the waiting ones
    // then never hold CUs that later linearization workgroups need
    if (s->n <= kPanelN && 1 + s->nch * s->N_kf <= kFzWgPerCu * s->cus) {
        // Overlapped steps: the first linearization (which keeps a copy of the
        // poses it used), then per step the assembly and one launch of the
        // solve beside the next linearization. The pose copies alternate:
        // step k's launch relinearizes at pp[k & 1] while its solve writes
        // the new poses to pp[(k + 1) & 1].
        float* pp[2] = {s->poses_prev.as<float>(), s->poses_alt.as<float>()};
        FzArgs F1 = F;
        F1.pose_copy = pp[0];
        {
            ProfScope ps(ctx, "ba_fz_lin", stream);
            hipLaunchKernelGGL((k_ba_fz<false, true>), grid, dim3(kLinWG), 0, stream, F1);
        }
        SLK_HIP(hipGetLastError());
        G.ready = s->ready.as<int>();
        const FzWait wait = {s->ready.as<int>()};
        const dim3 sgrid(1 + s->nch * s->N_kf);
        for (int it = 0; it < iters; it++) {
            {
                ProfScope ps(ctx, "ba_fz_asm", stream);
                hipLaunchKernelGGL(k_ba_fz_assemble, dim3(s->P * s->P + s->P), dim3(256), 0,
                                   stream, G);
            }
            SLK_HIP(hipGetLastError());
            FzArgs Fk = F;
            Fk.poses_prev = pp[it & 1];
            SolveArgs Ak = A;
            Ak.poses_prev = nullptr;
            Ak.poses_next = pp[(it + 1) & 1];
            Ak.halt = s->flags.as<int>() + 5;
            Ak.publish = s->ready.as<int>();  // set by the solve before its retraction
            const bool panel = s->n > kSmallN;
            if (it + 1 < iters) {
                ProfScope ps(ctx, "ba_fz_step", stream);
                if (panel)
                    hipLaunchKernelGGL((k_ba_fz_step<true, true>), sgrid, dim3(kLinWG), 0, stream,
                                       Fk, Ak, wait);
                else
                    hipLaunchKernelGGL((k_ba_fz_step<true, false>), sgrid, dim3(kLinWG), 0,
                                       stream, Fk, Ak, wait);
            } else {
                ProfScope ps(ctx, "ba_fz_last", stream);
                if (panel)
                    hipLaunchKernelGGL((k_ba_fz_step<false, true>), sgrid, dim3(kLinWG), 0,
                                       stream, Fk, Ak, wait);
                else
                    hipLaunchKernelGGL((k_ba_fz_step<false, false>), sgrid, dim3(kLinWG), 0,
                                       stream, Fk, Ak, wait);
            }
            SLK_HIP(hipGetLastError());
        }
        return SLK_OK;
    }
    for (int it = 0; it < iters; it++) {
        {
            ProfScope ps(ctx, "ba_fz_lin", stream);
            if (it == 0)
                hipLaunchKernelGGL((k_ba_fz<false, true>), grid, dim3(kLinWG), 0, stream, F);
            else
                hipLaunchKernelGGL((k_ba_fz<true, true>), grid, dim3(kLinWG), 0, stream, F);
        }
        SLK_HIP(hipGetLastError());
        {
            ProfScope ps(ctx, "ba_fz_asm", stream);
            hipLaunchKernelGGL(k_ba_fz_assemble, dim3(s->P * s->P + s->P), dim3(256), 0, stream,
                               G);
        }
        SLK_HIP(hipGetLastError());
        SLK_TRY(launch_solve(ctx, s, A, stream));
    }
    {
        ProfScope ps(ctx, "ba_fz_bs", stream);
        hipLaunchKernelGGL(k_ba_fz_bs, grid, dim3(kLinWG), 0, stream, F);
    }
    SLK_HIP(hipGetLastError());
    return SLK_OK;
}

int ba_run(slk_ctx* ctx, const IterArgs& I, const int* ii_host, const int* jj_host, int M,
           int iters, hipStream_t stream) {
    if (iters < 1) return fail(SLK_E_ARG, "ba_iterate_n: need iters >= 1");
    SLK_TRY(ba_prepare(ctx, I, ii_host, jj_host, M, stream));
    BaState* s = ctx->ba;
    if (s->fz) {
        SLK_TRY(iterate_fused(ctx, s, I, iters, stream));
    } else {
        for (int it = 0; it < iters; it++) SLK_TRY(iterate_classic(ctx, s, I, stream));
    }
    s->has_system = true;
    return SLK_OK;
}

}  // namespace

extern "C" int slk_ba_iterate(slk_ctx* ctx, float* poses, float* disps, const float* intrinsics,
                              const float* target, const float* weight, const float* eta,
                              const int* ii_gpu, const int* jj_gpu, const int* ii_host,
                              const int* jj_host, int num_edges, int t0, int t1, float lm,
                              float ep, int motion_only, hipStream_t stream) {
    const IterArgs I = {poses, disps, intrinsics, target, weight, eta, ii_gpu, jj_gpu,
                        t0,    t1,    lm,         ep,     motion_only ? 1 : 0};
    return ba_run(ctx, I, ii_host, jj_host, num_edges, 1, stream);
}

extern "C" int slk_ba_iterate_n(slk_ctx* ctx, float* poses, float* disps,
                                const float* intrinsics, const float* target, const float* weight,
                                const float* eta, const int* ii_gpu, const int* jj_gpu,
                                const int* ii_host, const int* jj_host, int num_edges, int t0,
                                int t1, float lm, float ep, int motion_only, int iters,
                                hipStream_t stream) {
    const IterArgs I = {poses, disps, intrinsics, target, weight, eta, ii_gpu, jj_gpu,
                        t0,    t1,    lm,         ep,     motion_only ? 1 : 0};
    return ba_run(ctx, I, ii_host, jj_host, num_edges, iters, stream);
}

extern "C" int slk_ba_set_wait_limit(slk_ctx* ctx, int polls) {
    if (!ctx || !ctx->ba) return fail(SLK_E_ARG, "ba_set_wait_limit: null context");
    ctx->ba->spin_max = polls < 0 ? kFzSpinMax : polls;
    return SLK_OK;
}

extern "C" int slk_ba_status(slk_ctx* ctx, hipStream_t stream) {
    if (!ctx || !ctx->ba) return fail(SLK_E_ARG, "ba_status: null context");
    int f[kBaFlags];
    SLK_HIP(hipMemcpyAsync(f, ctx->ba->flags.ptr, sizeof f, hipMemcpyDeviceToHost, stream));
    SLK_HIP(hipStreamSynchronize(stream));
    const int bad = f[1], gave_up = f[3];
    SLK_HIP(hipMemsetAsync(ctx->ba->flags.ptr, 0, sizeof f, stream));
    SLK_HIP(hipStreamSynchronize(stream));
    if (gave_up)
        return fail(SLK_E_HIP, "ba_iterate: a fused step stopped waiting for its solve");
    return bad ? fail(SLK_E_NOT_SPD, "ba_iterate: system not positive definite") : SLK_OK;
}

extern "C" int slk_ba_last_system(slk_ctx* ctx, double* S_host, double* b_host, double* dx_host,
                                  int* n_out, hipStream_t stream) {
    if (!ctx || !ctx->ba) return fail(SLK_E_ARG, "ba_last_system: null context");
    BaState* s = ctx->ba;
    if (!s->has_system) return fail(SLK_E_STATE, "ba_last_system: no iterate yet");
    const size_t n = (size_t)s->n;
    if (n_out) *n_out = (int)n;
    if (S_host)
        SLK_HIP(hipMemcpyAsync(S_host, s->S_dbg.ptr, n * n * sizeof(double), hipMemcpyDeviceToHost,
                               stream));
    if (b_host)
        SLK_HIP(hipMemcpyAsync(b_host, s->b_dbg.ptr, n * sizeof(double), hipMemcpyDeviceToHost,
                               stream));
    if (dx_host)
        SLK_HIP(hipMemcpyAsync(dx_host, s->dx_dbg.ptr, n * sizeof(double), hipMemcpyDeviceToHost,
                               stream));
    SLK_HIP(hipStreamSynchronize(stream));
    return SLK_OK;
}

// ----------------------------------------------- reference stage kernels ---
namespace {

// acc[0..77] += weff J J^T (upper triangle of [Ji, Jj]), acc[78..89] += weff r J,
// with Ji[row] = -adj_se3(Jj[row]) per pixel as the reference evaluates it
__device__ __forceinline__ void accum_hessian(const Lin& L, const double (*Ji)[6], bool stereo,
                                              double (&acc)[kNH]) {
#pragma unroll
    for (int row = 0; row < 2; row++) {
        const double we = stereo ? 0.0 : L.w[row];
        double Jx[12];
#pragma unroll
        for (int n = 0; n < 6; n++) {
            Jx[n] = Ji[row][n];
            Jx[6 + n] = L.Jj[row][n];
        }
        int l = 0;
#pragma unroll
        for (int n = 0; n < 12; n++) {
            const double wn = we * Jx[n];
#pragma unroll
            for (int m = 0; m <= n; m++) acc[l++] += wn * Jx[m];
        }
        const double wr = we * L.r[row];
#pragma unroll
        for (int n = 0; n < 12; n++) acc[78 + n] += wr * Jx[n];
    }
}

// projective_transform_kernel (ba.cuh:39-221): one workgroup per edge.
__global__ __launch_bounds__(256) void k_pt(const float* __restrict__ target,
                                            const float* __restrict__ weight,
                                            const float* __restrict__ poses,
                                            const float* __restrict__ disps,
                                            const float* __restrict__ intr,
                                            const int* __restrict__ ii, const int* __restrict__ jj,
                                            float* __restrict__ Hs, float* __restrict__ vs,
                                            float* __restrict__ Eii, float* __restrict__ Eij,
                                            float* __restrict__ Cii, float* __restrict__ bz, int M,
                                            int H, int W) {
    __shared__ double red[kNH * 4];
    __shared__ double rel[7];
    __shared__ double tot[kNH];
    const int e = blockIdx.x;
    const int ix = ii[e], jx = jj[e];
    const bool stereo = ix == jx;
    const int HW = H * W;
    if (threadIdx.x == 0) edge_rel(poses, ix, jx, rel, rel + 3);
    __syncthreads();
    const double tij[3] = {rel[0], rel[1], rel[2]};
    const double qij[4] = {rel[3], rel[4], rel[5], rel[6]};
    const double fx = intr[0], fy = intr[1], cx = intr[2], cy = intr[3];
    double acc[kNH];
#pragma unroll
    for (int n = 0; n < kNH; n++) acc[n] = 0.0;
    for (int k = threadIdx.x; k < HW; k += blockDim.x) {
        const size_t base = (size_t)e * 2 * HW + k;
        Lin L;
        lin_pixel(tij, qij, fx, fy, cx, cy, k, W, (double)disps[(size_t)ix * HW + k],
                  (double)target[base], (double)target[base + HW], (double)weight[base],
                  (double)weight[base + HW], L);
        double Ji[2][6];
#pragma unroll
        for (int row = 0; row < 2; row++) {
            adj_se3(tij, qij, L.Jj[row], Ji[row]);
#pragma unroll
            for (int n = 0; n < 6; n++) Ji[row][n] = -Ji[row][n];
        }
        accum_hessian(L, Ji, stereo, acc);
        Cii[(size_t)e * HW + k] = (float)(L.w[0] * L.Jz[0] * L.Jz[0] + L.w[1] * L.Jz[1] * L.Jz[1]);
        bz[(size_t)e * HW + k] =
            (float)(L.w[0] * L.r[0] * L.Jz[0] + L.w[1] * L.r[1] * L.Jz[1]);
        const double a0 = stereo ? 0.0 : L.w[0] * L.Jz[0];
        const double a1 = stereo ? 0.0 : L.w[1] * L.Jz[1];
        for (int n = 0; n < 6; n++) {
            Eii[((size_t)e * 6 + n) * HW + k] = (float)(a0 * Ji[0][n] + a1 * Ji[1][n]);
            Eij[((size_t)e * 6 + n) * HW + k] = (float)(a0 * L.Jj[0][n] + a1 * L.Jj[1][n]);
        }
    }
    block_sum(acc, red);
    if (threadIdx.x == 0)
        for (int n = 0; n < kNH; n++) tot[n] = acc[n];
    __syncthreads();
    for (int t = threadIdx.x; t < 144; t += blockDim.x) {
        const int blk = t / 36, r = (t % 36) / 6, c = t % 6;
        int idx;
        if (blk == 0) idx = tri(max(r, c), min(r, c));
        else if (blk == 1) idx = tri(6 + c, r);
        else if (blk == 2) idx = tri(6 + r, c);
        else idx = tri(6 + max(r, c), 6 + min(r, c));
        Hs[(size_t)blk * M * 36 + e * 36 + r * 6 + c] = (float)tot[idx];
    }
    if (threadIdx.x < 12) {
        const int which = threadIdx.x / 6, n = threadIdx.x % 6;
        vs[(size_t)which * M * 6 + e * 6 + n] = (float)tot[78 + which * 6 + n];
    }
}

__global__ void k_accum(const float* __restrict__ inps, const int* __restrict__ ptrs,
                        const int* __restrict__ idxs, float* __restrict__ outs, int D, int add) {
    const int row = blockIdx.y;
    const int k = blockIdx.x * blockDim.x + threadIdx.x;
    if (k >= D) return;
    double x = 0.0;
    for (int i = ptrs[row]; i < ptrs[row + 1]; i++) x += (double)inps[(size_t)idxs[i] * D + k];
    float* o = outs + (size_t)row * D + k;
    *o = add ? (float)((double)*o + x) : (float)x;
}

__global__ void k_damping_q(float* __restrict__ C, const float* __restrict__ eta,
                            const int* __restrict__ kf_map, float* __restrict__ Q, int N_kf, int HW,
                            float ep) {
    const long idx = blockIdx.x * (long)blockDim.x + threadIdx.x;
    if (idx >= (long)N_kf * HW) return;
    const int kf = (int)(idx / HW), d = (int)(idx % HW);
    const double c = (double)C[idx] + 0.2 * (double)eta[(size_t)kf_map[kf] * HW + d] + (double)ep;
    C[idx] = (float)c;
    Q[idx] = (float)(1.0 / c);
}

__global__ __launch_bounds__(256) void k_eet(const float* __restrict__ E,
                                             const float* __restrict__ Q,
                                             const int* __restrict__ idx, float* __restrict__ S,
                                             int D) {
    __shared__ double red[36 * 4];
    const int p = blockIdx.x;
    const int ix = idx[p * 3], jx = idx[p * 3 + 1], kx = idx[p * 3 + 2];
    double acc[36];
#pragma unroll
    for (int n = 0; n < 36; n++) acc[n] = 0.0;
    for (int k = threadIdx.x; k < D; k += blockDim.x) {
        const double q = Q[(size_t)kx * D + k];
        double a[6], b[6];
        for (int n = 0; n < 6; n++) {
            a[n] = (double)E[((size_t)ix * 6 + n) * D + k] * q;
            b[n] = (double)E[((size_t)jx * 6 + n) * D + k];
        }
#pragma unroll
        for (int n = 0; n < 6; n++)
#pragma unroll
            for (int m = 0; m < 6; m++) acc[n * 6 + m] += a[n] * b[m];
    }
    block_sum(acc, red);
    if (threadIdx.x == 0)
        for (int n = 0; n < 36; n++) S[(size_t)p * 36 + n] = (float)acc[n];
}

__global__ __launch_bounds__(256) void k_ev(const float* __restrict__ E, const float* __restrict__ Q,
                                            const float* __restrict__ w,
                                            const int* __restrict__ idx, float* __restrict__ v,
                                            int D) {
    __shared__ double red[6 * 4];
    const int r = blockIdx.x;
    const int kx = idx[r];
    double acc[6] = {0, 0, 0, 0, 0, 0};
    for (int k = threadIdx.x; k < D; k += blockDim.x) {
        const double qw = (double)Q[(size_t)kx * D + k] * (double)w[(size_t)kx * D + k];
        for (int n = 0; n < 6; n++) acc[n] += qw * (double)E[((size_t)r * 6 + n) * D + k];
    }
    block_sum(acc, red);
    if (threadIdx.x == 0)
        for (int n = 0; n < 6; n++) v[r * 6 + n] = (float)((double)v[r * 6 + n] + acc[n]);
}

__global__ void k_evt(const float* __restrict__ E, const float* __restrict__ x,
                      const int* __restrict__ idx, float* __restrict__ w, int D, int P) {
    const int r = blockIdx.y;
    const int ix = idx[r];
    if (ix < 0 || ix >= P) return;
    const int k = blockIdx.x * blockDim.x + threadIdx.x;
    if (k >= D) return;
    double dw = 0.0;
    for (int n = 0; n < 6; n++) dw += (double)E[((size_t)r * 6 + n) * D + k] * (double)x[ix * 6 + n];
    w[(size_t)r * D + k] = (float)dw;
}

__global__ void k_depth_update(const float* __restrict__ Q, const float* __restrict__ w,
                               const float* __restrict__ dw, float* __restrict__ disps,
                               const int* __restrict__ kf_map, int N_kf, int HW) {
    const long idx = blockIdx.x * (long)blockDim.x + threadIdx.x;
    if (idx >= (long)N_kf * HW) return;
    const int kf = (int)(idx / HW), d = (int)(idx % HW);
    const double dz = (double)Q[idx] * ((double)w[idx] - (double)dw[idx]);
    float* o = disps + (size_t)kf_map[kf] * HW + d;
    *o = (float)((double)*o + dz);
}

}  // namespace

extern "C" int slk_ba_projective_transform(const float* target, const float* weight,
                                           const float* poses, const float* disps,
                                           const float* intrinsics, const int* ii, const int* jj,
                                           float* Hs, float* vs, float* Eii, float* Eij, float* Cii,
                                           float* bz, int M, int H, int W, hipStream_t stream) {
    if (M <= 0) return SLK_OK;
    if (!target || !weight || !poses || !disps || !intrinsics || !ii || !jj || !Hs || !vs ||
        !Eii || !Eij || !Cii || !bz || H < 1 || W < 1)
        return fail(SLK_E_ARG, "ba_projective_transform: bad args");
    hipLaunchKernelGGL(k_pt, dim3(M), dim3(256), 0, stream, target, weight, poses, disps,
                       intrinsics, ii, jj, Hs, vs, Eii, Eij, Cii, bz, M, H, W);
    SLK_HIP(hipGetLastError());
    return SLK_OK;
}

extern "C" int slk_ba_accum(const float* inps, const int* ptrs, const int* idxs, float* outs,
                            int N_out, int D, int add, hipStream_t stream) {
    if (N_out <= 0 || D <= 0) return SLK_OK;
    if (!inps || !ptrs || !idxs || !outs) return fail(SLK_E_ARG, "ba_accum: null argument");
    hipLaunchKernelGGL(k_accum, dim3((D + 255) / 256, N_out), dim3(256), 0, stream, inps, ptrs,
                       idxs, outs, D, add);
    SLK_HIP(hipGetLastError());
    return SLK_OK;
}

extern "C" int slk_ba_damping_q(float* C, const float* eta, const int* kf_map, float* Q, int N_kf,
                                int HW, float ep, hipStream_t stream) {
    const long total = (long)N_kf * HW;
    if (total <= 0) return SLK_OK;
    if (!C || !eta || !kf_map || !Q) return fail(SLK_E_ARG, "ba_damping_q: null argument");
    hipLaunchKernelGGL(k_damping_q, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, C,
                       eta, kf_map, Q, N_kf, HW, ep);
    SLK_HIP(hipGetLastError());
    return SLK_OK;
}

extern "C" int slk_ba_eet6x6(const float* E, const float* Q, const int* idx, float* S, int D,
                             int N_pairs, hipStream_t stream) {
    if (N_pairs <= 0) return SLK_OK;
    if (!E || !Q || !idx || !S || D <= 0) return fail(SLK_E_ARG, "ba_eet6x6: bad args");
    hipLaunchKernelGGL(k_eet, dim3(N_pairs), dim3(256), 0, stream, E, Q, idx, S, D);
    SLK_HIP(hipGetLastError());
    return SLK_OK;
}

extern "C" int slk_ba_ev6x1(const float* E, const float* Q, const float* w, const int* idx,
                            float* v, int D, int N_v, hipStream_t stream) {
    if (N_v <= 0) return SLK_OK;
    if (!E || !Q || !w || !idx || !v || D <= 0) return fail(SLK_E_ARG, "ba_ev6x1: bad args");
    hipLaunchKernelGGL(k_ev, dim3(N_v), dim3(256), 0, stream, E, Q, w, idx, v, D);
    SLK_HIP(hipGetLastError());
    return SLK_OK;
}

extern "C" int slk_ba_evt6x1(const float* E, const float* x, const int* idx, float* w, int D,
                             int N_E, int P, hipStream_t stream) {
    if (N_E <= 0 || D <= 0) return SLK_OK;
    if (!E || !x || !idx || !w) return fail(SLK_E_ARG, "ba_evt6x1: null argument");
    hipLaunchKernelGGL(k_evt, dim3((D + 255) / 256, N_E), dim3(256), 0, stream, E, x, idx, w, D, P);
    SLK_HIP(hipGetLastError());
    return SLK_OK;
}

extern "C" int slk_ba_depth_update(const float* Q, const float* w, const float* dw, float* disps,
                                   const int* kf_map, int N_kf, int HW, hipStream_t stream) {
    const long total = (long)N_kf * HW;
    if (total <= 0) return SLK_OK;
    if (!Q || !w || !dw || !disps || !kf_map) return fail(SLK_E_ARG, "ba_depth_update: null argument");
    hipLaunchKernelGGL(k_depth_update, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream,
                       Q, w, dw, disps, kf_map, N_kf, HW);
    SLK_HIP(hipGetLastError());
    return SLK_OK;
}
