/*
 * oracle.c -- CPU restatement of the DROID-SLAM per-edge update path
 * (vibekernels/slam-hands, cuda_slam/). TEST INFRASTRUCTURE ONLY: tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg are its only users.
 * The product library never links it, and nothing here is a fallback for it.
 *
 * Everything is carried in fp64 internally; inputs/outputs are fp32 like the
 * reference. Function-level citations are in oracle.h; statement-level ones
 * are inline below.
 */
#include "oracle.h"

#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

#define MIN_DEPTH 0.25 /* se3.cuh:6 */

/* ------------------------------------------------------------------------ */
/* correlation                                                               */
/* ------------------------------------------------------------------------ */

void orc_corr_volume(const float* fi, const float* fj, int C, int HW,
                     double alpha, float* vol) {
    /* main.cu:1508-1515 (column-major GEMM with A=f_j, B=f_i) gives row-major
     * rows = source pixel of frame ii, columns = target pixel of frame jj. */
#pragma omp parallel
    {
        double* acc = (double*)malloc(sizeof(double) * (size_t)HW);
#pragma omp for schedule(static)
        for (int p = 0; p < HW; p++) {
            for (int q = 0; q < HW; q++) acc[q] = 0.0;
            for (int c = 0; c < C; c++) {
                const double a = (double)fi[(size_t)c * HW + p];
                const float* row = fj + (size_t)c * HW;
                for (int q = 0; q < HW; q++) acc[q] += a * (double)row[q];
            }
            float* out = vol + (size_t)p * HW;
            for (int q = 0; q < HW; q++) out[q] = (float)(alpha * acc[q]);
        }
        free(acc);
    }
}

/* IEEE binary16 -> binary32, exact. */
static float half_bits_to_float(unsigned short h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: normalise */
            int e = -1;
            do { e++; man <<= 1; } while ((man & 0x400u) == 0);
            man &= 0x3ffu;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

void orc_corr_volume_f16(const unsigned short* fi, const unsigned short* fj,
                         int C, int HW, double alpha, float* vol) {
    size_t n = (size_t)C * HW;
    float* a = (float*)malloc(n * sizeof(float));
    float* b = (float*)malloc(n * sizeof(float));
    for (size_t k = 0; k < n; k++) {
        a[k] = half_bits_to_float(fi[k]);
        b[k] = half_bits_to_float(fj[k]);
    }
    orc_corr_volume(a, b, C, HW, alpha, vol);
    free(a);
    free(b);
}

void orc_avg_pool_2x2(const float* in, float* out, long N, int H, int W) {
    /* main.cu:1150-1170; cuDNN AVERAGE_COUNT_INCLUDE_PADDING 2x2/2 no padding
     * gives the same floor shapes (nn.cuh:389-410). */
    const int oH = H / 2, oW = W / 2;
    /* small calls run on the calling thread: a thread team costs more */
#pragma omp parallel for schedule(static) if (N * oH * oW >= 65536)
    for (long n = 0; n < N; n++) {
        const float* src = in + (size_t)n * H * W;
        float* dst = out + (size_t)n * oH * oW;
        for (int oy = 0; oy < oH; oy++)
            for (int ox = 0; ox < oW; ox++) {
                const int iy = 2 * oy, ix = 2 * ox;
                float s = src[iy * W + ix];
                s = s + src[iy * W + ix + 1];
                s = s + src[(iy + 1) * W + ix];
                s = s + src[(iy + 1) * W + ix + 1];
                dst[oy * oW + ox] = 0.25f * s;
            }
    }
}

void orc_corr_lookup_level(const float* level, const float* coords, float* out,
                           int r, int H1, int W1, int H2, int W2,
                           float coord_scale, int level_idx) {
    const int D = 2 * r + 1;
    const int hw1 = H1 * W1;
    const size_t plane = (size_t)H2 * W2;
    double* acc = NULL;
#pragma omp parallel private(acc) if (hw1 >= 1024)
    {
        acc = (double*)malloc(sizeof(double) * D * D);
#pragma omp for schedule(static)
        for (int src = 0; src < hw1; src++) {
            /* main.cu:1189-1192: coordinates scaled in fp32, fractions exact */
            const float x0 = coords[0 * hw1 + src] * coord_scale;
            const float y0 = coords[1 * hw1 + src] * coord_scale;
            for (int k = 0; k < D * D; k++) acc[k] = 0.0;
            if (isfinite(x0) && isfinite(y0)) {
                const double fx = floor((double)x0), fy = floor((double)y0);
                const double dx = (double)x0 - fx, dy = (double)y0 - fy;
                /* clamp far-away corners: everything is out of bounds there */
                const long bx = (long)fmax(fmin(fx, 1e9), -1e9);
                const long by = (long)fmax(fmin(fy, 1e9), -1e9);
                const float* vol = level + (size_t)src * plane;
                /* main.cu:1200-1216: corner (i,j) at x = floor(x0)-r+i,
                 * y = floor(y0)-r+j feeds channels (i-1|i)*D + (j-1|j). */
                for (int i = 0; i < D + 1; i++) {
                    for (int j = 0; j < D + 1; j++) {
                        const long x1 = bx - r + i;
                        const long y1 = by - r + j;
                        if (y1 < 0 || y1 >= H2 || x1 < 0 || x1 >= W2) continue;
                        const double s = (double)vol[y1 * W2 + x1];
                        if (i > 0 && j > 0) acc[(i - 1) * D + (j - 1)] += s * dx * dy;
                        if (i > 0 && j < D) acc[(i - 1) * D + j] += s * dx * (1.0 - dy);
                        if (i < D && j > 0) acc[i * D + (j - 1)] += s * (1.0 - dx) * dy;
                        if (i < D && j < D) acc[i * D + j] += s * (1.0 - dx) * (1.0 - dy);
                    }
                }
            }
            float* o = out + (size_t)level_idx * D * D * hw1;
            for (int k = 0; k < D * D; k++) o[(size_t)k * hw1 + src] = (float)acc[k];
        }
        free(acc);
    }
}

void orc_corr_batch(const float* fmaps, int C, int h, int w,
                    const int* ii, const int* jj, int B,
                    const float* coords, float* out,
                    int levels, int r, double alpha) {
    const int HW = h * w;
    const int D = 2 * r + 1;
    const int nch = levels * D * D;
    float* pyr[8] = {0};
    int ph[8], pw[8];
    ph[0] = h;
    pw[0] = w;
    pyr[0] = (float*)malloc(sizeof(float) * (size_t)HW * HW);
    for (int l = 1; l < levels; l++) {
        ph[l] = ph[l - 1] / 2;
        pw[l] = pw[l - 1] / 2;
        pyr[l] = (float*)malloc(sizeof(float) * (size_t)HW * ph[l] * pw[l] + 4);
    }
    for (int e = 0; e < B; e++) {
        const float* fi = fmaps + (size_t)ii[e] * C * HW;
        const float* fj = fmaps + (size_t)jj[e] * C * HW;
        orc_corr_volume(fi, fj, C, HW, alpha, pyr[0]);
        for (int l = 1; l < levels; l++)
            orc_avg_pool_2x2(pyr[l - 1], pyr[l], HW, ph[l - 1], pw[l - 1]);
        for (int l = 0; l < levels; l++) {
            /* main.cu:1606-1611: coord_scale = 1/2^l */
            const float scale = 1.0f / (float)(1 << l);
            orc_corr_lookup_level(pyr[l], coords + (size_t)e * 2 * HW,
                                  out + (size_t)e * nch * HW, r, h, w, ph[l], pw[l],
                                  scale, l);
        }
    }
    for (int l = 0; l < levels; l++) free(pyr[l]);
}

/* ------------------------------------------------------------------------ */
/* SE3 (se3.cuh:8-114)                                                       */
/* ------------------------------------------------------------------------ */

static void act_so3(const double* q, const double* X, double* Y) {
    /* se3.cuh:8-17 */
    double uv[3];
    uv[0] = 2.0 * (q[1] * X[2] - q[2] * X[1]);
    uv[1] = 2.0 * (q[2] * X[0] - q[0] * X[2]);
    uv[2] = 2.0 * (q[0] * X[1] - q[1] * X[0]);
    Y[0] = X[0] + q[3] * uv[0] + (q[1] * uv[2] - q[2] * uv[1]);
    Y[1] = X[1] + q[3] * uv[1] + (q[2] * uv[0] - q[0] * uv[2]);
    Y[2] = X[2] + q[3] * uv[2] + (q[0] * uv[1] - q[1] * uv[0]);
}

void orc_act_se3(const double* t, const double* q, const double* X, double* Y) {
    /* se3.cuh:19-26: homogeneous point [X,Y,Z,W] -> [R X + W t, W] */
    act_so3(q, X, Y);
    Y[3] = X[3];
    Y[0] += X[3] * t[0];
    Y[1] += X[3] * t[1];
    Y[2] += X[3] * t[2];
}

void orc_adj_se3(const double* t, const double* q, const double* X, double* Y) {
    /* se3.cuh:28-41 */
    const double qinv[4] = {-q[0], -q[1], -q[2], q[3]};
    act_so3(qinv, &X[0], &Y[0]);
    act_so3(qinv, &X[3], &Y[3]);
    double u[3], v[3];
    u[0] = t[2] * X[1] - t[1] * X[2];
    u[1] = t[0] * X[2] - t[2] * X[0];
    u[2] = t[1] * X[0] - t[0] * X[1];
    act_so3(qinv, u, v);
    Y[3] += v[0];
    Y[4] += v[1];
    Y[5] += v[2];
}

void orc_rel_se3(const double* ti, const double* qi, const double* tj,
                 const double* qj, double* tij, double* qij) {
    /* se3.cuh:43-54: Tij = Tj * Ti^-1 */
    qij[0] = -qj[3] * qi[0] + qj[0] * qi[3] - qj[1] * qi[2] + qj[2] * qi[1];
    qij[1] = -qj[3] * qi[1] + qj[1] * qi[3] - qj[2] * qi[0] + qj[0] * qi[2];
    qij[2] = -qj[3] * qi[2] + qj[2] * qi[3] - qj[0] * qi[1] + qj[1] * qi[0];
    qij[3] = qj[3] * qi[3] + qj[0] * qi[0] + qj[1] * qi[1] + qj[2] * qi[2];
    act_so3(qij, ti, tij);
    tij[0] = tj[0] - tij[0];
    tij[1] = tj[1] - tij[1];
    tij[2] = tj[2] - tij[2];
}

static void exp_so3(const double* phi, double* q) {
    /* se3.cuh:56-73 */
    const double theta_sq = phi[0] * phi[0] + phi[1] * phi[1] + phi[2] * phi[2];
    const double theta_p4 = theta_sq * theta_sq;
    const double theta = sqrt(theta_sq);
    double imag, real;
    if (theta_sq < 1e-8) {
        imag = 0.5 - (1.0 / 48.0) * theta_sq + (1.0 / 3840.0) * theta_p4;
        real = 1.0 - (1.0 / 8.0) * theta_sq + (1.0 / 384.0) * theta_p4;
    } else {
        imag = sin(0.5 * theta) / theta;
        real = cos(0.5 * theta);
    }
    q[0] = imag * phi[0];
    q[1] = imag * phi[1];
    q[2] = imag * phi[2];
    q[3] = real;
}

static void cross_inplace(const double* a, double* b) {
    /* se3.cuh:75-83: b <- a x b */
    const double x[3] = {a[1] * b[2] - a[2] * b[1], a[2] * b[0] - a[0] * b[2],
                         a[0] * b[1] - a[1] * b[0]};
    b[0] = x[0];
    b[1] = x[1];
    b[2] = x[2];
}

void orc_exp_se3(const double* xi, double* t, double* q) {
    /* se3.cuh:85-101 */
    exp_so3(xi + 3, q);
    double tau[3] = {xi[0], xi[1], xi[2]};
    const double phi[3] = {xi[3], xi[4], xi[5]};
    const double theta_sq = phi[0] * phi[0] + phi[1] * phi[1] + phi[2] * phi[2];
    const double theta = sqrt(theta_sq);
    t[0] = tau[0];
    t[1] = tau[1];
    t[2] = tau[2];
    if (theta > 1e-4) {
        const double a = (1.0 - cos(theta)) / theta_sq;
        cross_inplace(phi, tau);
        t[0] += a * tau[0];
        t[1] += a * tau[1];
        t[2] += a * tau[2];
        const double b = (theta - sin(theta)) / (theta * theta_sq);
        cross_inplace(phi, tau);
        t[0] += b * tau[0];
        t[1] += b * tau[1];
        t[2] += b * tau[2];
    }
}

void orc_retr_se3(const double* xi, const double* t, const double* q,
                  double* t1, double* q1) {
    /* se3.cuh:103-114: T1 = exp(xi) * T (left-multiplicative) */
    double dt[3] = {0, 0, 0};
    double dq[4] = {0, 0, 0, 1};
    orc_exp_se3(xi, dt, dq);
    q1[0] = dq[3] * q[0] + dq[0] * q[3] + dq[1] * q[2] - dq[2] * q[1];
    q1[1] = dq[3] * q[1] + dq[1] * q[3] + dq[2] * q[0] - dq[0] * q[2];
    q1[2] = dq[3] * q[2] + dq[2] * q[3] + dq[0] * q[1] - dq[1] * q[0];
    q1[3] = dq[3] * q[3] - dq[0] * q[0] - dq[1] * q[1] - dq[2] * q[2];
    act_so3(dq, t, t1);
    t1[0] += dt[0];
    t1[1] += dt[1];
    t1[2] += dt[2];
}

static void load_pose(const float* poses, int k, double* t, double* q) {
    for (int n = 0; n < 3; n++) t[n] = (double)poses[k * 7 + n];
    for (int n = 0; n < 4; n++) q[n] = (double)poses[k * 7 + 3 + n];
}

void orc_projmap(const float* poses, const float* disps, const float* intr,
                 const int* ii, const int* jj, float* coords, float* valid,
                 int M, int H, int W) {
    const double fx = intr[0], fy = intr[1], cx = intr[2], cy = intr[3];
    const int HW = H * W;
    for (int e = 0; e < M; e++) {
        double ti[3], qi[4], tj[3], qj[4], tij[3], qij[4];
        load_pose(poses, ii[e], ti, qi);
        load_pose(poses, jj[e], tj, qj);
        orc_rel_se3(ti, qi, tj, qj, tij, qij);
        for (int k = 0; k < HW; k++) {
            /* se3.cuh:158-176 */
            const int i = k / W, j = k % W;
            const double u = (double)j, v = (double)i;
            double Xi[4], Xj[4];
            Xi[0] = (u - cx) / fx;
            Xi[1] = (v - cy) / fy;
            Xi[2] = 1.0;
            Xi[3] = (double)disps[(size_t)ii[e] * HW + k];
            orc_act_se3(tij, qij, Xi, Xj);
            const size_t base = ((size_t)e * HW + k) * 2;
            if (Xj[2] > 0.01) {
                coords[base + 0] = (float)(fx * (Xj[0] / Xj[2]) + cx);
                coords[base + 1] = (float)(fy * (Xj[1] / Xj[2]) + cy);
            } else {
                coords[base + 0] = (float)u;
                coords[base + 1] = (float)v;
            }
            valid[(size_t)e * HW + k] = (Xj[2] > MIN_DEPTH) ? 1.0f : 0.0f;
        }
    }
}

void orc_pose_retr(float* poses, const float* dx, int t0, int t1) {
    /* se3.cuh:179-193 */
    for (int k = t0; k < t1; k++) {
        double xi[6], t[3], q[4], t1_[3], q1_[4];
        load_pose(poses, k, t, q);
        for (int n = 0; n < 6; n++) xi[n] = (double)dx[(k - t0) * 6 + n];
        orc_retr_se3(xi, t, q, t1_, q1_);
        for (int n = 0; n < 3; n++) poses[k * 7 + n] = (float)t1_[n];
        for (int n = 0; n < 4; n++) poses[k * 7 + 3 + n] = (float)q1_[n];
    }
}

void orc_disp_retr(float* disps, const float* dz, const int* inds, int num_inds,
                   int HW) {
    /* se3.cuh:195-206 */
    for (int b = 0; b < num_inds; b++) {
        const int idx = inds[b];
        for (int k = 0; k < HW; k++) {
            const float d = disps[(size_t)idx * HW + k] + dz[(size_t)b * HW + k];
            disps[(size_t)idx * HW + k] = fmaxf(d, 0.001f);
        }
    }
}

void orc_frame_distance(const float* poses, const float* disps, const float* intr,
                        const int* ii, const int* jj, float* dist,
                        int M, int H, int W, float beta_f) {
    /* se3.cuh:209-277 */
    const double fx = intr[0], fy = intr[1], cx = intr[2], cy = intr[3];
    const double beta = (double)beta_f;
    const int HW = H * W;
    for (int e = 0; e < M; e++) {
        double ti[3], qi[4], tj[3], qj[4], tij[3], qij[4];
        load_pose(poses, ii[e], ti, qi);
        load_pose(poses, jj[e], tj, qj);
        orc_rel_se3(ti, qi, tj, qj, tij, qij);
        double accum = 0, valid = 0, total = 0;
        for (int k = 0; k < HW; k++) {
            const int i = k / W, j = k % W;
            const double u = j, v = i;
            double Xi[4], Xj[4];
            Xi[0] = (u - cx) / fx;
            Xi[1] = (v - cy) / fy;
            Xi[2] = 1;
            Xi[3] = disps[(size_t)ii[e] * HW + k];
            orc_act_se3(tij, qij, Xi, Xj);
            double du = fx * (Xj[0] / Xj[2]) + cx - u, dv = fy * (Xj[1] / Xj[2]) + cy - v;
            double d = sqrt(du * du + dv * dv);
            total += beta;
            if (Xj[2] > MIN_DEPTH) {
                accum += beta * d;
                valid += beta;
            }
            /* translation-only term, se3.cuh:252-257 */
            Xj[0] = Xi[0] + Xi[3] * tij[0];
            Xj[1] = Xi[1] + Xi[3] * tij[1];
            Xj[2] = Xi[2] + Xi[3] * tij[2];
            du = fx * (Xj[0] / Xj[2]) + cx - u;
            dv = fy * (Xj[1] / Xj[2]) + cy - v;
            d = sqrt(du * du + dv * dv);
            total += (1 - beta);
            if (Xj[2] > MIN_DEPTH) {
                accum += (1 - beta) * d;
                valid += (1 - beta);
            }
        }
        /* the final test and mean in fp32 as in se3.cuh:274-276: there 4.0f + 1e-8f
           is 4.0f, so a coverage of exactly 0.75 passes (in fp64 it would not) */
        const float vf = (float)valid, tf = (float)total;
        dist[e] = (vf / (tf + 1e-8f) < 0.75f) ? 1000.0f : (float)accum / vf;
    }
}

/* ------------------------------------------------------------------------ */
/* bundle adjustment (ba.cuh)                                                */
/* ------------------------------------------------------------------------ */

void orc_ba_linearize(const float* target, const float* weight,
                      const float* poses, const float* disps, const float* intr,
                      const int* ii, const int* jj,
                      double* Hs, double* vs, double* Eii, double* Eij,
                      double* Cii, double* bz, int M, int H, int W) {
    const double fx = intr[0], fy = intr[1], cx = intr[2], cy = intr[3];
    const int HW = H * W;
    for (int e = 0; e < M; e++) {
        const int ix = ii[e], jx = jj[e];
        double tij[3], qij[4];
        if (ix == jx) {
            /* ba.cuh:73-78: stereo pair, baseline -0.1 */
            tij[0] = -0.1; tij[1] = 0; tij[2] = 0;
            qij[0] = 0; qij[1] = 0; qij[2] = 0; qij[3] = 1;
        } else {
            double ti[3], qi[4], tj[3], qj[4];
            load_pose(poses, ix, ti, qi);
            load_pose(poses, jx, tj, qj);
            orc_rel_se3(ti, qi, tj, qj, tij, qij);
        }
        double hij[78];
        double vi_[6], vj_[6];
        memset(hij, 0, sizeof hij);
        memset(vi_, 0, sizeof vi_);
        memset(vj_, 0, sizeof vj_);
        const float* tg = target + (size_t)e * 2 * HW;
        const float* wt = weight + (size_t)e * 2 * HW;
        double* eii = Eii + (size_t)e * 6 * HW;
        double* eij = Eij + (size_t)e * 6 * HW;
        for (int k = 0; k < HW; k++) {
            /* ba.cuh:104-189 */
            const int i = k / W, j = k % W;
            const double u = j, v = i;
            double Xi[4], Xj[4], Jx[12];
            double* Ji = &Jx[0];
            double* Jj = &Jx[6];
            Xi[0] = (u - cx) / fx;
            Xi[1] = (v - cy) / fy;
            Xi[2] = 1.0;
            Xi[3] = disps[(size_t)ix * HW + k];
            orc_act_se3(tij, qij, Xi, Xj);
            const double x = Xj[0], y = Xj[1], h = Xj[3];
            const double d = (Xj[2] < MIN_DEPTH) ? 0.0 : 1.0 / Xj[2];
            const double d2 = d * d;
            const double wu = (Xj[2] < MIN_DEPTH) ? 0.0 : 0.001 * (double)wt[0 * HW + k];
            const double wv = (Xj[2] < MIN_DEPTH) ? 0.0 : 0.001 * (double)wt[1 * HW + k];
            const double ru = (double)tg[0 * HW + k] - (fx * d * x + cx);
            const double rv = (double)tg[1 * HW + k] - (fy * d * y + cy);

            /* x-coordinate (ba.cuh:126-152) */
            Jj[0] = fx * (h * d);
            Jj[1] = 0;
            Jj[2] = fx * (-x * h * d2);
            Jj[3] = fx * (-x * y * d2);
            Jj[4] = fx * (1 + x * x * d2);
            Jj[5] = fx * (-y * d);
            double Jz = fx * (tij[0] * d - tij[2] * (x * d2));
            double c = wu * Jz * Jz;
            double b = wu * ru * Jz;
            const double wu_eff = (ix == jx) ? 0.0 : wu;
            orc_adj_se3(tij, qij, Jj, Ji);
            for (int n = 0; n < 6; n++) Ji[n] = -Ji[n];
            int l = 0;
            for (int n = 0; n < 12; n++)
                for (int m = 0; m <= n; m++) hij[l++] += wu_eff * Jx[n] * Jx[m];
            for (int n = 0; n < 6; n++) {
                vi_[n] += wu_eff * ru * Ji[n];
                vj_[n] += wu_eff * ru * Jj[n];
                eii[(size_t)n * HW + k] = wu_eff * Jz * Ji[n];
                eij[(size_t)n * HW + k] = wu_eff * Jz * Jj[n];
            }

            /* y-coordinate (ba.cuh:154-188) */
            Jj[0] = 0;
            Jj[1] = fy * (h * d);
            Jj[2] = fy * (-y * h * d2);
            Jj[3] = fy * (-1 - y * y * d2);
            Jj[4] = fy * (x * y * d2);
            Jj[5] = fy * (x * d);
            Jz = fy * (tij[1] * d - tij[2] * (y * d2));
            c += wv * Jz * Jz;
            b += wv * rv * Jz;
            const double wv_eff = (ix == jx) ? 0.0 : wv;
            orc_adj_se3(tij, qij, Jj, Ji);
            for (int n = 0; n < 6; n++) Ji[n] = -Ji[n];
            l = 0;
            for (int n = 0; n < 12; n++)
                for (int m = 0; m <= n; m++) hij[l++] += wv_eff * Jx[n] * Jx[m];
            for (int n = 0; n < 6; n++) {
                vi_[n] += wv_eff * rv * Ji[n];
                vj_[n] += wv_eff * rv * Jj[n];
                eii[(size_t)n * HW + k] += wv_eff * Jz * Ji[n];
                eij[(size_t)n * HW + k] += wv_eff * Jz * Jj[n];
            }
            Cii[(size_t)e * HW + k] = c;
            bz[(size_t)e * HW + k] = b;
        }
        for (int n = 0; n < 6; n++) {
            vs[0 * M * 6 + e * 6 + n] = vi_[n];
            vs[1 * M * 6 + e * 6 + n] = vj_[n];
        }
        /* ba.cuh:198-220: scatter the 12x12 upper triangle into 4 blocks */
        int l = 0;
        for (int n = 0; n < 12; n++) {
            for (int m = 0; m <= n; m++, l++) {
                const double s = hij[l];
                if (n < 6 && m < 6) {
                    Hs[0 * M * 36 + e * 36 + n * 6 + m] = s;
                    Hs[0 * M * 36 + e * 36 + m * 6 + n] = s;
                } else if (n >= 6 && m < 6) {
                    Hs[1 * M * 36 + e * 36 + m * 6 + (n - 6)] = s;
                    Hs[2 * M * 36 + e * 36 + (n - 6) * 6 + m] = s;
                } else {
                    Hs[3 * M * 36 + e * 36 + (n - 6) * 6 + (m - 6)] = s;
                    Hs[3 * M * 36 + e * 36 + (m - 6) * 6 + (n - 6)] = s;
                }
            }
        }
    }
}

int orc_cholesky_solve(double* S, double* b, int N) {
    /* ba.cuh:416-445 (lower Cholesky, forward then backward substitution) */
    for (int j = 0; j < N; j++) {
        double sum = 0;
        for (int k = 0; k < j; k++) sum += S[j * N + k] * S[j * N + k];
        const double piv = S[j * N + j] - sum;
        if (!(piv > 0.0)) return 3;
        S[j * N + j] = sqrt(piv);
        for (int i = j + 1; i < N; i++) {
            double sum2 = 0;
            for (int k = 0; k < j; k++) sum2 += S[i * N + k] * S[j * N + k];
            S[i * N + j] = (S[i * N + j] - sum2) / S[j * N + j];
        }
    }
    for (int i = 0; i < N; i++) {
        double sum = 0;
        for (int k = 0; k < i; k++) sum += S[i * N + k] * b[k];
        b[i] = (b[i] - sum) / S[i * N + i];
    }
    for (int i = N - 1; i >= 0; i--) {
        double sum = 0;
        for (int k = i + 1; k < N; k++) sum += S[k * N + i] * b[k];
        b[i] = (b[i] - sum) / S[i * N + i];
    }
    return 0;
}

int orc_ba_iterate(float* poses, float* disps, const float* intr,
                   const float* target, const float* weight, const float* eta,
                   const int* ii, const int* jj, int M, int nframes,
                   int H, int W, int t0, int t1, float lm, float ep,
                   int motion_only,
                   double* S_out, double* b_out, double* dx_out, double* dz_out) {
    const int HW = H * W;
    const int P = t1 - t0;
    const int n = 6 * P;
    if (P <= 0) return 1;

    double* Hs = (double*)calloc((size_t)4 * M * 36, sizeof(double));
    double* vs = (double*)calloc((size_t)2 * M * 6, sizeof(double));
    double* Eii = (double*)calloc((size_t)M * 6 * HW, sizeof(double));
    double* Eij = (double*)calloc((size_t)M * 6 * HW, sizeof(double));
    double* Cii = (double*)calloc((size_t)M * HW, sizeof(double));
    double* bz = (double*)calloc((size_t)M * HW, sizeof(double));
    orc_ba_linearize(target, weight, poses, disps, intr, ii, jj, Hs, vs, Eii, Eij,
                     Cii, bz, M, H, W);

    double* S = (double*)calloc((size_t)n * n, sizeof(double));
    double* b = (double*)calloc((size_t)n, sizeof(double));
    /* ba.cuh:520-548: dense S/b from the per-edge blocks, in-range endpoints */
    for (int e = 0; e < M; e++) {
        const int i_idx = ii[e] - t0, j_idx = jj[e] - t0;
        const int iv = (i_idx >= 0 && i_idx < P), jv = (j_idx >= 0 && j_idx < P);
        if (!iv && !jv) continue;
        for (int r = 0; r < 6; r++)
            for (int c = 0; c < 6; c++) {
                if (iv) S[(size_t)(i_idx * 6 + r) * n + i_idx * 6 + c] += Hs[0 * M * 36 + e * 36 + r * 6 + c];
                if (iv && jv) {
                    S[(size_t)(i_idx * 6 + r) * n + j_idx * 6 + c] += Hs[1 * M * 36 + e * 36 + r * 6 + c];
                    S[(size_t)(j_idx * 6 + r) * n + i_idx * 6 + c] += Hs[2 * M * 36 + e * 36 + r * 6 + c];
                }
                if (jv) S[(size_t)(j_idx * 6 + r) * n + j_idx * 6 + c] += Hs[3 * M * 36 + e * 36 + r * 6 + c];
            }
        for (int k = 0; k < 6; k++) {
            if (iv) b[i_idx * 6 + k] += vs[0 * M * 6 + e * 6 + k];
            if (jv) b[j_idx * 6 + k] += vs[1 * M * 6 + e * 6 + k];
        }
    }

    /* Schur complement over the depths (ba.cuh:566-743) */
    int N_kf = 0, N_E = 0;
    int* kf_list = NULL;      /* compact kf -> absolute kf, ascending */
    int* kf_compact = NULL;   /* absolute kf -> compact or -1 */
    int* row_pose = NULL;     /* E row -> pose index in [0,P) */
    int* row_kf = NULL;       /* E row -> compact kf */
    double* E = NULL;         /* [N_E][6][HW] */
    double* Cq = NULL;        /* [N_kf][HW]: C, then Q = 1/C */
    double* wv = NULL;        /* [N_kf][HW] */
    if (!motion_only) {
        kf_compact = (int*)malloc(sizeof(int) * (size_t)nframes);
        for (int k = 0; k < nframes; k++) kf_compact[k] = -1;
        for (int e = 0; e < M; e++) kf_compact[ii[e]] = 0;
        kf_list = (int*)malloc(sizeof(int) * (size_t)nframes);
        for (int k = 0; k < nframes; k++)
            if (kf_compact[k] == 0) { kf_compact[k] = N_kf; kf_list[N_kf++] = k; }
        /* E rows keyed by (pose, kf) in order of first appearance, ba.cuh:577-598 */
        int* key = (int*)malloc(sizeof(int) * (size_t)P * nframes);
        for (int k = 0; k < P * nframes; k++) key[k] = -1;
        row_pose = (int*)malloc(sizeof(int) * (size_t)2 * M);
        row_kf = (int*)malloc(sizeof(int) * (size_t)2 * M);
        for (int e = 0; e < M; e++) {
            const int pe[2] = {ii[e] - t0, jj[e] - t0};
            for (int s = 0; s < 2; s++) {
                const int p = pe[s];
                if (p < 0 || p >= P) continue;
                if (key[p * nframes + ii[e]] < 0) {
                    key[p * nframes + ii[e]] = N_E;
                    row_pose[N_E] = p;
                    row_kf[N_E] = kf_compact[ii[e]];
                    N_E++;
                }
            }
        }
        E = (double*)calloc((size_t)N_E * 6 * HW, sizeof(double));
        Cq = (double*)calloc((size_t)N_kf * HW, sizeof(double));
        wv = (double*)calloc((size_t)N_kf * HW, sizeof(double));
        for (int e = 0; e < M; e++) {
            /* accum_kernel / accum_add_kernel (ba.cuh:226-263, 680-695) */
            const int pi = ii[e] - t0, pj = jj[e] - t0;
            if (pi >= 0 && pi < P) {
                double* dst = E + (size_t)key[pi * nframes + ii[e]] * 6 * HW;
                const double* src = Eii + (size_t)e * 6 * HW;
                for (size_t k = 0; k < (size_t)6 * HW; k++) dst[k] += src[k];
            }
            if (pj >= 0 && pj < P) {
                double* dst = E + (size_t)key[pj * nframes + ii[e]] * 6 * HW;
                const double* src = Eij + (size_t)e * 6 * HW;
                for (size_t k = 0; k < (size_t)6 * HW; k++) dst[k] += src[k];
            }
            const int kc = kf_compact[ii[e]];
            for (int k = 0; k < HW; k++) {
                Cq[(size_t)kc * HW + k] += Cii[(size_t)e * HW + k];
                wv[(size_t)kc * HW + k] += bz[(size_t)e * HW + k];
            }
        }
        free(key);
        /* damping_Q_kernel (ba.cuh:266-281), ep fixed at 1e-7 (ba.cuh:701-702) */
        for (int kc = 0; kc < N_kf; kc++)
            for (int k = 0; k < HW; k++) {
                const double c = Cq[(size_t)kc * HW + k] +
                                 0.2 * (double)eta[(size_t)kf_list[kc] * HW + k] + 1e-7;
                Cq[(size_t)kc * HW + k] = 1.0 / c;
            }
        /* EEt6x6 + Ev6x1 (ba.cuh:303-372), subtracted on the host (ba.cuh:722-742) */
        for (int r1 = 0; r1 < N_E; r1++) {
            const int kc = row_kf[r1];
            const double* q = Cq + (size_t)kc * HW;
            const double* w = wv + (size_t)kc * HW;
            const double* e1 = E + (size_t)r1 * 6 * HW;
            for (int r2 = 0; r2 < N_E; r2++) {
                if (row_kf[r2] != kc) continue;
                const double* e2 = E + (size_t)r2 * 6 * HW;
                for (int a = 0; a < 6; a++)
                    for (int c = 0; c < 6; c++) {
                        double s = 0;
                        for (int k = 0; k < HW; k++)
                            s += e1[(size_t)a * HW + k] * q[k] * e2[(size_t)c * HW + k];
                        S[(size_t)(row_pose[r1] * 6 + a) * n + row_pose[r2] * 6 + c] -= s;
                    }
            }
            for (int a = 0; a < 6; a++) {
                double s = 0;
                for (int k = 0; k < HW; k++) s += q[k] * w[k] * e1[(size_t)a * HW + k];
                b[row_pose[r1] * 6 + a] -= s;
            }
        }
    }

    /* LM damping after the Schur step (ba.cuh:749-750) */
    for (int i = 0; i < n; i++)
        S[(size_t)i * n + i] += (double)ep + (double)lm * S[(size_t)i * n + i];
    if (S_out) memcpy(S_out, S, sizeof(double) * (size_t)n * n);
    if (b_out) memcpy(b_out, b, sizeof(double) * (size_t)n);

    int status = orc_cholesky_solve(S, b, n);
    if (status == 0) {
        if (dx_out) memcpy(dx_out, b, sizeof(double) * (size_t)n);
        /* pose_retr_kernel on the fp32-rounded dx (ba.cuh:757-760) */
        float* dxf = (float*)malloc(sizeof(float) * (size_t)n);
        for (int i = 0; i < n; i++) dxf[i] = (float)b[i];
        if (dz_out) memset(dz_out, 0, sizeof(double) * (size_t)nframes * HW);
        if (!motion_only && N_E > 0) {
            /* EvT6x1 + accum + depth_update (ba.cuh:762-783), on the fp32 dx */
            for (int kc = 0; kc < N_kf; kc++) {
                const int kf = kf_list[kc];
                for (int k = 0; k < HW; k++) {
                    double dw = 0;
                    for (int r = 0; r < N_E; r++) {
                        if (row_kf[r] != kc) continue;
                        const double* er = E + (size_t)r * 6 * HW;
                        for (int a = 0; a < 6; a++)
                            dw += er[(size_t)a * HW + k] * (double)dxf[row_pose[r] * 6 + a];
                    }
                    const double dz = Cq[(size_t)kc * HW + k] * (wv[(size_t)kc * HW + k] - dw);
                    if (dz_out) dz_out[(size_t)kf * HW + k] = dz;
                    disps[(size_t)kf * HW + k] = (float)((double)disps[(size_t)kf * HW + k] + dz);
                }
            }
        }
        orc_pose_retr(poses, dxf, t0, t1);
        free(dxf);
    }

    free(Hs); free(vs); free(Eii); free(Eij); free(Cii); free(bz);
    free(S); free(b);
    free(kf_list); free(kf_compact); free(row_pose); free(row_kf);
    free(E); free(Cq); free(wv);
    return status;
}

/* ------------------------------------------------------------------------ */
/* update-pass glue                                                          */
/* ------------------------------------------------------------------------ */

static float clamp64(float v) { return fminf(fmaxf(v, -64.0f), 64.0f); } /* main.cu:1268 */

void orc_compute_motion(float* motion, const float* coords1, const float* coords0,
                        const float* target, int batch, int h, int w) {
    const long HW = (long)h * w;
    for (int e = 0; e < batch; e++)
        for (long k = 0; k < HW; k++) {
            const float* c1 = coords1 + (long)e * 2 * HW;
            const float* tg = target + (long)e * 2 * HW;
            /* coords0_buf holds x = pixel column, y = pixel row (main.cu:2157-2158) */
            const float c0x = coords0 ? coords0[(long)e * 2 * HW + k] : (float)(k % w);
            const float c0y = coords0 ? coords0[(long)e * 2 * HW + HW + k] : (float)(k / w);
            float* m = motion + (long)e * 4 * HW;
            m[k] = clamp64(c1[k] - c0x);                     /* main.cu:1269 */
            m[HW + k] = clamp64(c1[HW + k] - c0y);           /* main.cu:1270 */
            m[2 * HW + k] = clamp64(tg[k] - c1[k]);          /* main.cu:1271 */
            m[3 * HW + k] = clamp64(tg[HW + k] - c1[HW + k]); /* main.cu:1272 */
        }
}

void orc_compute_target(float* target, float* weight_out, const float* coords,
                        const float* delta, const float* wt_raw, int n, int hw) {
    for (int e = 0; e < n; e++)
        for (int c = 0; c < 2; c++)
            for (int k = 0; k < hw; k++) {
                const long o2 = ((long)e * 2 + c) * hw + k, o3 = ((long)e * 3 + c) * hw + k;
                target[o2] = coords[o2] + delta[o3]; /* main.cu:1295-1296 */
                weight_out[o2] = wt_raw[o3];         /* main.cu:1299 */
            }
}

void orc_gather_rows(float* dst, const float* src, const int* idx, int n, long row) {
    for (int e = 0; e < n; e++)
        memcpy(dst + (long)e * row, src + (long)(idx ? idx[e] : e) * row, row * sizeof(float));
}

void orc_scatter_rows(float* dst, const float* src, const int* idx, int n, long row) {
    for (int e = 0; e < n; e++)
        memcpy(dst + (long)(idx ? idx[e] : e) * row, src + (long)e * row, row * sizeof(float));
}

static int cmp_int(const void* a, const void* b) {
    const int x = *(const int*)a, y = *(const int*)b;
    return (x > y) - (x < y);
}

int orc_scatter_mean(float* dst, const float* src, const int* ii, int n, long row,
                     int* active) {
    /* active keyframes: std::set over ii_host, ascending (main.cu:2265-2269) */
    int* tmp = (int*)malloc(sizeof(int) * (n > 0 ? n : 1));
    memcpy(tmp, ii, sizeof(int) * n);
    qsort(tmp, n, sizeof(int), cmp_int);
    int na = 0;
    for (int e = 0; e < n; e++)
        if (na == 0 || tmp[e] != active[na - 1]) active[na++] = tmp[e];
    free(tmp);
    for (int a = 0; a < na; a++) {
        float* d = dst + (long)a * row;
        for (long k = 0; k < row; k++) d[k] = 0.0f; /* cudaMemset, main.cu:2272-2273 */
        int count = 0;
        for (int e = 0; e < n; e++) /* edge order, main.cu:2281-2288 */
            if (ii[e] == active[a]) {
                const float* x = src + (long)e * row;
                for (long k = 0; k < row; k++) d[k] = fmaf(1.0f, x[k], d[k]);
                count++;
            }
        if (count > 1) { /* main.cu:2291-2296 */
            const float inv = 1.0f / (float)count;
            for (long k = 0; k < row; k++) d[k] = fmaf(inv - 1.0f, d[k], d[k]);
        }
    }
    return na;
}

int orc_ba_edge_set(const int* ii, const int* jj, int n, const int* ii_inac,
                    const int* jj_inac, int n_inac, const float* target,
                    const float* weight, const float* target_inac,
                    const float* weight_inac, int hw, int num_keyframes, int forced_t0,
                    int use_inactive, int* ba_ii, int* ba_jj, float* ba_target,
                    float* ba_weight, int* t0_out) {
    int t0 = forced_t0;
    if (t0 < 0) { /* main.cu:2312-2322 */
        int mn = num_keyframes;
        for (int e = 0; e < n; e++) mn = ii[e] < mn ? ii[e] : mn;
        t0 = mn + 1 > 1 ? mn + 1 : 1;
    }
    *t0_out = t0;
    const long r = 2L * hw;
    int m = 0;
    for (int e = 0; e < n; e++, m++) { /* active edges first, main.cu:2331-2333, 2346-2349 */
        ba_ii[m] = ii[e];
        ba_jj[m] = jj[e];
        memcpy(ba_target + m * r, target + e * r, r * sizeof(float));
        memcpy(ba_weight + m * r, weight + e * r, r * sizeof(float));
    }
    if (use_inactive && n_inac > 0) /* main.cu:2330 */
        for (int e = 0; e < n_inac; e++)
            if (ii_inac[e] >= t0 - 3 && jj_inac[e] >= t0 - 3) { /* main.cu:2334-2339, 2351-2361 */
                ba_ii[m] = ii_inac[e];
                ba_jj[m] = jj_inac[e];
                memcpy(ba_target + m * r, target_inac + e * r, r * sizeof(float));
                memcpy(ba_weight + m * r, weight_inac + e * r, r * sizeof(float));
                m++;
            }
    return m;
}

/* ------------------------------------------------------------------------ */
/* factor graph                                                              */
/* ------------------------------------------------------------------------ */

static int has_pair(const int* a, const int* b, int n, int i, int j) {
    for (int e = 0; e < n; e++)
        if (a[e] == i && b[e] == j) return 1;
    return 0;
}

static const float* g_sort_d; /* qsort context (single-threaded use) */
static int cmp_dist_then_index(const void* pa, const void* pb) {
    const int a = *(const int*)pa, b = *(const int*)pb;
    if (g_sort_d[a] < g_sort_d[b]) return -1;
    if (g_sort_d[a] > g_sort_d[b]) return 1;
    return (a > b) - (a < b);
}

static void nms_suppress(float* d, int i, int j, int nms, int t0, int t1, int t, int jrange,
                         int np) {
    /* main.cu:1709-1721 */
    int r = abs(i - j) - 2;
    r = r < nms ? r : nms;
    r = r > 0 ? r : 0;
    for (int di = -nms; di <= nms; di++)
        for (int dj = -nms; dj <= nms; dj++)
            if (abs(di) + abs(dj) <= r) {
                const int i1 = i + di, j1 = j + dj;
                if (i1 >= t0 && i1 < t && j1 >= t1 && j1 < t) {
                    const int idx = (i1 - t0) * jrange + (j1 - t1);
                    if (idx >= 0 && idx < np) d[idx] = 1e6f;
                }
            }
}

int orc_proximity_select(const float* dr, int t, int t0, int t1, int rad, int nms,
                         float thresh, const int* ii, const int* jj, int n,
                         const int* ii_inac, const int* jj_inac, int n_inac,
                         int max_factors, int* new_ii, int* new_jj, int cap, int* n_new) {
    *n_new = 0;
    if (t < 2) return 0; /* main.cu:1682 */
    t0 = t0 > 0 ? t0 : 0;
    t1 = t1 > 0 ? t1 : 0;
    const int jrange = t - t1 > 0 ? t - t1 : 0;
    const int np = (t - t0 > 0 ? t - t0 : 0) * jrange;
    if (np == 0) return 0;
    float* d = (float*)malloc(sizeof(float) * np);
    memcpy(d, dr, sizeof(float) * np);
    for (int k = 0; k < np; k++) { /* main.cu:1702-1706 */
        const int i = t0 + k / jrange, j = t1 + k % jrange;
        if (i - rad < j) d[k] = 1e6f;
        if (d[k] > 100.0f) d[k] = 1e6f;
    }
    for (int e = 0; e < n; e++) nms_suppress(d, ii[e], jj[e], nms, t0, t1, t, jrange, np);
    for (int e = 0; e < n_inac; e++)
        nms_suppress(d, ii_inac[e], jj_inac[e], nms, t0, t1, t, jrange, np);
    /* es: up to 2 edges per neighbour slot and per pair */
    const int es_cap = 2 * ((t - t0) * (rad + 1) + np) + 2;
    int* ei = (int*)malloc(sizeof(int) * es_cap);
    int* ej = (int*)malloc(sizeof(int) * es_cap);
    int ne = 0;
    for (int i = t0; i < t; i++) /* main.cu:1729-1736 */
        for (int j = (i - rad - 1 > 0 ? i - rad - 1 : 0); j < i; j++) {
            if (!has_pair(ii, jj, n, i, j) && !has_pair(ii_inac, jj_inac, n_inac, i, j)) {
                ei[ne] = i; ej[ne++] = j;
                ei[ne] = j; ej[ne++] = i;
            }
            const int idx = (i - t0) * jrange + (j - t1);
            if (idx >= 0 && idx < np) d[idx] = 1e6f;
        }
    int* order = (int*)malloc(sizeof(int) * np);
    for (int k = 0; k < np; k++) order[k] = k;
    g_sort_d = d;
    qsort(order, np, sizeof(int), cmp_dist_then_index); /* main.cu:1739-1742 */
    for (int q = 0; q < np; q++) { /* main.cu:1744-1755 */
        const int k = order[q];
        if (d[k] > thresh) continue;
        if (max_factors > 0 && n + ne > max_factors) break;
        const int i = t0 + k / jrange, j = t1 + k % jrange;
        ei[ne] = i; ej[ne++] = j;
        ei[ne] = j; ej[ne++] = i;
        nms_suppress(d, i, j, nms, t0, t1, t, jrange, np);
    }
    /* main.cu:1773-1781: append what has_edge does not find, growing the set */
    int m = 0;
    for (int q = 0; q < ne; q++) {
        int dup = has_pair(ii, jj, n, ei[q], ej[q]) ||
                  has_pair(ii_inac, jj_inac, n_inac, ei[q], ej[q]);
        for (int r = 0; r < m && !dup && r < cap; r++)
            dup = new_ii[r] == ei[q] && new_jj[r] == ej[q];
        if (dup) continue;
        if (m < cap) { new_ii[m] = ei[q]; new_jj[m] = ej[q]; }
        m++;
    }
    *n_new = m;
    free(d); free(ei); free(ej); free(order);
    return ne;
}

/* ------------------------------------------------------------------------ */
/* factor-graph edge state (main.cu:795-836, 1757-1796)                      */
/* ------------------------------------------------------------------------ */

void orc_oldest_mask(const int* age, int n, int to_remove, unsigned char* mask) {
    /* main.cu:1762-1769: indices sorted by age, largest first, the first
       to_remove masked; equal ages keep edge order (a stable insertion sort,
       where the reference's std::sort leaves their order unspecified) */
    int* order = (int*)malloc(sizeof(int) * (n > 0 ? n : 1));
    for (int e = 0; e < n; e++) {
        int k = e;
        while (k > 0 && age[order[k - 1]] < age[e]) {
            order[k] = order[k - 1];
            k--;
        }
        order[k] = e;
    }
    for (int e = 0; e < n; e++) mask[e] = 0;
    for (int r = 0; r < to_remove && r < n; r++) mask[order[r]] = 1;
    free(order);
}

int orc_store_and_remove_edges(const unsigned char* mask, int n, int* ii, int* jj, int* age,
                               int* ii_inac, int* jj_inac, int* num_inac, int max_inac,
                               float* nets, long net_row, float* target, float* weight,
                               float* target_inac, float* weight_inac, long tw_row) {
    /* main.cu:795-836, one edge at a time with one row copy per array, as
       the reference's cudaMemcpy calls; returns the number of edges kept */
    int kept = 0;
    for (int e = 0; e < n; e++) {
        if (mask[e]) {
            if (*num_inac < max_inac) {
                memcpy(target_inac + (size_t)*num_inac * tw_row, target + (size_t)e * tw_row,
                       sizeof(float) * tw_row);
                memcpy(weight_inac + (size_t)*num_inac * tw_row, weight + (size_t)e * tw_row,
                       sizeof(float) * tw_row);
                ii_inac[*num_inac] = ii[e];
                jj_inac[*num_inac] = jj[e];
                (*num_inac)++;
            }
        } else {
            if (kept != e) {
                memcpy(nets + (size_t)kept * net_row, nets + (size_t)e * net_row,
                       sizeof(float) * net_row);
                memcpy(target + (size_t)kept * tw_row, target + (size_t)e * tw_row,
                       sizeof(float) * tw_row);
                memcpy(weight + (size_t)kept * tw_row, weight + (size_t)e * tw_row,
                       sizeof(float) * tw_row);
            }
            ii[kept] = ii[e];
            jj[kept] = jj[e];
            age[kept] = age[e];
            kept++;
        }
    }
    return kept;
}

void orc_init_new_edges(const float* nets, float* edge_nets, float* weight, const int* ii,
                        int first, int count, long net_row, long tw_row) {
    /* main.cu:1786-1796: edge_nets[e] = nets[ii[e]], weight[e] = 0 */
    for (int e = first; e < first + count; e++) {
        memcpy(edge_nets + (size_t)e * net_row, nets + (size_t)ii[e] * net_row,
               sizeof(float) * net_row);
        memset(weight + (size_t)e * tw_row, 0, sizeof(float) * tw_row);
    }
}

static int rm_kf_edges(int ix, int* ii, int* jj, int* age, int n, float* r1, float* r2,
                       float* r3, long row1, long row23) {
    /* main.cu:889-917 / 920-940: edges touching ix go, indices above ix drop
       by one, the others close up with one copy per row and array */
    int kept = 0;
    for (int e = 0; e < n; e++) {
        int ei = ii[e], ej = jj[e];
        if (ei == ix || ej == ix) continue;
        if (ei > ix) ei--;
        if (ej > ix) ej--;
        if (kept != e) {
            if (r1) memcpy(r1 + (size_t)kept * row1, r1 + (size_t)e * row1, sizeof(float) * row1);
            if (r2) memcpy(r2 + (size_t)kept * row23, r2 + (size_t)e * row23, sizeof(float) * row23);
            if (r3) memcpy(r3 + (size_t)kept * row23, r3 + (size_t)e * row23, sizeof(float) * row23);
        }
        ii[kept] = ei;
        jj[kept] = ej;
        if (age) age[kept] = age[e];
        kept++;
    }
    return kept;
}

void orc_rm_keyframe(int ix, int t, float* poses, float* disps, float* fmaps, long fmap_row,
                     float* nets, float* inps, long net_row, long hw, int* ii, int* jj,
                     int* age, int n, int* n_kept, int* ii_inac, int* jj_inac, int n_inac,
                     int* n_inac_kept, float* edge_nets, float* target, float* weight,
                     float* target_inac, float* weight_inac) {
    /* CudaDroid::rm_keyframe, main.cu:866-941 (fmaps as fmap_row floats of
       raw bytes, whatever their element type) */
    *n_kept = n;
    *n_inac_kept = n_inac;
    if (ix < 0 || ix >= t) return;
    for (int k = ix; k < t - 1; k++) {
        memcpy(poses + (size_t)k * 7, poses + (size_t)(k + 1) * 7, sizeof(float) * 7);
        memcpy(disps + (size_t)k * hw, disps + (size_t)(k + 1) * hw, sizeof(float) * hw);
        memcpy(fmaps + (size_t)k * fmap_row, fmaps + (size_t)(k + 1) * fmap_row,
               sizeof(float) * fmap_row);
        memcpy(nets + (size_t)k * net_row, nets + (size_t)(k + 1) * net_row,
               sizeof(float) * net_row);
        memcpy(inps + (size_t)k * net_row, inps + (size_t)(k + 1) * net_row,
               sizeof(float) * net_row);
    }
    *n_kept = rm_kf_edges(ix, ii, jj, age, n, edge_nets, target, weight, net_row, 2 * hw);
    *n_inac_kept = rm_kf_edges(ix, ii_inac, jj_inac, NULL, n_inac, NULL, target_inac,
                               weight_inac, 0, 2 * hw);
}
