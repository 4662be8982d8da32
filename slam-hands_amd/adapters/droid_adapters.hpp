// C++ adapters over the libslk C ABI that keep the member-function spellings
// and argument lists of the reference's correlation and bundle-adjustment code
// (vibekernels/slam-hands cuda_slam), so a host written against those classes
// switches to the MI355X path by swapping the type.
//
//   CorrEngine        the correlation members of CudaDroid:
//                     build_correlation / sample_correlation /
//                     batch_build_and_sample_correlation (main.cu:1500-1613),
//                     reading the same state (fmaps [n][128][h][w], the host
//                     edge arrays ii_host/jj_host) the reference reads from
//                     DroidState.
//   BundleAdjustment  init / iterate / print_profile / destroy (ba.cuh:397-819).
//   projmap, pose_retr, frame_distance, clamp_disps
//                     the SE3 kernel launches with the reference's argument
//                     lists (se3.cuh:118-277, main.cu:2392-2397).
//
// Error behaviour follows the reference: its *_CHECK macros print and exit(1)
// (nn.cuh:17-41), and so does every adapter on a nonzero status. The single
// exception is a non-positive-definite BA system: the reference writes NaN
// poses there (ba.cuh:422) and carries on; the adapter reports it on stderr,
// leaves poses and disps untouched and carries on.
//
// Synchronisation follows the reference too: BundleAdjustment::iterate
// returns with poses/disps final (the reference copies to the host inside),
// and the correlation calls are ordered on the legacy default stream, as the
// reference's launches are.
#pragma once

#include <cstdio>
#include <cstdlib>

#include <hip/hip_runtime_api.h>

#include "slk.h"

namespace slk_droid {

inline void check(int status, const char* what) {
    if (status != SLK_OK) {
        std::fprintf(stderr, "%s failed (%d): %s\n", what, status, slk_last_error());
        std::exit(1);
    }
}

// Correlation of CudaDroid. `fmaps` are the keyframe feature maps
// ([n][C][h][w], fp16 as DroidState::fmaps, main.cu:677, or fp32); `ii_host`
// and `jj_host` the edge arrays batch_build_and_sample_correlation indexes
// with edge_start (main.cu:1561-1562). The pointers are read at every call,
// like the reference's members.
class CorrEngine {
  public:
    void init(int h, int w, const void* fmaps, slk_dtype dtype, const int* ii_host,
              const int* jj_host, int max_batch = 48, int C = 128,
              float corr_scale = 1.0f / 16.0f) {
        h_ = h;
        w_ = w;
        C_ = C;
        fmaps_ = fmaps;
        dtype_ = dtype;
        ii_host_ = ii_host;
        jj_host_ = jj_host;
        check(slk_create(&ctx_, h, w, C, max_batch, 4, 3, corr_scale), "CorrEngine::init");
    }

    // main.cu:1500 -- volume of frames (i, j) and its pyramid, kept for
    // sample_correlation and corr_level.
    void build_correlation(int i, int j) {
        check(slk_corr_build(ctx_, frame(i), frame(j), dtype_, nullptr), "build_correlation");
    }

    // main.cu:1529 -- lookup of the last built volume: corr_out [196][h*w].
    void sample_correlation(float* coords_2hw, float* corr_out) {
        check(slk_corr_sample(ctx_, coords_2hw, corr_out, nullptr), "sample_correlation");
    }

    // main.cu:1555 -- edges [edge_start, edge_start + batch_size) of the host
    // edge arrays; coords [B][2][h*w] -> corr_out [B][196][h*w].
    void batch_build_and_sample_correlation(int batch_size, int edge_start, float* coords_2hw,
                                            float* corr_out_196hw) {
        check(slk_corr_batch_build_and_sample(ctx_, fmaps_, dtype_, frame_stride(),
                                              ii_host_ + edge_start, jj_host_ + edge_start,
                                              batch_size, coords_2hw, corr_out_196hw, nullptr),
              "batch_build_and_sample_correlation");
    }

    // corr_volume (l = 0) / corr_pyramid[l] of the last build (main.cu:1324-1326).
    const float* corr_level(int l, int* h2 = nullptr, int* w2 = nullptr) {
        const float* p = nullptr;
        int a = 0, b = 0;
        check(slk_corr_level(ctx_, l, &p, &a, &b), "corr_level");
        if (h2) *h2 = a;
        if (w2) *w2 = b;
        return p;
    }

    void destroy() {
        if (ctx_) slk_destroy(ctx_);
        ctx_ = nullptr;
    }

    slk_ctx* context() const { return ctx_; }

  private:
    long frame_stride() const { return (long)C_ * h_ * w_; }
    const void* frame(int k) const {
        const size_t esz = dtype_ == SLK_F16 ? 2 : 4;
        return static_cast<const char*>(fmaps_) + (size_t)k * frame_stride() * esz;
    }

    slk_ctx* ctx_ = nullptr;
    int h_ = 0, w_ = 0, C_ = 0;
    const void* fmaps_ = nullptr;
    slk_dtype dtype_ = SLK_F16;
    const int* ii_host_ = nullptr;
    const int* jj_host_ = nullptr;
};

// BundleAdjustment of cuda_slam/ba.cuh:397-819 (and, with motion_only, the
// pipeline variant cuda_pipeline/slam.cuh:1475-1592).
class BundleAdjustment {
  public:
    void init(int h, int w) {
        check(slk_create(&ctx_, h, w, 128, 1, 1, 3, 1.0f / 16.0f), "BundleAdjustment::init");
    }

    void iterate(float* poses, float* disps, float* intrinsics, float* target, float* weight,
                 float* eta, int* ii_gpu, int* jj_gpu, int* ii_host, int* jj_host,
                 int num_edges, int t0, int t1, float lm, float ep, bool motion_only) {
        if (profile_) check(slk_profile_enable(ctx_, 1), "profile");
        check(slk_ba_iterate(ctx_, poses, disps, intrinsics, target, weight, eta, ii_gpu, jj_gpu,
                             ii_host, jj_host, num_edges, t0, t1, lm, ep, motion_only ? 1 : 0,
                             nullptr),
              "BundleAdjustment::iterate");
        const int st = slk_ba_status(ctx_, nullptr);  // synchronises, as the reference does
        if (st == SLK_E_NOT_SPD)
            std::fprintf(stderr, "BundleAdjustment::iterate: system not positive definite; "
                                 "poses and disps left unchanged\n");
        else
            check(st, "BundleAdjustment::iterate");
    }

    // Totals per kernel since the first profiled iterate (ba.cuh:805).
    void print_profile() {
        for (int k = 0;; k++) {
            const char* name = nullptr;
            double ms = 0.0;
            int n = 0;
            if (slk_profile_kernel(ctx_, k, &name, &ms, &n) != SLK_OK || !name) break;
            std::printf("  %-16s %9.3f ms  (%d launches)\n", name, ms, n);
        }
    }

    void enable_profile(bool on) { profile_ = on; }

    void destroy() {
        if (ctx_) slk_destroy(ctx_);
        ctx_ = nullptr;
    }

    slk_ctx* context() const { return ctx_; }

  private:
    slk_ctx* ctx_ = nullptr;
    bool profile_ = false;
};

// projmap_kernel<<<M, 256>>>(poses, disps, intr, ii, jj, coords, valid, M, H, W)
// (se3.cuh:118-177; caller main.cu:2189-2193)
inline void projmap(float* poses, float* disps, float* intrinsics, int* ii, int* jj,
                    float* coords, float* valid, int M, int H, int W) {
    check(slk_projmap(poses, disps, intrinsics, ii, jj, coords, valid, M, H, W, nullptr),
          "projmap");
}

// pose_retr_kernel<<<1, ...>>>(poses, dx, t0, t1) (se3.cuh:179-193)
inline void pose_retr(float* poses, float* dx, int t0, int t1) {
    check(slk_pose_retr(poses, dx, t0, t1, nullptr), "pose_retr");
}

// frame_distance_kernel (se3.cuh:209-277; callers main.cu:1637-1676)
inline void frame_distance(float* poses, float* disps, float* intrinsics, int* ii, int* jj,
                           float* dist, int M, int H, int W, float beta) {
    check(slk_frame_distance(poses, disps, intrinsics, ii, jj, dist, M, H, W, beta, nullptr),
          "frame_distance");
}

// clamp_disps_kernel (main.cu:2392-2397)
inline void clamp_disps(float* disps, int n, float min_val) {
    check(slk_clamp_disps(disps, n, min_val, nullptr), "clamp_disps");
}

}  // namespace slk_droid
