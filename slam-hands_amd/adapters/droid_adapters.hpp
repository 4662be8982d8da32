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
//   CorrBlock         init / build / sample_single / destroy of the
//                     standalone correlation block (corr.cuh:61-263).
//   BundleAdjustment  init / iterate / print_profile / destroy (ba.cuh:397-819),
//                     and iterate_n for the caller's loop of iterates
//                     (main.cu:2371-2389).
//   projmap, pose_retr, frame_distance, clamp_disps
//                     the SE3 kernel launches with the reference's argument
//                     lists (se3.cuh:118-277, main.cu:2392-2397).
//   UpdateModule      init / forward / compute_eta of the update operator with
//                     its ConvGRU (main.cu:535-667), weights from the
//                     reference's exported tensor files.
//   CorrEngine::compute_motion_gru
//                     the frontend's motion filter (main.cu:1934-1983).
//   UpdateGlue        the steps of run_update_pass around correlation and BA
//                     (main.cu:2186-2390): motion and target kernels, the
//                     hidden-state loads and saves, GraphAgg's scatter-mean
//                     and eta write-back, and the BA edge set.
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
#include <cstring>
#include <vector>

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
        if (prepared_ > 0)
            check(slk_corr_batch_build_and_sample_prepared(
                      ctx_, ii_host_ + edge_start, jj_host_ + edge_start, batch_size,
                      coords_2hw, corr_out_196hw, nullptr),
                  "batch_build_and_sample_correlation");
        else
            check(slk_corr_batch_build_and_sample(ctx_, fmaps_, dtype_, frame_stride(),
                                                  ii_host_ + edge_start, jj_host_ + edge_start,
                                                  batch_size, coords_2hw, corr_out_196hw,
                                                  nullptr),
                  "batch_build_and_sample_correlation");
    }

    // Optional: split keyframes [0, nframes) once (at the start of an update
    // pass); the batched calls then skip per-call feature preparation until
    // unprepare() or the next prepare_frames(). Call it again when fmaps change.
    void prepare_frames(int nframes) {
        check(slk_corr_prepare_frames(ctx_, fmaps_, dtype_, frame_stride(), nframes, nullptr),
              "prepare_frames");
        prepared_ = nframes;
    }
    void unprepare() { prepared_ = 0; }

    // corr_volume (l = 0) / corr_pyramid[l] of the last build (main.cu:1324-1326).
    const float* corr_level(int l, int* h2 = nullptr, int* w2 = nullptr) {
        const float* p = nullptr;
        int a = 0, b = 0;
        check(slk_corr_level(ctx_, l, &p, &a, &b), "corr_level");
        if (h2) *h2 = a;
        if (w2) *w2 = b;
        return p;
    }

    // main.cu:1934 -- the motion filter between keyframe last_kf_idx and the
    // frame in temp_slot of the fmaps, from that keyframe's hidden state and
    // context (nets/inps [n][128][h*w]); returns the mean flow magnitude.
    float compute_motion_gru(slk_update* update, int last_kf_idx, int temp_slot,
                             const float* nets, const float* inps) {
        float mean = 0.0f;
        const long row = 128L * h_ * w_;
        check(slk_motion_filter(ctx_, update, frame(last_kf_idx), frame(temp_slot), dtype_,
                                nets + last_kf_idx * row, inps + last_kf_idx * row, &mean,
                                nullptr),
              "compute_motion_gru");
        return mean;
    }

    void destroy() {
        if (ctx_) slk_destroy(ctx_);
        ctx_ = nullptr;
    }

    slk_ctx* context() const { return ctx_; }

  private:
    int prepared_ = 0;
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

// CorrBlock of cuda_slam/corr.cuh:61-263 with its member signatures. The
// reference passes cuBLAS and cuDNN handles to init; this path has no such
// handles, so the two parameters are opaque pointers that are accepted and
// ignored. build(fmap1, fmap2, bn, c, h, w) keeps the volume of pair n = 0,
// the one sample_single reads (corr.cuh:234-256 samples corr_pyramid[l] from
// its start); the reference's batched sample() mis-addresses its output
// (corr.cuh:186-231) and is not offered. The scale is the one the live
// correlation path uses, 1/16 (main.cu:1506,1572), not corr.cuh:100's 1/c;
// set_scale() changes it. The context is created on the first build and
// again whenever (c, h, w) change.
class CorrBlock {
  public:
    using BlasHandle = void*;
    using DnnHandle = void*;

    void init(BlasHandle /*cublas*/, DnnHandle /*cudnn*/, int num_lvl = 4, int rad = 3) {
        num_levels = num_lvl;
        radius = rad;
    }

    void set_scale(float alpha) {
        if (alpha != scale_) release();
        scale_ = alpha;
    }

    // fmap1, fmap2: [bn][c][h][w] fp32 device arrays (corr.cuh:84).
    void build(float* fmap1, float* fmap2, int bn, int c, int h, int w) {
        if (bn < 1) check(SLK_E_ARG, "CorrBlock::build (bn < 1)");
        if (!ctx_ || c != C || h != H || w != W) {
            release();
            check(slk_create(&ctx_, h, w, c, 1, num_levels, radius, scale_),
                  "CorrBlock::build");
        }
        BN = bn;
        C = c;
        H = h;
        W = w;
        check(slk_corr_build(ctx_, fmap1, fmap2, SLK_F32, nullptr), "CorrBlock::build");
    }

    // coords [2][H][W] -> output [num_levels * 49][H][W] (corr.cuh:234-256);
    // coords_scaled_buf is the reference's scratch and is not used here.
    void sample_single(float* coords, float* output, float* /*coords_scaled_buf*/) {
        if (!ctx_) check(SLK_E_STATE, "CorrBlock::sample_single before build");
        check(slk_corr_sample(ctx_, coords, output, nullptr), "CorrBlock::sample_single");
    }

    void destroy() { release(); }

    int num_levels = 4;
    int radius = 3;
    int BN = 0, H = 0, W = 0, C = 0;

  private:
    void release() {
        if (ctx_) slk_destroy(ctx_);
        ctx_ = nullptr;
    }
    slk_ctx* ctx_ = nullptr;
    float scale_ = 1.0f / 16.0f;
};

// UpdateModule of cuda_slam/main.cu:535-667 with its member signatures. The
// reference's init takes a cuDNN handle and a WeightStore reading
// <dir>/<name>.bin tensor files; here the handle is an opaque pointer that is
// ignored and the store is its directory. forward/compute_eta keep the
// reference's argument lists; the temp buffers and workspace the reference
// passes are not needed (the module owns its activations) and may be null.
class UpdateModule {
  public:
    void init(void* /*cudnn*/, const char* weight_dir, int batch, int h, int w) {
        h_ = h;
        w_ = w;
        check(slk_update_create(&um_, batch, h, w), "UpdateModule::init");
        check(slk_update_load_dir(um_, weight_dir), "UpdateModule::init (weights)");
    }

    // main.cu:606
    void forward(void* /*cudnn*/, float* corr_features, float* motion, float* net, float* inp,
                 float* delta_out, float* weight_out, float* agg_conv1_out, float* /*temp1*/,
                 float* /*temp2*/, float* /*workspace*/, int batch, int h, int w) {
        if (h != h_ || w != w_) check(SLK_E_ARG, "UpdateModule::forward (map size)");
        check(slk_update_forward(um_, corr_features, motion, net, inp, delta_out, weight_out,
                                 agg_conv1_out, batch, nullptr),
              "UpdateModule::forward");
    }

    // main.cu:654
    void compute_eta(void* /*cudnn*/, float* agg_features, float* eta_out, float* /*temp1*/,
                     float* /*temp2*/, float* /*workspace*/, int num_kf, int h, int w) {
        if (h != h_ || w != w_) check(SLK_E_ARG, "UpdateModule::compute_eta (map size)");
        check(slk_update_compute_eta(um_, agg_features, eta_out, num_kf, nullptr),
              "UpdateModule::compute_eta");
    }

    void destroy() {
        if (um_) slk_update_destroy(um_);
        um_ = nullptr;
    }

    slk_update* module() const { return um_; }

  private:
    slk_update* um_ = nullptr;
    int h_ = 0, w_ = 0;
};

// HalfBasicEncoder of cuda_slam/main.cu:306-381 with its member signatures.
// init takes the reference's cuDNN handle (ignored) and a WeightStore; here
// the store is its directory, and the prefix ("fnet" / "cnet") names the
// weight files <dir>/<prefix>_<layer>_weight.bin as load_conv does. forward
// keeps the reference's argument list; its three half buffers and the
// workspace are not needed (the encoder owns its activations) and may be
// null.
class HalfBasicEncoder {
  public:
    void init(void* /*cudnn*/, const char* weight_dir, const char* prefix, int batch, int inH,
              int inW, int out_dim, bool use_norm) {
        check(slk_encoder_create(&enc_, inH, inW, out_dim, use_norm ? 1 : 0, batch),
              "HalfBasicEncoder::init");
        check(slk_encoder_load_dir(enc_, weight_dir, prefix), "HalfBasicEncoder::init (weights)");
    }

    // main.cu:357: FP32 input [batch][3][inH][inW] -> FP16 output
    void forward(void* /*cudnn*/, float* input, void* output_half, void* /*buf_a*/,
                 void* /*buf_b*/, void* /*buf_c*/, float* /*workspace*/, int batch, int /*inH*/,
                 int /*inW*/) {
        check(slk_encoder_forward(enc_, input, output_half, batch, nullptr),
              "HalfBasicEncoder::forward");
    }

    void destroy() {
        if (enc_) slk_encoder_destroy(enc_);
        enc_ = nullptr;
    }

    slk_encoder* encoder() const { return enc_; }

  private:
    slk_encoder* enc_ = nullptr;
};

// CudaDroid::encode_frame (main.cu:1465-1497): the BGR frame [H][W][3] ->
// fmap (fp16, the keyframe's slot of state.fmaps), net = tanh and inp = relu
// of the context halves (fp32).
inline void encode_frame(HalfBasicEncoder& fnet, HalfBasicEncoder& cnet, float* bgr_hwc,
                         void* fmap_half, float* net, float* inp) {
    check(slk_encode_frame(fnet.encoder(), cnet.encoder(), bgr_hwc, fmap_half, net, inp, nullptr),
          "encode_frame");
}

// The decode-side conversions of main.cu:2729-2753 (launch shapes are the
// library's own): NV12 / P010 planes from the hardware decoder, or a
// CPU-decoded 8-bit BGR upload, to the float BGR frame of process_frame.
inline void nv12_to_bgr_resize(const uint8_t* y, const uint8_t* uv, float* bgr, int src_w,
                               int src_h, int y_stride, int uv_stride, int dst_w, int dst_h) {
    check(slk_nv12_to_bgr(y, uv, bgr, src_w, src_h, y_stride, uv_stride, dst_w, dst_h, nullptr),
          "nv12_to_bgr_resize");
}
inline void p010_to_bgr_resize(const uint16_t* y, const uint16_t* uv, float* bgr, int src_w,
                               int src_h, int y_stride_bytes, int uv_stride_bytes, int dst_w,
                               int dst_h) {
    check(slk_p010_to_bgr(y, uv, bgr, src_w, src_h, y_stride_bytes, uv_stride_bytes, dst_w,
                          dst_h, nullptr),
          "p010_to_bgr_resize");
}
inline void bgr8_to_bgrf_resize(const uint8_t* bgr8, float* bgr, int src_w, int src_h,
                                int src_stride, int dst_w, int dst_h) {
    check(slk_bgr8_to_bgrf(bgr8, bgr, src_w, src_h, src_stride, dst_w, dst_h, nullptr),
          "bgr8_to_bgrf_resize");
}

// The pose file written at the end of a run (main.cu:2893-2937): poses are
// the host copy of state.poses, timestamps the keyframes' frame indices.
inline void save_poses(const char* path, int num_keyframes, const int* timestamps,
                       const float* poses_host, bool cam_to_world) {
    check(slk_write_poses_bin(path, num_keyframes, timestamps, poses_host, cam_to_world ? 1 : 0),
          "save_poses");
}

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

    // The caller's loop of `iters` iterate() calls on one edge set
    // (run_update_pass, main.cu:2371-2389) as one call: the steps run back to
    // back on the stream, fused where the edge set allows, and the call
    // returns with poses and disps final. A step whose system is not positive
    // definite changes neither poses nor disps, as in iterate().
    void iterate_n(float* poses, float* disps, float* intrinsics, float* target, float* weight,
                   float* eta, int* ii_gpu, int* jj_gpu, int* ii_host, int* jj_host,
                   int num_edges, int t0, int t1, float lm, float ep, bool motion_only,
                   int iters) {
        check(slk_ba_iterate_n(ctx_, poses, disps, intrinsics, target, weight, eta, ii_gpu,
                               jj_gpu, ii_host, jj_host, num_edges, t0, t1, lm, ep,
                               motion_only ? 1 : 0, iters, nullptr),
              "BundleAdjustment::iterate_n");
        const int st = slk_ba_status(ctx_, nullptr);
        if (st == SLK_E_NOT_SPD)
            std::fprintf(stderr, "BundleAdjustment::iterate_n: system not positive definite; "
                                 "rejected steps left poses and disps unchanged\n");
        else
            check(st, "BundleAdjustment::iterate_n");
    }

    // Totals per kernel over the iterates since enable_profile(true)
    // (ba.cuh:805 prints its totals over prof_count iterations).
    void print_profile() {
        for (int k = 0;; k++) {
            const char* name = nullptr;
            double ms = 0.0;
            int n = 0;
            if (slk_profile_kernel(ctx_, k, &name, &ms, &n) != SLK_OK || !name) break;
            std::printf("  %-16s %9.3f ms  (%d launches)\n", name, ms, n);
        }
    }

    // Starts (clearing earlier totals) or stops the per-kernel timing.
    void enable_profile(bool on) { check(slk_profile_enable(ctx_, on ? 1 : 0), "profile"); }

    // Launch count of the named kernel in the current totals (0 if none).
    int profiled_launches(const char* kernel) {
        for (int k = 0;; k++) {
            const char* name = nullptr;
            double ms = 0.0;
            int n = 0;
            if (slk_profile_kernel(ctx_, k, &name, &ms, &n) != SLK_OK || !name) return 0;
            if (std::strcmp(name, kernel) == 0) return n;
        }
    }

    void destroy() {
        if (ctx_) slk_destroy(ctx_);
        ctx_ = nullptr;
    }

    slk_ctx* context() const { return ctx_; }

  private:
    slk_ctx* ctx_ = nullptr;
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

// The update-pass glue of CudaDroid::run_update_pass for h x w maps with the
// reference's 128-channel hidden states (rows of 128*h*w floats), ordered on
// the legacy default stream like the reference's launches and copies.
class UpdateGlue {
  public:
    void init(int h, int w) {
        h_ = h;
        w_ = w;
        check(slk_create(&ctx_, h, w, 128, 1, 1, 3, 1.0f / 16.0f), "UpdateGlue::init");
    }

    // compute_motion_kernel (main.cu:2204-2213); coords0 == nullptr is the
    // identity grid coords0_buf holds
    void compute_motion(float* motion, const float* coords1, const float* coords0,
                        const float* target, int batch) {
        check(slk_compute_motion(motion, coords1, coords0, target, batch, h_, w_, nullptr),
              "compute_motion");
    }

    // compute_target_kernel (main.cu:2234-2242)
    void compute_target(float* target, float* weight_out, const float* coords,
                        const float* delta, const float* wt_raw, int num_edges) {
        check(slk_compute_target(target, weight_out, coords, delta, wt_raw, num_edges,
                                 h_ * w_, nullptr),
              "compute_target");
    }

    // step 5, main.cu:2216-2224: batch_nets[e] = edge_nets[bs + e],
    // batch_inps[e] = inps[ii[bs + e]] (ii_gpu: the device copy of ii_host)
    void load_hidden(float* batch_nets, float* batch_inps, const float* edge_nets,
                     const float* inps, const int* ii_gpu, int bs, int batch_size) {
        const long row = 128L * h_ * w_;
        check(slk_gather_rows(batch_nets, edge_nets + bs * row, nullptr, batch_size, row,
                              nullptr),
              "load_hidden");
        check(slk_gather_rows(batch_inps, inps, ii_gpu + bs, batch_size, row, nullptr),
              "load_hidden");
    }

    // step 8, main.cu:2245-2252: edge_nets[bs + e] = batch_nets[e],
    // all_agg1[bs + e] = batch_agg1[e]
    void save_hidden(float* edge_nets, float* all_agg1, const float* batch_nets,
                     const float* batch_agg1, int bs, int batch_size) {
        const long row = 128L * h_ * w_;
        check(slk_scatter_rows(edge_nets + bs * row, batch_nets, nullptr, batch_size, row,
                               nullptr),
              "save_hidden");
        check(slk_scatter_rows(all_agg1 + bs * row, batch_agg1, nullptr, batch_size, row,
                               nullptr),
              "save_hidden");
    }

    // GraphAgg scatter_mean (main.cu:2258-2296) into kf_agg; returns the
    // active keyframes (ascending) and writes them to active_kf_gpu
    std::vector<int> scatter_mean(float* kf_agg, const float* all_agg1, const int* ii_host,
                                  int total_edges, int* active_kf_gpu) {
        std::vector<int> act(total_edges > 0 ? total_edges : 1);
        int na = 0;
        check(slk_scatter_mean(ctx_, kf_agg, all_agg1, ii_host, total_edges,
                               128L * h_ * w_, active_kf_gpu, act.data(), &na, nullptr),
              "scatter_mean");
        act.resize(na);
        return act;
    }

    // main.cu:2303-2309: damping[active[i]] = kf_eta[i]
    void write_eta(float* damping, const float* kf_eta, const int* active_kf_gpu,
                   int num_active) {
        check(slk_scatter_rows(damping, kf_eta, active_kf_gpu, num_active, (long)h_ * w_,
                               nullptr),
              "write_eta");
    }

    // steps 9-10, main.cu:2312-2369: t0 and the combined edge set; returns
    // the edge count (ba_ii_host/ba_jj_host sized n + n_inac)
    int ba_edge_set(const int* ii_host, const int* jj_host, int n, const int* ii_inac,
                    const int* jj_inac, int n_inac, const float* target, const float* weight,
                    const float* target_inac, const float* weight_inac, int num_keyframes,
                    int forced_t0, bool use_inactive, int* ba_ii_host, int* ba_jj_host,
                    int* ba_ii_gpu, int* ba_jj_gpu, float* ba_target, float* ba_weight,
                    int* t0) {
        int count = 0;
        check(slk_ba_edge_set(ctx_, ii_host, jj_host, n, ii_inac, jj_inac, n_inac, target,
                              weight, target_inac, weight_inac, h_ * w_, num_keyframes,
                              forced_t0, use_inactive ? 1 : 0, ba_ii_host, ba_jj_host,
                              ba_ii_gpu, ba_jj_gpu, ba_target, ba_weight, &count, t0, nullptr),
              "ba_edge_set");
        return count;
    }

    void destroy() {
        if (ctx_) slk_destroy(ctx_);
        ctx_ = nullptr;
    }

  private:
    int h_ = 0, w_ = 0;
    slk_ctx* ctx_ = nullptr;
};

}  // namespace slk_droid
