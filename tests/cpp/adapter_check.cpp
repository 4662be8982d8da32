// Test harness for slam-hands_amd/adapters/droid_adapters.hpp: drives the C++
// adapters the way the reference's host code drives CudaDroid and
// BundleAdjustment (device buffers, host edge arrays, legacy default stream),
// from host arrays handed over by the Python tests. Built into
// tests/cpp/libadapter_check.so and loaded in-process with ctypes.
#include <hip/hip_runtime.h>

#include <cstring>
#include <vector>

#include "../../slam-hands_amd/adapters/droid_adapters.hpp"

namespace {

template <typename T>
T* upload(const T* host, size_t n) {
    T* d = nullptr;
    if (hipMalloc(&d, n * sizeof(T)) != hipSuccess) return nullptr;
    if (hipMemcpy(d, host, n * sizeof(T), hipMemcpyHostToDevice) != hipSuccess) return nullptr;
    return d;
}

template <typename T>
int download(T* host, const T* dev, size_t n) {
    return hipMemcpy(host, dev, n * sizeof(T), hipMemcpyDeviceToHost) == hipSuccess ? 0 : 1;
}

}  // namespace

// Batched correlation of edges [0, B) through CorrEngine (two calls: edges
// [0, B/2) and [B/2, B), exercising edge_start) and the single-edge
// build_correlation(ii[0], jj[0]) + sample_correlation of edge 0's coords.
// fmaps [nframes][128][h][w] of dtype (0 f32, 1 f16); coords [B][2][h*w];
// out_batch [B][196][h*w]; out_single [196][h*w].
extern "C" int adapter_corr(const void* fmaps, int dtype, int nframes, int h, int w,
                            const int* ii, const int* jj, int B, const float* coords,
                            float* out_batch, float* out_single) {
    const size_t hw = (size_t)h * w;
    const size_t esz = dtype == SLK_F16 ? 2 : 4;
    const size_t fbytes = (size_t)nframes * 128 * hw * esz;
    void* d_f = nullptr;
    if (hipMalloc(&d_f, fbytes) != hipSuccess) return 1;
    if (hipMemcpy(d_f, fmaps, fbytes, hipMemcpyHostToDevice) != hipSuccess) return 1;
    float* d_c = upload(coords, (size_t)B * 2 * hw);
    float* d_o = nullptr;
    float* d_s = nullptr;
    if (!d_c || hipMalloc(&d_o, (size_t)B * 196 * hw * 4) != hipSuccess ||
        hipMalloc(&d_s, 196 * hw * 4) != hipSuccess)
        return 1;
    slk_droid::CorrEngine corr;
    corr.init(h, w, d_f, dtype == SLK_F16 ? SLK_F16 : SLK_F32, ii, jj, B);
    const int half = B / 2;
    corr.batch_build_and_sample_correlation(half, 0, d_c, d_o);
    corr.batch_build_and_sample_correlation(B - half, half, d_c + (size_t)half * 2 * hw,
                                            d_o + (size_t)half * 196 * hw);
    corr.build_correlation(ii[0], jj[0]);
    corr.sample_correlation(d_c, d_s);
    int bad = download(out_batch, d_o, (size_t)B * 196 * hw);
    bad |= download(out_single, d_s, 196 * hw);
    corr.destroy();
    (void)hipFree(d_f);
    (void)hipFree(d_c);
    (void)hipFree(d_o);
    (void)hipFree(d_s);
    return bad;
}

// CorrBlock (corr.cuh:61-263) as a host would drive it: init with (absent)
// library handles, build(fmap1, fmap2, bn, c, h, w) of bn pairs, then
// sample_single(coords, output, scratch), which reads pair 0. A second build
// at another size rebuilds the context. fmap1/fmap2 [bn][c][h][w] fp32,
// coords [2][h*w], out [196][h*w]; out2 receives the lookup of a second build
// with (h2, w2) maps fmap1b/fmap2b [c][h2][w2] and coords2 [2][h2*w2].
extern "C" int adapter_corrblock(const float* fmap1, const float* fmap2, int bn, int c, int h,
                                 int w, const float* coords, float* out, const float* fmap1b,
                                 const float* fmap2b, int h2, int w2, const float* coords2,
                                 float* out2) {
    const size_t hw = (size_t)h * w, hw2 = (size_t)h2 * w2;
    float* d_a = upload(fmap1, (size_t)bn * c * hw);
    float* d_b = upload(fmap2, (size_t)bn * c * hw);
    float* d_c = upload(coords, 2 * hw);
    float* d_a2 = upload(fmap1b, (size_t)c * hw2);
    float* d_b2 = upload(fmap2b, (size_t)c * hw2);
    float* d_c2 = upload(coords2, 2 * hw2);
    float *d_o = nullptr, *d_o2 = nullptr, *d_s = nullptr;
    if (!d_a || !d_b || !d_c || !d_a2 || !d_b2 || !d_c2 ||
        hipMalloc(&d_o, 196 * hw * 4) != hipSuccess ||
        hipMalloc(&d_o2, 196 * hw2 * 4) != hipSuccess ||
        hipMalloc(&d_s, 2 * hw * 4) != hipSuccess)
        return 1;
    slk_droid::CorrBlock cb;
    cb.init(nullptr, nullptr, 4, 3);
    cb.build(d_a, d_b, bn, c, h, w);
    cb.sample_single(d_c, d_o, d_s);
    cb.build(d_a2, d_b2, 1, c, h2, w2);
    cb.sample_single(d_c2, d_o2, d_s);
    int bad = download(out, d_o, 196 * hw);
    bad |= download(out2, d_o2, 196 * hw2);
    cb.destroy();
    for (void* p : {(void*)d_a, (void*)d_b, (void*)d_c, (void*)d_a2, (void*)d_b2, (void*)d_c2,
                    (void*)d_o, (void*)d_o2, (void*)d_s})
        (void)hipFree(p);
    return bad;
}

// `iters` BundleAdjustment::iterate calls followed by clamp_disps(0.001), as
// run_update_pass does (main.cu:2371-2397), or with one_call != 0 the same
// loop as one iterate_n call. poses [N][7] and disps [N][h*w] are updated in
// place. With launches != NULL the iterates run profiled and launches[0..1]
// receive the total launch counts of the linearization and solve kernels.
extern "C" int adapter_ba(int N, int h, int w, float* poses, float* disps, const float* intr,
                          const float* target, const float* weight, const float* eta,
                          const int* ii, const int* jj, int M, int t0, int t1, float lm,
                          float ep, int motion_only, int iters, int one_call, int* launches) {
    const size_t hw = (size_t)h * w;
    float* d_p = upload(poses, (size_t)N * 7);
    float* d_d = upload(disps, (size_t)N * hw);
    float* d_i = upload(intr, 4);
    float* d_t = upload(target, (size_t)M * 2 * hw);
    float* d_w = upload(weight, (size_t)M * 2 * hw);
    float* d_e = upload(eta, (size_t)N * hw);
    int* d_ii = upload(ii, M);
    int* d_jj = upload(jj, M);
    if (!d_p || !d_d || !d_i || !d_t || !d_w || !d_e || !d_ii || !d_jj) return 1;
    std::vector<int> ii_h(ii, ii + M), jj_h(jj, jj + M);
    slk_droid::BundleAdjustment ba;
    ba.init(h, w);
    if (launches) ba.enable_profile(true);
    if (one_call)
        ba.iterate_n(d_p, d_d, d_i, d_t, d_w, d_e, d_ii, d_jj, ii_h.data(), jj_h.data(), M, t0,
                     t1, lm, ep, motion_only != 0, iters);
    else
        for (int k = 0; k < iters; k++)
            ba.iterate(d_p, d_d, d_i, d_t, d_w, d_e, d_ii, d_jj, ii_h.data(), jj_h.data(), M,
                       t0, t1, lm, ep, motion_only != 0);
    if (launches) {
        // launches of the linearization (five-kernel iteration: one wave per
        // edge or edge by edge; fused iteration) and of the solve over all
        // iterates; an overlapped fused step launch holds a solve and the
        // next linearization, the last one a solve
        const int steps = ba.profiled_launches("ba_fz_step");
        launches[0] = ba.profiled_launches("ba_lin_wv") + ba.profiled_launches("ba_lin_kf") +
                      ba.profiled_launches("ba_fz_lin") + steps;
        launches[1] = ba.profiled_launches("ba_solve") + steps + ba.profiled_launches("ba_fz_last");
        ba.print_profile();
    }
    slk_droid::clamp_disps(d_d, (int)(N * hw), 0.001f);
    int bad = download(poses, d_p, (size_t)N * 7);
    bad |= download(disps, d_d, (size_t)N * hw);
    ba.destroy();
    for (void* p : {(void*)d_p, (void*)d_d, (void*)d_i, (void*)d_t, (void*)d_w, (void*)d_e,
                    (void*)d_ii, (void*)d_jj})
        (void)hipFree(p);
    return bad;
}

// One batch of run_update_pass's glue through UpdateGlue, in the reference's
// order: motion (identity coords0), hidden-state loads, target/weight, saves,
// GraphAgg scatter-mean over all edges, eta write-back, BA edge set. Inputs
// and outputs are host arrays; rows are 128*h*w floats. Sizes: coords1,
// target_prev [B][2][hw]; edge_nets, all_agg1 [E][row] (updated in place);
// inps [nkf][row]; batch_agg1 [B][row]; delta, wt [B][3][hw]; kf_eta
// [nkf][hw]; damping [nkf][hw] (updated); inactive: [n_inac] edges with rows
// [n_inac][2][hw]. Outputs: motion [B][4][hw], batch_nets, batch_inps
// [B][row], target/weight of the batch [B][2][hw] (written at bs), kf_agg
// [na][row], active [na], ba_ii/ba_jj [cap], ba_target/ba_weight [cap][2][hw].
extern "C" int adapter_glue(int h, int w, int E, int bs, int B, int nkf, const int* ii,
                            const int* jj, const float* coords1, const float* target_prev,
                            float* edge_nets, const float* inps, const float* batch_agg1,
                            float* all_agg1, const float* delta, const float* wt,
                            const float* kf_eta, float* damping, int n_inac, const int* ii_inac,
                            const int* jj_inac, const float* target_inac,
                            const float* weight_inac, float* motion, float* batch_nets,
                            float* batch_inps, float* target_all, float* weight_all,
                            float* kf_agg, int* active, int* num_active, int* ba_ii,
                            int* ba_jj, float* ba_target, float* ba_weight, int* count,
                            int* t0) {
    const size_t hw = (size_t)h * w, row = 128 * hw;
    float* d_c1 = upload(coords1, B * 2 * hw);
    float* d_tp = upload(target_prev, B * 2 * hw);
    float* d_nets = upload(edge_nets, E * row);
    float* d_inps = upload(inps, nkf * row);
    float* d_bagg = upload(batch_agg1, B * row);
    float* d_agg = upload(all_agg1, E * row);
    float* d_delta = upload(delta, B * 3 * hw);
    float* d_wt = upload(wt, B * 3 * hw);
    float* d_eta = upload(kf_eta, nkf * hw);
    float* d_damp = upload(damping, nkf * hw);
    int* d_ii = upload(ii, E);
    float* d_ti = upload(target_inac, (size_t)(n_inac > 0 ? n_inac : 1) * 2 * hw);
    float* d_wi = upload(weight_inac, (size_t)(n_inac > 0 ? n_inac : 1) * 2 * hw);
    std::vector<float> zeros_t((size_t)E * 2 * hw, 0.0f);
    float* d_tall = upload(zeros_t.data(), E * 2 * hw);
    float* d_wall = upload(zeros_t.data(), E * 2 * hw);
    const size_t cap = (size_t)E + n_inac;
    std::vector<float> zcap(cap * 2 * hw, 0.0f);
    float* d_bt = upload(zcap.data(), cap * 2 * hw);
    float* d_bw = upload(zcap.data(), cap * 2 * hw);
    std::vector<int> zi(cap > 0 ? cap : 1, 0);
    int* d_bi = upload(zi.data(), zi.size());
    int* d_bj = upload(zi.data(), zi.size());
    int* d_act = upload(zi.data(), zi.size());
    float *d_mot = nullptr, *d_bn = nullptr, *d_bi2 = nullptr, *d_kf = nullptr;
    if (hipMalloc(&d_mot, B * 4 * hw * sizeof(float)) != hipSuccess ||
        hipMalloc(&d_bn, B * row * sizeof(float)) != hipSuccess ||
        hipMalloc(&d_bi2, B * row * sizeof(float)) != hipSuccess ||
        hipMalloc(&d_kf, (size_t)nkf * row * sizeof(float)) != hipSuccess)
        return 1;
    if (!d_c1 || !d_tp || !d_nets || !d_inps || !d_bagg || !d_agg || !d_delta || !d_wt ||
        !d_eta || !d_damp || !d_ii || !d_ti || !d_wi || !d_tall || !d_wall || !d_bt || !d_bw ||
        !d_bi || !d_bj || !d_act)
        return 1;

    slk_droid::UpdateGlue glue;
    glue.init(h, w);
    glue.compute_motion(d_mot, d_c1, nullptr, d_tp, B);
    glue.load_hidden(d_bn, d_bi2, d_nets, d_inps, d_ii, bs, B);
    int bad = download(batch_nets, d_bn, B * row);
    bad |= download(batch_inps, d_bi2, B * row);
    // the GRU updates batch_nets in place; here it adds 1 (host side)
    std::vector<float> upd(B * row);
    for (size_t k = 0; k < upd.size(); k++) upd[k] = batch_nets[k] + 1.0f;
    bad |= hipMemcpy(d_bn, upd.data(), upd.size() * sizeof(float), hipMemcpyHostToDevice) !=
           hipSuccess;
    glue.compute_target(d_tall + bs * 2 * hw, d_wall + bs * 2 * hw, d_c1, d_delta, d_wt, B);
    glue.save_hidden(d_nets, d_agg, d_bn, d_bagg, bs, B);
    std::vector<int> ii_h(ii, ii + E), jj_h(jj, jj + E);
    std::vector<int> act = glue.scatter_mean(d_kf, d_agg, ii_h.data(), E, d_act);
    glue.write_eta(d_damp, d_eta, d_act, (int)act.size());
    std::vector<int> bi_h(cap > 0 ? cap : 1), bj_h(cap > 0 ? cap : 1);
    *count = glue.ba_edge_set(ii_h.data(), jj_h.data(), E, ii_inac, jj_inac, n_inac, d_tall,
                              d_wall, d_ti, d_wi, nkf, -1, true, bi_h.data(), bj_h.data(),
                              d_bi, d_bj, d_bt, d_bw, t0);
    *num_active = (int)act.size();
    std::copy(act.begin(), act.end(), active);
    bad |= download(motion, d_mot, B * 4 * hw);
    bad |= download(edge_nets, d_nets, E * row);
    bad |= download(all_agg1, d_agg, E * row);
    bad |= download(target_all, d_tall, E * 2 * hw);
    bad |= download(weight_all, d_wall, E * 2 * hw);
    bad |= download(kf_agg, d_kf, act.size() * row);
    bad |= download(damping, d_damp, nkf * hw);
    bad |= download(ba_ii, d_bi, *count);
    bad |= download(ba_jj, d_bj, *count);
    bad |= download(ba_target, d_bt, (size_t)*count * 2 * hw);
    bad |= download(ba_weight, d_bw, (size_t)*count * 2 * hw);
    for (int k = 0; k < *count; k++) bad |= (bi_h[k] != ba_ii[k] || bj_h[k] != ba_jj[k]);
    glue.destroy();
    for (void* p : {(void*)d_c1, (void*)d_tp, (void*)d_nets, (void*)d_inps, (void*)d_bagg,
                    (void*)d_agg, (void*)d_delta, (void*)d_wt, (void*)d_eta, (void*)d_damp,
                    (void*)d_ii, (void*)d_ti, (void*)d_wi, (void*)d_tall, (void*)d_wall,
                    (void*)d_bt, (void*)d_bw, (void*)d_bi, (void*)d_bj, (void*)d_act,
                    (void*)d_mot, (void*)d_bn, (void*)d_bi2, (void*)d_kf})
        (void)hipFree(p);
    return bad;
}

// UpdateModule (main.cu:535-667) through the adapter: weights from the
// reference's tensor files in `dir`, forward on host inputs corr
// [B][196][hw], motion [B][4][hw], net [B][128][hw] (updated), inp, then
// compute_eta on agg_kf [K][128][hw]; and the motion filter between frames 0
// and 1 of fmaps [2][128][hw] fp32 from state 0 of net/inp (before the
// update), written to *mean_flow.
extern "C" int adapter_update(const char* dir, int B, int K, int h, int w, const float* corr,
                              const float* motion, float* net, const float* inp, float* delta,
                              float* weight, float* agg, const float* agg_kf, float* eta,
                              const float* fmaps, float* mean_flow) {
    const size_t hw = (size_t)h * w;
    float* d_c = upload(corr, B * 196 * hw);
    float* d_m = upload(motion, B * 4 * hw);
    float* d_n = upload(net, B * 128 * hw);
    float* d_i = upload(inp, B * 128 * hw);
    float* d_k = upload(agg_kf, K * 128 * hw);
    float* d_f = upload(fmaps, 2 * 128 * hw);
    float *d_d = nullptr, *d_w = nullptr, *d_a = nullptr, *d_e = nullptr;
    if (!d_c || !d_m || !d_n || !d_i || !d_k || !d_f ||
        hipMalloc(&d_d, B * 3 * hw * 4) != hipSuccess ||
        hipMalloc(&d_w, B * 3 * hw * 4) != hipSuccess ||
        hipMalloc(&d_a, B * 128 * hw * 4) != hipSuccess ||
        hipMalloc(&d_e, K * hw * 4) != hipSuccess)
        return 1;
    slk_droid::UpdateModule update;
    update.init(nullptr, dir, B, h, w);
    slk_droid::CorrEngine corr_engine;
    const int ii[1] = {0}, jj[1] = {1};
    corr_engine.init(h, w, d_f, SLK_F32, ii, jj, 1);
    *mean_flow = corr_engine.compute_motion_gru(update.module(), 0, 1, d_n, d_i);
    update.forward(nullptr, d_c, d_m, d_n, d_i, d_d, d_w, d_a, nullptr, nullptr, nullptr, B, h, w);
    update.compute_eta(nullptr, d_k, d_e, nullptr, nullptr, nullptr, K, h, w);
    int bad = download(net, d_n, B * 128 * hw);
    bad |= download(delta, d_d, B * 3 * hw);
    bad |= download(weight, d_w, B * 3 * hw);
    bad |= download(agg, d_a, B * 128 * hw);
    bad |= download(eta, d_e, K * hw);
    corr_engine.destroy();
    update.destroy();
    for (void* p : {(void*)d_c, (void*)d_m, (void*)d_n, (void*)d_i, (void*)d_k, (void*)d_f,
                    (void*)d_d, (void*)d_w, (void*)d_a, (void*)d_e})
        (void)hipFree(p);
    return bad;
}

// The front of the pipe through the adapters, in the reference's order
// (main.cu:2729-2753, 1465-1497, 2924-2937): an 8-bit BGR frame resized to
// H x W, fnet/cnet HalfBasicEncoders from <dir>, encode_frame, and the pose
// file. fmap [128][H/8][W/8] (fp16 bits), net / inp [128][H/8][W/8].
extern "C" int adapter_frontend(const char* dir, const unsigned char* bgr8, int src_w, int src_h,
                                int H, int W, unsigned short* fmap, float* net, float* inp,
                                const char* pose_path, int nk, const int* ts, const float* poses) {
    const size_t hw = (size_t)(H / 8) * (W / 8);
    unsigned char* d_src = upload(bgr8, (size_t)src_w * src_h * 3);
    float *d_bgr = nullptr, *d_n = nullptr, *d_i = nullptr;
    unsigned short* d_f = nullptr;
    if (!d_src || hipMalloc(&d_bgr, (size_t)H * W * 3 * 4) != hipSuccess ||
        hipMalloc(&d_f, 128 * hw * 2) != hipSuccess || hipMalloc(&d_n, 128 * hw * 4) != hipSuccess ||
        hipMalloc(&d_i, 128 * hw * 4) != hipSuccess)
        return 1;
    slk_droid::bgr8_to_bgrf_resize(d_src, d_bgr, src_w, src_h, src_w * 3, W, H);
    slk_droid::HalfBasicEncoder fnet, cnet;
    fnet.init(nullptr, dir, "fnet", 1, H, W, 128, true);
    cnet.init(nullptr, dir, "cnet", 1, H, W, 256, false);
    slk_droid::encode_frame(fnet, cnet, d_bgr, d_f, d_n, d_i);
    int bad = download(fmap, d_f, 128 * hw);
    bad |= download(net, d_n, 128 * hw);
    bad |= download(inp, d_i, 128 * hw);
    slk_droid::save_poses(pose_path, nk, ts, poses, true);
    fnet.destroy();
    cnet.destroy();
    for (void* p : {(void*)d_src, (void*)d_bgr, (void*)d_f, (void*)d_n, (void*)d_i}) (void)hipFree(p);
    return bad;
}
