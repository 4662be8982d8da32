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

// `iters` BundleAdjustment::iterate calls followed by clamp_disps(0.001), as
// run_update_pass does (main.cu:2371-2397). poses [N][7] and disps [N][h*w]
// are updated in place.
extern "C" int adapter_ba(int N, int h, int w, float* poses, float* disps, const float* intr,
                          const float* target, const float* weight, const float* eta,
                          const int* ii, const int* jj, int M, int t0, int t1, float lm,
                          float ep, int motion_only, int iters) {
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
    for (int k = 0; k < iters; k++)
        ba.iterate(d_p, d_d, d_i, d_t, d_w, d_e, d_ii, d_jj, ii_h.data(), jj_h.data(), M, t0,
                   t1, lm, ep, motion_only != 0);
    slk_droid::clamp_disps(d_d, (int)(N * hw), 0.001f);
    int bad = download(poses, d_p, (size_t)N * 7);
    bad |= download(disps, d_d, (size_t)N * hw);
    ba.destroy();
    for (void* p : {(void*)d_p, (void*)d_d, (void*)d_i, (void*)d_t, (void*)d_w, (void*)d_e,
                    (void*)d_ii, (void*)d_jj})
        (void)hipFree(p);
    return bad;
}
