// Context lifetime, error reporting and buffer helpers of libslk.
#include <cstdio>

#include "slk_internal.hpp"

namespace slk {

static thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

int DevBuf::ensure(size_t n) {
    if (n <= bytes && ptr) return SLK_OK;
    release();
    if (n == 0) return SLK_OK;
    SLK_HIP(hipMalloc(&ptr, n));
    bytes = n;
    return SLK_OK;
}

void DevBuf::release() {
    if (ptr) (void)hipFree(ptr);
    ptr = nullptr;
    bytes = 0;
}

int HostStage::ensure(size_t n) {
    SLK_TRY(wait());
    if (!done) SLK_HIP(hipEventCreateWithFlags(&done, hipEventDisableTiming));
    if (n <= bytes && ptr) return SLK_OK;
    if (ptr) (void)hipHostFree(ptr);
    ptr = nullptr;
    bytes = 0;
    SLK_HIP(hipHostMalloc(&ptr, n, hipHostMallocDefault));
    bytes = n;
    return SLK_OK;
}

int HostStage::wait() {
    if (pending) {
        pending = false;
        SLK_HIP(hipEventSynchronize(done));
    }
    return SLK_OK;
}

void HostStage::release() {
    if (pending) (void)hipEventSynchronize(done);
    pending = false;
    if (ptr) (void)hipHostFree(ptr);
    if (done) (void)hipEventDestroy(done);
    ptr = nullptr;
    done = nullptr;
    bytes = 0;
}

}  // namespace slk

extern "C" const char* slk_last_error(void) { return slk::g_last_error.c_str(); }

extern "C" int slk_create(slk_ctx** out, int h, int w, int C, int max_batch, int levels,
                          int radius, float corr_scale) {
    using namespace slk;
    if (!out) return fail(SLK_E_ARG, "slk_create: null output pointer");
    *out = nullptr;
    if (h < 1 || w < 1 || C < 2 || (C & 1) || max_batch < 1)
        return fail(SLK_E_ARG, "slk_create: need h,w >= 1, even C >= 2, max_batch >= 1");
    if (levels < 1 || levels > kMaxLevels)
        return fail(SLK_E_ARG, "slk_create: levels must be in [1, 4]");
    if (radius != 3) return fail(SLK_E_ARG, "slk_create: only radius 3 is implemented");
    if ((h >> (levels - 1)) < 1 || (w >> (levels - 1)) < 1)
        return fail(SLK_E_ARG, "slk_create: feature map too small for the pyramid depth");
    // The batched path addresses a slot of lookup windows (1 KB per source
    // pixel) with 32-bit byte offsets and a buffer-resource range of
    // 1024*h*w bytes, so h*w stays below 2^21 (the single-edge volume,
    // (h*w)^2 floats, is far beyond memory long before that).
    if ((long)h * w >= (1L << 21) || h > 65536 || w > 65536)
        return fail(SLK_E_ARG, "slk_create: h*w must be below 2^21 and each side at most 2^16");
    slk_ctx* ctx = new slk_ctx();
    ctx->h = h;
    ctx->w = w;
    ctx->HW = h * w;
    ctx->C = C;
    ctx->levels = levels;
    ctx->radius = radius;
    ctx->max_batch = max_batch;
    ctx->alpha = corr_scale;
    for (int l = 0; l < levels; l++) {
        ctx->lh[l] = h >> l;
        ctx->lw[l] = w >> l;
    }
    int st = hipGetDevice(&ctx->device) == hipSuccess ? SLK_OK
                                                       : fail(SLK_E_HIP, "hipGetDevice failed");
    if (st == SLK_OK) st = corr_alloc(ctx);
    if (st == SLK_OK) st = ba_create(ctx);
    if (st != SLK_OK) {
        slk_destroy(ctx);
        return st;
    }
    *out = ctx;
    return SLK_OK;
}

namespace {
// Unfolded records' events go back to the pool once they have completed.
void prof_clear(slk_ctx* ctx) {
    for (auto& r : ctx->prof_recs) {
        (void)hipEventSynchronize(r.b);
        ctx->prof_pool.push_back(r.a);
        ctx->prof_pool.push_back(r.b);
    }
    ctx->prof_recs.clear();
    ctx->prof_names.clear();
    ctx->prof_ms.clear();
    ctx->prof_count.clear();
    ctx->prof_dirty = false;
}

// Folds finished launch records into per-name totals (synchronises on them).
int prof_fold(slk_ctx* ctx) {
    using namespace slk;
    for (auto& r : ctx->prof_recs) {
        SLK_HIP(hipEventSynchronize(r.b));
        float ms = 0.0f;
        SLK_HIP(hipEventElapsedTime(&ms, r.a, r.b));
        size_t k = 0;
        while (k < ctx->prof_names.size() && ctx->prof_names[k] != r.name) k++;
        if (k == ctx->prof_names.size()) {
            ctx->prof_names.emplace_back(r.name);
            ctx->prof_ms.push_back(0.0);
            ctx->prof_count.push_back(0);
        }
        ctx->prof_ms[k] += ms;
        ctx->prof_count[k] += 1;
        ctx->prof_pool.push_back(r.a);
        ctx->prof_pool.push_back(r.b);
    }
    ctx->prof_recs.clear();
    ctx->prof_dirty = false;
    return SLK_OK;
}
}  // namespace

extern "C" int slk_profile_enable(slk_ctx* ctx, int on) {
    if (!ctx) return slk::fail(SLK_E_ARG, "profile_enable: null context");
    prof_clear(ctx);
    ctx->prof = on != 0;
    return SLK_OK;
}

extern "C" int slk_profile_kernel(slk_ctx* ctx, int idx, const char** name, double* total_ms,
                                  int* launches) {
    if (!ctx) return slk::fail(SLK_E_ARG, "profile_kernel: null context");
    if (ctx->prof_dirty) SLK_TRY(prof_fold(ctx));
    if (idx < 0 || idx >= (int)ctx->prof_names.size())
        return slk::fail(SLK_E_ARG, "profile_kernel: index out of range");
    if (name) *name = ctx->prof_names[idx].c_str();
    if (total_ms) *total_ms = ctx->prof_ms[idx];
    if (launches) *launches = ctx->prof_count[idx];
    return SLK_OK;
}

extern "C" int slk_destroy(slk_ctx* ctx) {
    if (!ctx) return SLK_OK;
    prof_clear(ctx);
    for (hipEvent_t e : ctx->prof_pool) (void)hipEventDestroy(e);
    ctx->prof_pool.clear();
    slk::ba_destroy(ctx);
    ctx->batch_win.release();
    ctx->split_feat.release();
    ctx->prep_feat.release();
    ctx->tile_ctr.release();
    ctx->tile_list.release();
    ctx->src_order.release();
    for (int l = 0; l < slk::kMaxLevels; l++) ctx->single_lvl[l].release();
    ctx->zero_idx.release();
    ctx->glue_stage.release();
    ctx->glue_idx.release();
    ctx->edge_stage.release();
    ctx->graph_pairs.release();
    ctx->graph_dist.release();
    delete ctx;
    return SLK_OK;
}
