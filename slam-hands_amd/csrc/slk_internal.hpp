// Internal declarations of libslk (MI355X / gfx950 DROID-SLAM per-edge path).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

#include "slk.h"

namespace slk {

// Records a failure message for slk_last_error() and returns `code`.
int fail(int code, const std::string& msg);

#define SLK_HIP(expr)                                                              \
    do {                                                                           \
        hipError_t _e = (expr);                                                    \
        if (_e != hipSuccess)                                                      \
            return ::slk::fail(SLK_E_HIP, std::string(#expr " -> ") +             \
                                              hipGetErrorString(_e));             \
    } while (0)

#define SLK_TRY(expr)                      \
    do {                                   \
        int _s = (expr);                   \
        if (_s != SLK_OK) return _s;       \
    } while (0)

// Grow-only device buffer owned by a context (no allocation in steady state).
struct DevBuf {
    void* ptr = nullptr;
    size_t bytes = 0;
    int ensure(size_t n);
    void release();
    template <typename T>
    T* as() const { return static_cast<T*>(ptr); }
};

// Pinned host staging buffer, guarded by an event so a new upload never
// overwrites bytes an earlier asynchronous copy may still be reading.
struct HostStage {
    void* ptr = nullptr;
    size_t bytes = 0;
    hipEvent_t done = nullptr;
    bool pending = false;
    int ensure(size_t n);
    int wait();
    void release();
};

struct BaState;  // ba.hip

constexpr int kMaxLevels = 4;

// Per-kernel timing on the launch stream (hipEvents around each launch),
// enabled by slk_profile_enable; the reference's counterparts are CudaTimer
// (cuda_slam/main.cu:41-59) and BundleAdjustment::print_profile (ba.cuh:805).
struct ProfRec {
    const char* name;
    hipEvent_t a, b;
};

}  // namespace slk

struct slk_ctx {
    int device = 0;
    int h = 0, w = 0, HW = 0, C = 0, levels = 4, radius = 3, max_batch = 48;
    float alpha = 1.0f / 16.0f;
    int corr_prec = SLK_PREC_F16X3;  // contraction of fp32 features
    int lh[slk::kMaxLevels] = {0}, lw[slk::kMaxLevels] = {0};
    // batched-path scratch: 8x8 lookup windows [max_batch][4 levels][8 rows][HW][8]
    slk::DevBuf batch_win;
    // batched-path operands: hi/lo split of every level's features per
    // frame slot, with the frame's inverse split scale
    slk::DevBuf split_feat;
    // frames split once by slk_corr_prepare_frames (slot = frame index)
    slk::DevBuf prep_feat;
    int prep_nframes = 0;
    int prep_mode = 0;      // their split (fp16 scaled or bf16)
    bool prep_alo = true;   // whether their level-0 lo planes can be nonzero
    slk::DevBuf tile_list;  // the (edge, source tile, target tile) ids holding a window cell
    slk::DevBuf tile_ctr;   // listed-tile count and the correlation kernel's tile counters
    slk::DevBuf src_order;  // per edge: sources sorted by window position (pixel, x, y), boxes
    int ws_grid = 0;        // workgroups of the batched correlation kernel
    // single-edge persistent volume + pyramid (build_correlation/sample_correlation)
    slk::DevBuf single_lvl[slk::kMaxLevels];
    bool single_built = false;
    slk::DevBuf zero_idx;  // device int {0}
    // update-pass glue: index lists uploaded through a pinned stage
    slk::HostStage glue_stage;
    slk::DevBuf glue_idx;
    slk::DevBuf edge_stage;  // rows in transit of slk_store_and_remove_edges
    // proximity factors: the pair lists and their frame distances
    slk::DevBuf graph_pairs, graph_dist;
    slk::BaState* ba = nullptr;
    bool prof = false;
    std::vector<slk::ProfRec> prof_recs;
    std::vector<std::string> prof_names;
    std::vector<double> prof_ms;
    std::vector<int> prof_count;
    bool prof_dirty = false;
    // events of folded records, reused so that a profiled launch sequence
    // creates no events once the pool holds enough of them
    std::vector<hipEvent_t> prof_pool;
};

namespace slk {
// RAII bracket of one kernel launch for the profiler (no-op when disabled).
struct ProfScope {
    slk_ctx* ctx;
    const char* name;
    hipStream_t stream;
    hipEvent_t a = nullptr;
    static hipEvent_t take(slk_ctx* c) {
        if (!c->prof_pool.empty()) {
            hipEvent_t e = c->prof_pool.back();
            c->prof_pool.pop_back();
            return e;
        }
        hipEvent_t e = nullptr;
        return hipEventCreate(&e) == hipSuccess ? e : nullptr;
    }
    ProfScope(slk_ctx* c, const char* n, hipStream_t s) : ctx(c), name(n), stream(s) {
        if (ctx && ctx->prof && (a = take(ctx)) != nullptr) (void)hipEventRecord(a, stream);
    }
    ~ProfScope() {
        if (!a) return;
        hipEvent_t b = take(ctx);
        if (b && hipEventRecord(b, stream) == hipSuccess) {
            ctx->prof_recs.push_back({name, a, b});
            ctx->prof_dirty = true;
        } else {
            ctx->prof_pool.push_back(a);
            if (b) ctx->prof_pool.push_back(b);
        }
    }
};
}  // namespace slk

namespace slk {
// corr.hip
int corr_alloc(slk_ctx* ctx);
// corr_split.hip
bool corr_split_supported(const slk_ctx* ctx);
int corr_split_alloc(slk_ctx* ctx);
// bytes of one feature slot (two per edge of a launch), of one edge's tile
// list and source order, and of the launch's tile counters
void corr_split_footprint(const slk_ctx* ctx, size_t* slot_bytes, size_t* tiles_per_edge,
                          size_t* order_per_edge, size_t* ctr_bytes);
// workgroups of the batched correlation kernel on a part with `cus` CUs
int corr_split_grid(int cus);
int corr_split_windows(slk_ctx* ctx, const void* fmaps, int dtype, long fstride,
                       const int* ii_host, const int* jj_host, const int* ii_dev,
                       const int* jj_dev, int n, const float* coords, float* win, int slot0,
                       hipStream_t stream);
int corr_split_prepare(slk_ctx* ctx, const void* fmaps, int dtype, long fstride, int nframes,
                       hipStream_t stream);
int corr_split_windows_prepared(slk_ctx* ctx, const int* ii_host, const int* jj_host, int n,
                                const float* coords, float* win, int slot0, hipStream_t stream);
// ba.hip
int ba_create(slk_ctx* ctx);
void ba_destroy(slk_ctx* ctx);
}  // namespace slk
