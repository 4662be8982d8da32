// Update-pass glue around the correlation and BA entry points: the
// elementwise motion/target kernels of run_update_pass, one-launch row
// gathers and scatters in place of its per-edge cudaMemcpy loops, the
// keyframe scatter-mean of GraphAgg, and the active + inactive BA edge set
// (cuda_slam/main.cu:1246-1301, 2186-2400; cuda_pipeline/slam.cuh:2555-2603).
//
// All of it is HBM-bound copying: every kernel moves each byte once with
// 16-byte loads and stores when the row length and pointers allow it, and
// one launch covers all rows of a call (the reference issues a cudaMemcpy per
// edge and per array, each a separate host round trip).
#include <algorithm>
#include <climits>
#include <cstring>
#include <type_traits>
#include <vector>

#include "slk_internal.hpp"

namespace slk {
namespace {

__device__ __forceinline__ float clamp64(float v) { return fminf(fmaxf(v, -64.0f), 64.0f); }

// motion [B][4][HW] from coords1/target [B][2][HW] (and coords0, or the
// identity grid when c0 is null); one thread per 4 consecutive pixels when
// HW % 4 == 0 (kV = 4), else one per pixel.
template <int kV>
__global__ __launch_bounds__(256) void k_motion(float* __restrict__ motion,
                                                const float* __restrict__ c1,
                                                const float* __restrict__ c0,
                                                const float* __restrict__ tg, int B, int HW,
                                                int w) {
    using V = typename std::conditional<kV == 4, float4, float>::type;
    const long nv = (long)B * HW / kV;
    for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < nv;
         i += (long)gridDim.x * blockDim.x) {
        const long e = i * kV / HW;
        const int k = (int)(i * kV - e * HW);
        const long o2 = e * 2 * HW + k;
        float x1[kV], y1[kV], x0[kV], y0[kV], xt[kV], yt[kV];
        *reinterpret_cast<V*>(x1) = *reinterpret_cast<const V*>(c1 + o2);
        *reinterpret_cast<V*>(y1) = *reinterpret_cast<const V*>(c1 + o2 + HW);
        *reinterpret_cast<V*>(xt) = *reinterpret_cast<const V*>(tg + o2);
        *reinterpret_cast<V*>(yt) = *reinterpret_cast<const V*>(tg + o2 + HW);
        if (c0) {
            *reinterpret_cast<V*>(x0) = *reinterpret_cast<const V*>(c0 + o2);
            *reinterpret_cast<V*>(y0) = *reinterpret_cast<const V*>(c0 + o2 + HW);
        } else {
#pragma unroll
            for (int j = 0; j < kV; j++) {
                const int y = (k + j) / w;
                x0[j] = (float)(k + j - y * w);
                y0[j] = (float)y;
            }
        }
        float m0[kV], m1[kV], m2[kV], m3[kV];
#pragma unroll
        for (int j = 0; j < kV; j++) {
            m0[j] = clamp64(x1[j] - x0[j]);
            m1[j] = clamp64(y1[j] - y0[j]);
            m2[j] = clamp64(xt[j] - x1[j]);
            m3[j] = clamp64(yt[j] - y1[j]);
        }
        float* m = motion + e * 4 * HW + k;
        *reinterpret_cast<V*>(m) = *reinterpret_cast<V*>(m0);
        *reinterpret_cast<V*>(m + HW) = *reinterpret_cast<V*>(m1);
        *reinterpret_cast<V*>(m + 2 * HW) = *reinterpret_cast<V*>(m2);
        *reinterpret_cast<V*>(m + 3 * HW) = *reinterpret_cast<V*>(m3);
    }
}

template <int kV>
__global__ __launch_bounds__(256) void k_coords0(float* __restrict__ c0, int B, int HW, int w) {
    using V = typename std::conditional<kV == 4, float4, float>::type;
    const long nv = (long)B * HW / kV;
    for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < nv;
         i += (long)gridDim.x * blockDim.x) {
        const long e = i * kV / HW;
        const int k = (int)(i * kV - e * HW);
        float x[kV], y[kV];
#pragma unroll
        for (int j = 0; j < kV; j++) {
            const int r = (k + j) / w;
            x[j] = (float)(k + j - r * w);
            y[j] = (float)r;
        }
        *reinterpret_cast<V*>(c0 + e * 2 * HW + k) = *reinterpret_cast<V*>(x);
        *reinterpret_cast<V*>(c0 + e * 2 * HW + HW + k) = *reinterpret_cast<V*>(y);
    }
}

// target/weight [n][2][HW] from coords [n][2][HW] and delta/wt [n][3][HW]
template <int kV>
__global__ __launch_bounds__(256) void k_target(float* __restrict__ target,
                                                float* __restrict__ weight,
                                                const float* __restrict__ coords,
                                                const float* __restrict__ delta,
                                                const float* __restrict__ wt, int n, int HW) {
    using V = typename std::conditional<kV == 4, float4, float>::type;
    const long nv = (long)n * 2 * HW / kV;
    for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < nv;
         i += (long)gridDim.x * blockDim.x) {
        const long o2 = i * kV;               // offset in [n][2][HW]
        const long ec = o2 / HW;              // e * 2 + c
        const long o3 = (ec / 2) * 3 * HW + (ec & 1) * HW + (o2 - ec * HW);
        float a[kV], d[kV], t[kV];
        *reinterpret_cast<V*>(a) = *reinterpret_cast<const V*>(coords + o2);
        *reinterpret_cast<V*>(d) = *reinterpret_cast<const V*>(delta + o3);
#pragma unroll
        for (int j = 0; j < kV; j++) t[j] = a[j] + d[j];
        *reinterpret_cast<V*>(target + o2) = *reinterpret_cast<V*>(t);
        *reinterpret_cast<V*>(weight + o2) = *reinterpret_cast<const V*>(wt + o3);
    }
}

// dst row (scatter ? idx[e] : e) = src row (scatter ? e : idx[e]); idx null is
// the identity. Grid (chunks of a row, rows); kV floats per access.
template <int kV>
__global__ __launch_bounds__(256) void k_rows(float* __restrict__ dst,
                                              const float* __restrict__ src,
                                              const int* __restrict__ idx, long row,
                                              int scatter) {
    using V = typename std::conditional<kV == 4, float4, float>::type;
    const int e = blockIdx.y;
    const long r = idx ? idx[e] : e;
    const float* s = src + (scatter ? (long)e : r) * row;
    float* d = dst + (scatter ? r : (long)e) * row;
    const long nv = row / kV;
    for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < nv;
         i += (long)gridDim.x * blockDim.x)
        reinterpret_cast<V*>(d)[i] = reinterpret_cast<const V*>(s)[i];
}

// Keyframe means: csr = [na + 1 offsets][edge ids grouped by keyframe, edge
// order within a group]; dst row a = sum of its rows from zero, in that
// order, then fma(1/count - 1, S, S) when count > 1.
template <int kV>
__global__ __launch_bounds__(256) void k_scatter_mean(float* __restrict__ dst,
                                                      const float* __restrict__ src,
                                                      const int* __restrict__ csr, int na,
                                                      long row) {
    using V = typename std::conditional<kV == 4, float4, float>::type;
    const int a = blockIdx.y;
    const int b0 = csr[a], b1 = csr[a + 1];
    const int* ed = csr + na + 1;
    const int count = b1 - b0;
    const float inv = 1.0f / (float)count;
    const long nv = row / kV;
    for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < nv;
         i += (long)gridDim.x * blockDim.x) {
        float acc[kV];
#pragma unroll
        for (int j = 0; j < kV; j++) acc[j] = 0.0f;
        for (int b = b0; b < b1; b++) {
            float x[kV];
            *reinterpret_cast<V*>(x) =
                reinterpret_cast<const V*>(src + (long)ed[b] * row)[i];
#pragma unroll
            for (int j = 0; j < kV; j++) acc[j] = acc[j] + x[j];
        }
        if (count > 1) {
#pragma unroll
            for (int j = 0; j < kV; j++) acc[j] = __builtin_fmaf(inv - 1.0f, acc[j], acc[j]);
        }
        reinterpret_cast<V*>(dst + (long)a * row)[i] = *reinterpret_cast<V*>(acc);
    }
}

// BA edge rows: row m < n from target/weight row m, row m >= n from the
// inactive arrays' row sel[m - n]; rows of 2 * hw floats.
template <int kV>
__global__ __launch_bounds__(256) void k_edge_rows(float* __restrict__ bt, float* __restrict__ bw,
                                                   const float* __restrict__ t,
                                                   const float* __restrict__ w,
                                                   const float* __restrict__ ti,
                                                   const float* __restrict__ wi,
                                                   const int* __restrict__ sel, int n, long row) {
    using V = typename std::conditional<kV == 4, float4, float>::type;
    const int m = blockIdx.y;
    const float* st = m < n ? t + (long)m * row : ti + (long)sel[m - n] * row;
    const float* sw = m < n ? w + (long)m * row : wi + (long)sel[m - n] * row;
    const long nv = row / kV;
    for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < nv;
         i += (long)gridDim.x * blockDim.x) {
        reinterpret_cast<V*>(bt + (long)m * row)[i] = reinterpret_cast<const V*>(st)[i];
        reinterpret_cast<V*>(bw + (long)m * row)[i] = reinterpret_cast<const V*>(sw)[i];
    }
}

bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// grid for an elementwise pass over nv vector elements: enough workgroups to
// fill the chip several times over, each thread looping over the rest
dim3 flat_grid(long nv) {
    const long wg = (nv + 255) / 256;
    return dim3((unsigned)std::max(1L, std::min(wg, 256L * 16)));
}

// grid for per-row kernels: chunks of 256 vectors of each row, capped so that
// n rows x chunks stays in the tens of thousands of workgroups
dim3 row_grid(long nv, int rows) {
    long chunks = (nv + 255) / 256;
    chunks = std::max(1L, std::min(chunks, std::max(1L, 65536L / std::max(rows, 1))));
    return dim3((unsigned)chunks, (unsigned)rows);
}

// copies `bytes` of host data into the context's glue upload buffer and
// enqueues the upload on `stream` (the pinned stage is reused only after the
// previous upload has completed)
int upload(slk_ctx* ctx, const void* host, size_t bytes, hipStream_t stream) {
    SLK_TRY(ctx->glue_stage.ensure(bytes));
    if (bytes > ctx->glue_idx.bytes && ctx->glue_idx.ptr)
        SLK_HIP(hipDeviceSynchronize());  // earlier launches may still read the old list
    SLK_TRY(ctx->glue_idx.ensure(std::max(bytes, (size_t)4096)));
    std::memcpy(ctx->glue_stage.ptr, host, bytes);
    SLK_HIP(hipMemcpyAsync(ctx->glue_idx.ptr, ctx->glue_stage.ptr, bytes, hipMemcpyHostToDevice,
                           stream));
    SLK_HIP(hipEventRecord(ctx->glue_stage.done, stream));
    ctx->glue_stage.pending = true;
    return SLK_OK;
}

}  // namespace
}  // namespace slk

using namespace slk;

extern "C" int slk_compute_motion(float* motion, const float* coords1, const float* coords0,
                                  const float* target, int batch, int h, int w,
                                  hipStream_t stream) {
    if (batch <= 0) return SLK_OK;
    if (!motion || !coords1 || !target || h <= 0 || w <= 0)
        return fail(SLK_E_ARG, "compute_motion: null argument or empty grid");
    const int HW = h * w;
    const bool v4 = HW % 4 == 0 && al16(motion) && al16(coords1) && al16(target) &&
                    (!coords0 || al16(coords0));
    if (v4)
        hipLaunchKernelGGL(k_motion<4>, flat_grid((long)batch * HW / 4), dim3(256), 0, stream,
                           motion, coords1, coords0, target, batch, HW, w);
    else
        hipLaunchKernelGGL(k_motion<1>, flat_grid((long)batch * HW), dim3(256), 0, stream,
                           motion, coords1, coords0, target, batch, HW, w);
    SLK_HIP(hipGetLastError());
    return SLK_OK;
}

extern "C" int slk_fill_coords0(float* coords0, int batch, int h, int w, hipStream_t stream) {
    if (batch <= 0) return SLK_OK;
    if (!coords0 || h <= 0 || w <= 0) return fail(SLK_E_ARG, "fill_coords0: bad argument");
    const int HW = h * w;
    if (HW % 4 == 0 && al16(coords0))
        hipLaunchKernelGGL(k_coords0<4>, flat_grid((long)batch * HW / 4), dim3(256), 0, stream,
                           coords0, batch, HW, w);
    else
        hipLaunchKernelGGL(k_coords0<1>, flat_grid((long)batch * HW), dim3(256), 0, stream,
                           coords0, batch, HW, w);
    SLK_HIP(hipGetLastError());
    return SLK_OK;
}

extern "C" int slk_compute_target(float* target, float* weight_out, const float* coords,
                                  const float* delta, const float* wt_raw, int num_edges,
                                  int hw, hipStream_t stream) {
    if (num_edges <= 0) return SLK_OK;
    if (!target || !weight_out || !coords || !delta || !wt_raw || hw <= 0)
        return fail(SLK_E_ARG, "compute_target: null argument or hw <= 0");
    const bool v4 = hw % 4 == 0 && al16(target) && al16(weight_out) && al16(coords) &&
                    al16(delta) && al16(wt_raw);
    const long n2 = (long)num_edges * 2 * hw;
    if (v4)
        hipLaunchKernelGGL(k_target<4>, flat_grid(n2 / 4), dim3(256), 0, stream, target,
                           weight_out, coords, delta, wt_raw, num_edges, hw);
    else
        hipLaunchKernelGGL(k_target<1>, flat_grid(n2), dim3(256), 0, stream, target, weight_out,
                           coords, delta, wt_raw, num_edges, hw);
    SLK_HIP(hipGetLastError());
    return SLK_OK;
}

namespace {
int rows_launch(float* dst, const float* src, const int* idx, int n, long row, int scatter,
                hipStream_t stream, const char* what) {
    if (n <= 0 || row <= 0) return SLK_OK;
    if (!dst || !src) return fail(SLK_E_ARG, std::string(what) + ": null argument");
    if (n > 65535) return fail(SLK_E_ARG, std::string(what) + ": more than 65535 rows");
    if (row % 4 == 0 && al16(dst) && al16(src))
        hipLaunchKernelGGL(k_rows<4>, row_grid(row / 4, n), dim3(256), 0, stream, dst, src, idx,
                           row, scatter);
    else
        hipLaunchKernelGGL(k_rows<1>, row_grid(row, n), dim3(256), 0, stream, dst, src, idx, row,
                           scatter);
    SLK_HIP(hipGetLastError());
    return SLK_OK;
}
}  // namespace

extern "C" int slk_gather_rows(float* dst, const float* src, const int* idx, int n, long row,
                               hipStream_t stream) {
    return rows_launch(dst, src, idx, n, row, 0, stream, "gather_rows");
}

extern "C" int slk_scatter_rows(float* dst, const float* src, const int* idx, int n, long row,
                                hipStream_t stream) {
    return rows_launch(dst, src, idx, n, row, 1, stream, "scatter_rows");
}

extern "C" int slk_scatter_mean(slk_ctx* ctx, float* dst, const float* src, const int* ii_host,
                                int n, long row, int* active_kf, int* active_kf_host,
                                int* num_active_host, hipStream_t stream) {
    if (!ctx || !num_active_host) return fail(SLK_E_ARG, "scatter_mean: null argument");
    *num_active_host = 0;
    if (n <= 0 || row <= 0) return SLK_OK;
    if (!dst || !src || !ii_host) return fail(SLK_E_ARG, "scatter_mean: null argument");
    if (n > 65535) return fail(SLK_E_ARG, "scatter_mean: more than 65535 edges");
    // active keyframes ascending, and the edges of each in edge order
    // (std::set over ii_host and the edge loop, main.cu:2265-2288)
    std::vector<int> act(ii_host, ii_host + n);
    std::sort(act.begin(), act.end());
    act.erase(std::unique(act.begin(), act.end()), act.end());
    if (act.front() < 0) return fail(SLK_E_ARG, "scatter_mean: negative keyframe index");
    const int na = (int)act.size();
    std::vector<int> buf((size_t)na + 1 + n + na);  // offsets, edge ids, active list
    int* off = buf.data();
    int* ed = off + na + 1;
    std::vector<int> slot(n), fill(na, 0);
    for (int e = 0; e < n; e++) {
        slot[e] = (int)(std::lower_bound(act.begin(), act.end(), ii_host[e]) - act.begin());
        fill[slot[e]]++;
    }
    off[0] = 0;
    for (int a = 0; a < na; a++) off[a + 1] = off[a] + fill[a];
    std::fill(fill.begin(), fill.end(), 0);
    for (int e = 0; e < n; e++) ed[off[slot[e]] + fill[slot[e]]++] = e;
    std::copy(act.begin(), act.end(), ed + n);
    SLK_TRY(upload(ctx, buf.data(), buf.size() * sizeof(int), stream));
    const int* csr = ctx->glue_idx.as<int>();
    if (row % 4 == 0 && al16(dst) && al16(src))
        hipLaunchKernelGGL(k_scatter_mean<4>, row_grid(row / 4, na), dim3(256), 0, stream, dst,
                           src, csr, na, row);
    else
        hipLaunchKernelGGL(k_scatter_mean<1>, row_grid(row, na), dim3(256), 0, stream, dst, src,
                           csr, na, row);
    SLK_HIP(hipGetLastError());
    if (active_kf)
        SLK_HIP(hipMemcpyAsync(active_kf, csr + na + 1 + n, na * sizeof(int),
                               hipMemcpyDeviceToDevice, stream));
    if (active_kf_host) std::copy(act.begin(), act.end(), active_kf_host);
    *num_active_host = na;
    return SLK_OK;
}

extern "C" int slk_ba_edge_set(slk_ctx* ctx, const int* ii_host, const int* jj_host, int n,
                               const int* ii_inac_host, const int* jj_inac_host, int n_inac,
                               const float* target, const float* weight,
                               const float* target_inac, const float* weight_inac, int hw,
                               int num_keyframes, int forced_t0, int use_inactive,
                               int* ba_ii_host, int* ba_jj_host, int* ba_ii, int* ba_jj,
                               float* ba_target, float* ba_weight, int* count, int* t0_out,
                               hipStream_t stream) {
    if (!ctx || !count || !t0_out || !ba_ii_host || !ba_jj_host)
        return fail(SLK_E_ARG, "ba_edge_set: null argument");
    if (n < 0 || n_inac < 0 || hw <= 0) return fail(SLK_E_ARG, "ba_edge_set: bad sizes");
    if (n > 0 && (!ii_host || !jj_host)) return fail(SLK_E_ARG, "ba_edge_set: null edges");
    // t0 (main.cu:2312-2322)
    int t0 = forced_t0;
    if (t0 < 0) {
        int mn = num_keyframes;
        for (int e = 0; e < n; e++) mn = std::min(mn, ii_host[e]);
        t0 = std::max(1, mn + 1);
    }
    // active edges, then the inactive ones with both ends >= t0 - 3
    // (main.cu:2330-2339; without inactive edges the active set alone,
    // main.cu:2380-2389)
    std::vector<int> sel;
    const bool inac = use_inactive && n_inac > 0;
    if (inac) {
        if (!ii_inac_host || !jj_inac_host) return fail(SLK_E_ARG, "ba_edge_set: null edges");
        for (int e = 0; e < n_inac; e++)
            if (ii_inac_host[e] >= t0 - 3 && jj_inac_host[e] >= t0 - 3) sel.push_back(e);
    }
    const int m = n + (int)sel.size();
    if (m > 65535) return fail(SLK_E_ARG, "ba_edge_set: more than 65535 edges");
    if (m > 0 && (!ba_ii || !ba_jj || !ba_target || !ba_weight || (n > 0 && (!target || !weight))))
        return fail(SLK_E_ARG, "ba_edge_set: null output");
    if (!sel.empty() && (!target_inac || !weight_inac))
        return fail(SLK_E_ARG, "ba_edge_set: null inactive rows");
    std::copy(ii_host, ii_host + n, ba_ii_host);
    std::copy(jj_host, jj_host + n, ba_jj_host);
    for (size_t k = 0; k < sel.size(); k++) {
        ba_ii_host[n + k] = ii_inac_host[sel[k]];
        ba_jj_host[n + k] = jj_inac_host[sel[k]];
    }
    *count = m;
    *t0_out = t0;
    if (m == 0) return SLK_OK;
    // one upload: [ii][jj][sel]
    std::vector<int> buf((size_t)2 * m + sel.size() + 1);
    std::copy(ba_ii_host, ba_ii_host + m, buf.begin());
    std::copy(ba_jj_host, ba_jj_host + m, buf.begin() + m);
    std::copy(sel.begin(), sel.end(), buf.begin() + 2 * m);
    SLK_TRY(upload(ctx, buf.data(), buf.size() * sizeof(int), stream));
    const int* d = ctx->glue_idx.as<int>();
    SLK_HIP(hipMemcpyAsync(ba_ii, d, m * sizeof(int), hipMemcpyDeviceToDevice, stream));
    SLK_HIP(hipMemcpyAsync(ba_jj, d + m, m * sizeof(int), hipMemcpyDeviceToDevice, stream));
    const long row = 2L * hw;
    const bool v4 = row % 4 == 0 && al16(ba_target) && al16(ba_weight) &&
                    (n == 0 || (al16(target) && al16(weight))) &&
                    (sel.empty() || (al16(target_inac) && al16(weight_inac)));
    if (v4)
        hipLaunchKernelGGL(k_edge_rows<4>, row_grid(row / 4, m), dim3(256), 0, stream, ba_target,
                           ba_weight, target, weight, target_inac, weight_inac, d + 2 * m, n,
                           row);
    else
        hipLaunchKernelGGL(k_edge_rows<1>, row_grid(row, m), dim3(256), 0, stream, ba_target,
                           ba_weight, target, weight, target_inac, weight_inac, d + 2 * m, n,
                           row);
    SLK_HIP(hipGetLastError());
    return SLK_OK;
}

// --------------------------------------------- edge state of the factor graph
namespace slk {
namespace {
// dst rows [0, n) = 0
template <int kV>
__global__ __launch_bounds__(256) void k_zero_rows(float* __restrict__ dst, long row) {
    using V = typename std::conditional<kV == 4, float4, float>::type;
    V* d = reinterpret_cast<V*>(dst + (long)blockIdx.y * row);
    V z;
    if constexpr (kV == 4)
        z = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    else
        z = 0.0f;
    const long nv = row / kV;
    for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < nv;
         i += (long)gridDim.x * blockDim.x)
        d[i] = z;
}

// Moves rows src[e_k] -> dst[d_k] of one array in place (d_k < e_k, both
// increasing) through the context's staging buffer: a row that is the
// destination of one move can be the source of an earlier one, so all
// sources are read before any destination is written.
int move_rows(slk_ctx* ctx, float* base, long row, const int* d_src, const int* d_dst, int k,
              hipStream_t stream) {
    if (k == 0 || row == 0) return SLK_OK;
    const size_t bytes = (size_t)k * row * sizeof(float);
    if (bytes > ctx->edge_stage.bytes && ctx->edge_stage.ptr)
        SLK_HIP(hipDeviceSynchronize());  // earlier moves may still use the old buffer
    SLK_TRY(ctx->edge_stage.ensure(bytes));
    float* stage = ctx->edge_stage.as<float>();
    SLK_TRY(rows_launch(stage, base, d_src, k, row, 0, stream, "store_and_remove_edges"));
    SLK_TRY(rows_launch(base, stage, d_dst, k, row, 1, stream, "store_and_remove_edges"));
    return SLK_OK;
}
}  // namespace
}  // namespace slk

extern "C" void slk_oldest_edges_mask(const int* age_host, int n, int to_remove,
                                      unsigned char* mask_host) {
    if (!mask_host || n <= 0) return;
    std::fill(mask_host, mask_host + n, (unsigned char)0);
    if (!age_host || to_remove <= 0) return;
    std::vector<int> order(n);
    for (int e = 0; e < n; e++) order[e] = e;
    // oldest first; equal ages in edge order (std::sort leaves them unspecified)
    std::stable_sort(order.begin(), order.end(),
                     [&](int a, int b) { return age_host[a] > age_host[b]; });
    for (int r = 0; r < std::min(to_remove, n); r++) mask_host[order[r]] = 1;
}

extern "C" int slk_store_and_remove_edges(slk_ctx* ctx, const unsigned char* mask_host, int n,
                                          int* ii_host, int* jj_host, int* age_host,
                                          int* ii_inac_host, int* jj_inac_host, int* num_inac,
                                          int max_inac, float* edge_nets, long net_row,
                                          float* target, float* weight, float* target_inac,
                                          float* weight_inac, long tw_row, int* n_kept,
                                          hipStream_t stream) {
    if (!ctx || !n_kept || !num_inac) return fail(SLK_E_ARG, "store_and_remove_edges: null argument");
    if (n < 0 || *num_inac < 0 || max_inac < 0 || net_row < 0 || tw_row < 0)
        return fail(SLK_E_ARG, "store_and_remove_edges: bad sizes");
    *n_kept = n;
    if (n == 0) return SLK_OK;
    if (!mask_host || !ii_host || !jj_host)
        return fail(SLK_E_ARG, "store_and_remove_edges: null edge lists");
    if (n > 65535) return fail(SLK_E_ARG, "store_and_remove_edges: more than 65535 edges");
    // the reference's loop (main.cu:795-836): masked edges go to the inactive
    // list while it has room (beyond it they are dropped), kept edges close up
    // in order; rows move with their edges. The moves are listed first and
    // every argument checked before any list changes.
    std::vector<int> stored, src, dst;
    int kept = 0;
    for (int e = 0; e < n; e++) {
        if (mask_host[e]) {
            if (*num_inac + (int)stored.size() < max_inac) stored.push_back(e);
        } else {
            if (kept != e) {
                src.push_back(e);
                dst.push_back(kept);
            }
            kept++;
        }
    }
    const int s = (int)stored.size(), k = (int)src.size();
    if (s > 0 && (!ii_inac_host || !jj_inac_host))
        return fail(SLK_E_ARG, "store_and_remove_edges: null inactive lists");
    if (s > 0 && tw_row > 0 && (!target || !weight || !target_inac || !weight_inac))
        return fail(SLK_E_ARG, "store_and_remove_edges: null target/weight rows");
    if (k > 0 && ((net_row > 0 && !edge_nets) || (tw_row > 0 && (!target || !weight))))
        return fail(SLK_E_ARG, "store_and_remove_edges: null edge rows");
    const int first_inac = *num_inac;
    for (int q = 0; q < s; q++) {
        ii_inac_host[first_inac + q] = ii_host[stored[q]];
        jj_inac_host[first_inac + q] = jj_host[stored[q]];
    }
    for (int q = 0; q < k; q++) {  // src[q] > dst[q], both increasing: in place
        ii_host[dst[q]] = ii_host[src[q]];
        jj_host[dst[q]] = jj_host[src[q]];
        if (age_host) age_host[dst[q]] = age_host[src[q]];
    }
    const int ni = first_inac + s;
    *num_inac = ni;
    *n_kept = kept;
    if (s + k == 0) return SLK_OK;
    // one upload: [stored][src][dst]
    std::vector<int> buf((size_t)s + 2 * k);
    std::copy(stored.begin(), stored.end(), buf.begin());
    std::copy(src.begin(), src.end(), buf.begin() + s);
    std::copy(dst.begin(), dst.end(), buf.begin() + s + k);
    SLK_TRY(upload(ctx, buf.data(), buf.size() * sizeof(int), stream));
    const int* d = ctx->glue_idx.as<int>();
    // the stored rows are read before the moves overwrite them (stream order)
    if (s > 0 && tw_row > 0) {
        SLK_TRY(rows_launch(target_inac + (long)first_inac * tw_row, target, d, s, tw_row, 0,
                            stream, "store_and_remove_edges"));
        SLK_TRY(rows_launch(weight_inac + (long)first_inac * tw_row, weight, d, s, tw_row, 0,
                            stream, "store_and_remove_edges"));
    }
    if (k > 0) {
        SLK_TRY(move_rows(ctx, edge_nets, net_row, d + s, d + s + k, k, stream));
        SLK_TRY(move_rows(ctx, target, tw_row, d + s, d + s + k, k, stream));
        SLK_TRY(move_rows(ctx, weight, tw_row, d + s, d + s + k, k, stream));
    }
    return SLK_OK;
}

extern "C" int slk_init_new_edges(slk_ctx* ctx, const float* nets, float* edge_nets,
                                  float* weight, const int* ii_host, int first, int count,
                                  long net_row, long tw_row, hipStream_t stream) {
    if (count <= 0) return SLK_OK;
    if (!ctx || !ii_host || first < 0 || net_row < 0 || tw_row < 0)
        return fail(SLK_E_ARG, "init_new_edges: bad argument");
    if (count > 65535) return fail(SLK_E_ARG, "init_new_edges: more than 65535 edges");
    if (net_row > 0) {
        if (!nets || !edge_nets) return fail(SLK_E_ARG, "init_new_edges: null hidden states");
        SLK_TRY(upload(ctx, ii_host + first, (size_t)count * sizeof(int), stream));
        SLK_TRY(rows_launch(edge_nets + (long)first * net_row, nets, ctx->glue_idx.as<int>(),
                            count, net_row, 0, stream, "init_new_edges"));
    }
    if (tw_row > 0) {
        if (!weight) return fail(SLK_E_ARG, "init_new_edges: null weight");
        float* w0 = weight + (long)first * tw_row;
        if (tw_row % 4 == 0 && al16(w0))
            hipLaunchKernelGGL(k_zero_rows<4>, row_grid(tw_row / 4, count), dim3(256), 0, stream,
                               w0, tw_row);
        else
            hipLaunchKernelGGL(k_zero_rows<1>, row_grid(tw_row, count), dim3(256), 0, stream,
                               w0, tw_row);
        SLK_HIP(hipGetLastError());
    }
    return SLK_OK;
}

extern "C" int slk_rm_keyframe(slk_ctx* ctx, int ix, int num_keyframes, float* poses,
                               float* disps, void* fmaps, int fmap_dtype, float* nets,
                               float* inps, long net_row, int* ii_host, int* jj_host,
                               int* age_host, int n, int* n_kept, int* ii_inac_host,
                               int* jj_inac_host, int n_inac, int* n_inac_kept,
                               float* edge_nets, float* target, float* weight,
                               float* target_inac, float* weight_inac, hipStream_t stream) {
    if (!ctx || !n_kept || !n_inac_kept) return fail(SLK_E_ARG, "rm_keyframe: null argument");
    if (n < 0 || n_inac < 0 || net_row < 0 || num_keyframes < 0)
        return fail(SLK_E_ARG, "rm_keyframe: bad sizes");
    if (fmap_dtype != SLK_F32 && fmap_dtype != SLK_F16)
        return fail(SLK_E_ARG, "rm_keyframe: fmap dtype must be SLK_F32 or SLK_F16");
    *n_kept = n;
    *n_inac_kept = n_inac;
    const int t = num_keyframes;
    if (ix < 0 || ix >= t) return SLK_OK;  // main.cu:871
    if ((n > 0 && (!ii_host || !jj_host)) || (n_inac > 0 && (!ii_inac_host || !jj_inac_host)))
        return fail(SLK_E_ARG, "rm_keyframe: null edge lists");
    if (t > 65536 || n > 65535 || n_inac > 65535) return fail(SLK_E_ARG, "rm_keyframe: too many rows");
    // keyframe rows ix+1 .. t-1 move down by one (main.cu:874-885)
    std::vector<int> kf_src, kf_dst;
    for (int k = ix; k < t - 1; k++) {
        kf_src.push_back(k + 1);
        kf_dst.push_back(k);
    }
    // edges: those touching ix go, indices above ix drop by one, the rest
    // close up in order with their rows (main.cu:889-917, 920-940)
    auto filter = [ix](int* a, int* b, int* age, int cnt, std::vector<int>& src,
                       std::vector<int>& dst) {
        int kept = 0;
        for (int e = 0; e < cnt; e++) {
            int ei = a[e], ej = b[e];
            if (ei == ix || ej == ix) continue;
            if (ei > ix) ei--;
            if (ej > ix) ej--;
            if (kept != e) {
                src.push_back(e);
                dst.push_back(kept);
            }
            a[kept] = ei;
            b[kept] = ej;
            if (age) age[kept] = age[e];
            kept++;
        }
        return kept;
    };
    std::vector<int> a_src, a_dst, i_src, i_dst;
    const int ka = filter(ii_host, jj_host, age_host, n, a_src, a_dst);
    const int ki = filter(ii_inac_host, jj_inac_host, nullptr, n_inac, i_src, i_dst);
    *n_kept = ka;
    *n_inac_kept = ki;
    const int nk = (int)kf_src.size(), na = (int)a_src.size(), nin = (int)i_src.size();
    if (nk + na + nin == 0) return SLK_OK;
    std::vector<int> buf;
    for (auto* v : {&kf_src, &kf_dst, &a_src, &a_dst, &i_src, &i_dst})
        buf.insert(buf.end(), v->begin(), v->end());
    SLK_TRY(upload(ctx, buf.data(), buf.size() * sizeof(int), stream));
    const int* d = ctx->glue_idx.as<int>();
    const int *dks = d, *dkd = dks + nk, *das = dkd + nk, *dad = das + na, *dis = dad + na,
              *did = dis + nin;
    const long hw = ctx->HW;
    // each array present is moved; a null pointer skips it
    if (nk > 0) {
        if (poses) SLK_TRY(move_rows(ctx, poses, 7, dks, dkd, nk, stream));
        if (disps) SLK_TRY(move_rows(ctx, disps, hw, dks, dkd, nk, stream));
        if (fmaps) {
            const long frow = fmap_dtype == SLK_F16 ? (long)ctx->C * hw / 2 : (long)ctx->C * hw;
            SLK_TRY(move_rows(ctx, static_cast<float*>(fmaps), frow, dks, dkd, nk, stream));
        }
        if (nets) SLK_TRY(move_rows(ctx, nets, net_row, dks, dkd, nk, stream));
        if (inps) SLK_TRY(move_rows(ctx, inps, net_row, dks, dkd, nk, stream));
    }
    if (na > 0) {
        if (edge_nets) SLK_TRY(move_rows(ctx, edge_nets, net_row, das, dad, na, stream));
        if (target) SLK_TRY(move_rows(ctx, target, 2 * hw, das, dad, na, stream));
        if (weight) SLK_TRY(move_rows(ctx, weight, 2 * hw, das, dad, na, stream));
    }
    if (nin > 0) {
        if (target_inac) SLK_TRY(move_rows(ctx, target_inac, 2 * hw, dis, did, nin, stream));
        if (weight_inac) SLK_TRY(move_rows(ctx, weight_inac, 2 * hw, dis, did, nin, stream));
    }
    return SLK_OK;
}
