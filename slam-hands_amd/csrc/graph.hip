// Proximity factors of the factor graph: CudaDroid::add_proximity_factors
// (cuda_slam/main.cu:1679-1779) up to the edge-state update. The distances
// of every (i, j) pair of the window come from one frame_distance launch and
// one read-back (the reference launches and synchronises per 1024 pairs,
// compute_frame_distances_batch, main.cu:1655-1676); the selection that
// follows (invalidation, NMS against existing edges, mandatory neighbour
// edges, greedy best-distance edges) is the reference's host logic, step for
// step, over a few hundred values.
#include <algorithm>
#include <cstdlib>
#include <unordered_set>
#include <vector>

#include "slk_internal.hpp"

namespace slk {
namespace {

// pair k = (i - t0) * jrange + (j - t1): ii[k] = i, jj[k] = j
__global__ __launch_bounds__(256) void k_pairs(int* __restrict__ ii, int* __restrict__ jj, int t0,
                                               int t1, int jrange, int np) {
    const int k = blockIdx.x * blockDim.x + threadIdx.x;
    if (k >= np) return;
    ii[k] = t0 + k / jrange;
    jj[k] = t1 + k % jrange;
}

struct PairSet {
    std::unordered_set<long long> s;
    static long long key(int i, int j) { return ((long long)i << 32) ^ (unsigned)j; }
    bool has(int i, int j) const { return s.count(key(i, j)) != 0; }
    void add(int i, int j) { s.insert(key(i, j)); }
};

}  // namespace
}  // namespace slk

using namespace slk;

extern "C" int slk_proximity_factors(slk_ctx* ctx, const float* poses, const float* disps,
                                     const float* intrinsics, int num_keyframes, int t0, int t1,
                                     int rad, int nms, float thresh, float beta,
                                     const int* ii_host, const int* jj_host, int n_edges,
                                     const int* ii_inac_host, const int* jj_inac_host,
                                     int n_inac, int max_factors, int* new_ii_host,
                                     int* new_jj_host, int capacity, int* n_new, int* n_es,
                                     float* dists_host, hipStream_t stream) {
    if (!ctx || !n_new || !n_es) return fail(SLK_E_ARG, "proximity_factors: null argument");
    *n_new = 0;
    *n_es = 0;
    if (n_edges < 0 || n_inac < 0 || (n_edges > 0 && (!ii_host || !jj_host)) ||
        (n_inac > 0 && (!ii_inac_host || !jj_inac_host)))
        return fail(SLK_E_ARG, "proximity_factors: bad edge lists");
    const int t = num_keyframes;
    if (t < 2) return SLK_OK;  // main.cu:1682
    t0 = std::max(0, t0);
    t1 = std::max(0, t1);
    // 1. distances of all pairs i in [t0, t), j in [t1, t) (main.cu:1686-1697)
    const int irange = std::max(0, t - t0), jrange = std::max(0, t - t1);
    const int np = irange * jrange;
    if (np == 0) return SLK_OK;  // main.cu:1694-1695
    if (!poses || !disps || !intrinsics) return fail(SLK_E_ARG, "proximity_factors: null state");
    SLK_TRY(ctx->graph_pairs.ensure((size_t)np * 2 * sizeof(int)));
    SLK_TRY(ctx->graph_dist.ensure((size_t)np * sizeof(float)));
    int* d_ii = ctx->graph_pairs.as<int>();
    int* d_jj = d_ii + np;
    hipLaunchKernelGGL(k_pairs, dim3((np + 255) / 256), dim3(256), 0, stream, d_ii, d_jj, t0, t1,
                       jrange, np);
    SLK_HIP(hipGetLastError());
    SLK_TRY(slk_frame_distance(poses, disps, intrinsics, d_ii, d_jj,
                               ctx->graph_dist.as<float>(), np, ctx->h, ctx->w, beta, stream));
    std::vector<float> d(np);
    SLK_HIP(hipMemcpyAsync(d.data(), ctx->graph_dist.ptr, np * sizeof(float),
                           hipMemcpyDeviceToHost, stream));
    SLK_HIP(hipStreamSynchronize(stream));
    if (dists_host) std::copy(d.begin(), d.end(), dists_host);

    // 2. invalidate pairs too close in time or too far apart (main.cu:1702-1706)
    for (int k = 0; k < np; k++) {
        const int i = t0 + k / jrange, j = t1 + k % jrange;
        if (i - rad < j) d[k] = 1e6f;
        if (d[k] > 100.0f) d[k] = 1e6f;
    }
    // NMS around existing edges (main.cu:1708-1726)
    auto suppress = [&](int i, int j) {
        const int r = std::max(std::min(std::abs(i - j) - 2, nms), 0);
        for (int di = -nms; di <= nms; di++)
            for (int dj = -nms; dj <= nms; dj++) {
                if (std::abs(di) + std::abs(dj) > r) continue;
                const int i1 = i + di, j1 = j + dj;
                if (i1 >= t0 && i1 < t && j1 >= t1 && j1 < t) {
                    const int idx = (i1 - t0) * jrange + (j1 - t1);
                    if (idx >= 0 && idx < np) d[idx] = 1e6f;
                }
            }
    };
    PairSet have;  // has_edge (main.cu:786-792): active and inactive edges
    for (int e = 0; e < n_edges; e++) {
        suppress(ii_host[e], jj_host[e]);
        have.add(ii_host[e], jj_host[e]);
    }
    for (int e = 0; e < n_inac; e++) {
        suppress(ii_inac_host[e], jj_inac_host[e]);
        have.add(ii_inac_host[e], jj_inac_host[e]);
    }
    // 3. mandatory neighbour edges (main.cu:1728-1736); the index is formed
    // without checking j >= t1, as in the reference
    std::vector<int> es;
    for (int i = t0; i < t; i++)
        for (int j = std::max(i - rad - 1, 0); j < i; j++) {
            if (!have.has(i, j)) {
                es.push_back(i);
                es.push_back(j);
                es.push_back(j);
                es.push_back(i);
            }
            const int idx = (i - t0) * jrange + (j - t1);
            if (idx >= 0 && idx < np) d[idx] = 1e6f;
        }
    // 4. greedy best-distance edges (main.cu:1738-1755). Ascending distance;
    // equal distances in pair order (the reference's std::sort leaves their
    // order unspecified). Pairs above thresh are skipped before the
    // max_factors test and suppression only raises distances, so sorting the
    // pairs at or below thresh visits the same pairs in the same order.
    std::vector<int> order;
    for (int k = 0; k < np; k++)
        if (d[k] <= thresh) order.push_back(k);
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return d[a] < d[b]; });
    for (int k : order) {
        if (d[k] > thresh) continue;
        if (max_factors > 0 && n_edges + (int)es.size() / 2 > max_factors) break;
        const int i = t0 + k / jrange, j = t1 + k % jrange;
        es.push_back(i);
        es.push_back(j);
        es.push_back(j);
        es.push_back(i);
        suppress(i, j);
    }
    *n_es = (int)es.size() / 2;
    // 6. the edges the update appends: those not present yet, each once
    // (main.cu:1773-1781; the age-based removal in between moves edges from
    // the active to the inactive list, which has_edge treats alike)
    int m = 0;
    for (size_t q = 0; q < es.size(); q += 2) {
        const int i = es[q], j = es[q + 1];
        if (have.has(i, j)) continue;
        have.add(i, j);
        if (m < capacity && new_ii_host && new_jj_host) {
            new_ii_host[m] = i;
            new_jj_host[m] = j;
        }
        m++;
    }
    *n_new = m;
    if (m > capacity)
        return fail(SLK_E_ARG, "proximity_factors: more new edges than capacity (see n_new)");
    return SLK_OK;
}
