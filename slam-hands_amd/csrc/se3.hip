// SE3 reprojection kernels (cuda_slam/se3.cuh:116-277 and the clamp of
// main.cu:2392-2397) for gfx950.
#include "reduce.hpp"
#include "se3.hpp"
#include "slk_internal.hpp"

namespace slk {
namespace {

constexpr float kMinDepth = 0.25f;  // se3.cuh:6

// One workgroup per edge; the relative pose is formed once per workgroup in
// LDS, then every thread reprojects a strided set of pixels (se3.cuh:118-177).
__global__ __launch_bounds__(256) void k_projmap(const float* __restrict__ poses,
                                                 const float* __restrict__ disps,
                                                 const float* __restrict__ intr,
                                                 const int* __restrict__ ii,
                                                 const int* __restrict__ jj,
                                                 float* __restrict__ coords,
                                                 float* __restrict__ valid, int M, int H, int W) {
    const int e = blockIdx.y;
    __shared__ float rel[7];
    if (threadIdx.x == 0) {
        float ti[3], qi[4], tj[3], qj[4];
        load_pose(poses, ii[e], ti, qi);
        load_pose(poses, jj[e], tj, qj);
        rel_se3(ti, qi, tj, qj, rel, rel + 3);
    }
    __syncthreads();
    const float tij[3] = {rel[0], rel[1], rel[2]};
    const float qij[4] = {rel[3], rel[4], rel[5], rel[6]};
    const float fx = intr[0], fy = intr[1], cx = intr[2], cy = intr[3];
    const int HW = H * W;
    const int ix = ii[e];
    const int k = blockIdx.x * blockDim.x + threadIdx.x;
    if (k >= HW) return;
    const int i = k / W, j = k - (k / W) * W;
    const float u = (float)j, v = (float)i;
    float Xi[4], Xj[4];
    Xi[0] = (u - cx) / fx;
    Xi[1] = (v - cy) / fy;
    Xi[2] = 1.0f;
    Xi[3] = disps[(size_t)ix * HW + k];
    act_se3(tij, qij, Xi, Xj);
    float2 c;
    if (Xj[2] > 0.01f) {
        c.x = fx * (Xj[0] / Xj[2]) + cx;
        c.y = fy * (Xj[1] / Xj[2]) + cy;
    } else {
        c.x = u;
        c.y = v;
    }
    reinterpret_cast<float2*>(coords)[(size_t)e * HW + k] = c;
    valid[(size_t)e * HW + k] = (Xj[2] > kMinDepth) ? 1.0f : 0.0f;
}

// T_k <- exp(dx[k - t0]) * T_k for k in [t0, t1), evaluated in fp64 and
// rounded once to fp32 (se3.cuh:179-193).
__global__ void k_pose_retr(float* __restrict__ poses, const float* __restrict__ dx, int t0,
                            int t1) {
    for (int k = t0 + blockIdx.x * blockDim.x + threadIdx.x; k < t1;
         k += gridDim.x * blockDim.x) {
        double t[3], q[4], xi[6], t1_[3], q1_[4];
        load_pose(poses, k, t, q);
        for (int n = 0; n < 6; n++) xi[n] = (double)dx[(k - t0) * 6 + n];
        retr_se3(xi, t, q, t1_, q1_);
        for (int n = 0; n < 3; n++) poses[k * 7 + n] = (float)t1_[n];
        for (int n = 0; n < 4; n++) poses[k * 7 + 3 + n] = (float)q1_[n];
    }
}

__global__ void k_disp_retr(float* __restrict__ disps, const float* __restrict__ dz,
                            const int* __restrict__ inds, int HW) {
    const int idx = inds[blockIdx.y];
    const int k = blockIdx.x * blockDim.x + threadIdx.x;
    if (k >= HW) return;
    const float d = disps[(size_t)idx * HW + k] + dz[(size_t)blockIdx.y * HW + k];
    disps[(size_t)idx * HW + k] = fmaxf(d, 0.001f);
}

// Mean flow magnitude of the full and the translation-only reprojection
// (se3.cuh:209-277), one wavefront per pair (four pairs per workgroup): every
// lane forms the pair's relative pose itself (uniform arithmetic, no barrier),
// takes pixels lane, lane + 64, ... and the three sums are reduced across the
// wavefront in a fixed order (deterministic).
__global__ __launch_bounds__(256) void k_frame_distance(const float* __restrict__ poses,
                                                        const float* __restrict__ disps,
                                                        const float* __restrict__ intr,
                                                        const int* __restrict__ ii,
                                                        const int* __restrict__ jj,
                                                        float* __restrict__ dist, int M, int H,
                                                        int W, float beta) {
    const int e = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
    if (e >= M) return;  // uniform over the wavefront
    const int lane = threadIdx.x & 63;
    float tij[3], qij[4];
    {
        float ti[3], qi[4], tj[3], qj[4];
        load_pose(poses, ii[e], ti, qi);
        load_pose(poses, jj[e], tj, qj);
        rel_se3(ti, qi, tj, qj, tij, qij);
    }
    const float fx = intr[0], fy = intr[1], cx = intr[2], cy = intr[3];
    // the reference builds with --use_fast_math (approximate divisions); here
    // each projection takes one hardware reciprocal (v_rcp_f32, 1 ulp) of the
    // depth and the normalised coordinates one reciprocal of each focal length
    const float ifx = 1.0f / fx, ify = 1.0f / fy;
    const int HW = H * W;
    const int ix = ii[e];
    float acc[3] = {0.0f, 0.0f, 0.0f};  // accum, valid, total
    for (int k = lane; k < HW; k += 64) {
        const int i = k / W, j = k - (k / W) * W;
        const float u = (float)j, v = (float)i;
        float Xi[4], Xj[4];
        Xi[0] = (u - cx) * ifx;
        Xi[1] = (v - cy) * ify;
        Xi[2] = 1.0f;
        Xi[3] = disps[(size_t)ix * HW + k];
        act_se3(tij, qij, Xi, Xj);
        float iz = __builtin_amdgcn_rcpf(Xj[2]);
        float du = fx * (Xj[0] * iz) + cx - u, dv = fy * (Xj[1] * iz) + cy - v;
        float d = sqrtf(du * du + dv * dv);
        acc[2] += beta;
        if (Xj[2] > kMinDepth) {
            acc[0] += beta * d;
            acc[1] += beta;
        }
        Xj[0] = Xi[0] + Xi[3] * tij[0];
        Xj[1] = Xi[1] + Xi[3] * tij[1];
        Xj[2] = Xi[2] + Xi[3] * tij[2];
        iz = __builtin_amdgcn_rcpf(Xj[2]);
        du = fx * (Xj[0] * iz) + cx - u;
        dv = fy * (Xj[1] * iz) + cy - v;
        d = sqrtf(du * du + dv * dv);
        acc[2] += (1.0f - beta);
        if (Xj[2] > kMinDepth) {
            acc[0] += (1.0f - beta) * d;
            acc[1] += (1.0f - beta);
        }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1)
#pragma unroll
        for (int q = 0; q < 3; q++) acc[q] += __shfl_xor(acc[q], off, 64);
    if (lane == 0)
        dist[e] = (acc[1] / (acc[2] + 1e-8f) < 0.75f) ? 1000.0f : acc[0] / acc[1];
}


__global__ void k_clamp(float* __restrict__ d, int n, float lo) {
    const int k = blockIdx.x * blockDim.x + threadIdx.x;
    if (k < n) d[k] = fmaxf(d[k], lo);
}

}  // namespace
}  // namespace slk

using namespace slk;

extern "C" int slk_projmap(const float* poses, const float* disps, const float* intrinsics,
                           const int* ii, const int* jj, float* coords, float* valid, int M,
                           int H, int W, hipStream_t stream) {
    if (M < 0 || H < 1 || W < 1) return fail(SLK_E_ARG, "projmap: bad shape");
    if (M == 0) return SLK_OK;
    if (!poses || !disps || !intrinsics || !ii || !jj || !coords || !valid)
        return fail(SLK_E_ARG, "projmap: null argument");
    dim3 grid((H * W + 255) / 256, M);
    hipLaunchKernelGGL(k_projmap, grid, dim3(256), 0, stream, poses, disps, intrinsics, ii, jj,
                       coords, valid, M, H, W);
    SLK_HIP(hipGetLastError());
    return SLK_OK;
}

extern "C" int slk_pose_retr(float* poses, const float* dx, int t0, int t1, hipStream_t stream) {
    if (t1 <= t0) return SLK_OK;
    if (!poses || !dx || t0 < 0) return fail(SLK_E_ARG, "pose_retr: bad args");
    hipLaunchKernelGGL(k_pose_retr, dim3((t1 - t0 + 63) / 64), dim3(64), 0, stream, poses, dx, t0,
                       t1);
    SLK_HIP(hipGetLastError());
    return SLK_OK;
}

extern "C" int slk_disp_retr(float* disps, const float* dz, const int* inds, int num_inds, int HW,
                             hipStream_t stream) {
    if (num_inds <= 0 || HW <= 0) return SLK_OK;
    if (!disps || !dz || !inds) return fail(SLK_E_ARG, "disp_retr: null argument");
    hipLaunchKernelGGL(k_disp_retr, dim3((HW + 255) / 256, num_inds), dim3(256), 0, stream, disps,
                       dz, inds, HW);
    SLK_HIP(hipGetLastError());
    return SLK_OK;
}

extern "C" int slk_frame_distance(const float* poses, const float* disps, const float* intrinsics,
                                  const int* ii, const int* jj, float* dist, int M, int H, int W,
                                  float beta, hipStream_t stream) {
    if (M <= 0) return SLK_OK;
    if (!poses || !disps || !intrinsics || !ii || !jj || !dist || H < 1 || W < 1)
        return fail(SLK_E_ARG, "frame_distance: bad args");
    hipLaunchKernelGGL(k_frame_distance, dim3((M + 3) / 4), dim3(256), 0, stream, poses, disps,
                       intrinsics, ii, jj, dist, M, H, W, beta);
    SLK_HIP(hipGetLastError());
    return SLK_OK;
}

extern "C" int slk_clamp_disps(float* disps, int n, float min_val, hipStream_t stream) {
    if (n <= 0) return SLK_OK;
    if (!disps) return fail(SLK_E_ARG, "clamp_disps: null argument");
    hipLaunchKernelGGL(k_clamp, dim3((n + 255) / 256), dim3(256), 0, stream, disps, n, min_val);
    SLK_HIP(hipGetLastError());
    return SLK_OK;
}
