// The front of the pipe for gfx950: decoded video frames to the float BGR
// frame the SLAM path takes (cuda_slam/main.cu:944-1058), the frame
// preprocessing of encode_frame (main.cu:1062-1075), and the keyframe pose
// file written at the end of a run (main.cu:2893-2937).
//
// The conversions are one thread per output pixel (HBM-bound: a source
// pixel's 2x2 neighbourhood in, 12 bytes out). Floating-point contraction is
// off in their bodies, so each product and sum is rounded once in the
// written order and a float32 restatement on the CPU reproduces every
// output bit.

#include <cmath>
#include <cstdio>
#include <string>
#include <vector>

#include "slk_internal.hpp"

namespace slk {
namespace {

struct Bilin {
    int x0, x1, y0, y1;
    float wx, wy, sx, sy;
};

// the source sampling position of output pixel (dx, dy) and its clamped
// 2x2 neighbourhood (pixel-centre aligned, main.cu:957-962)
__device__ __forceinline__ Bilin bilin(int dx, int dy, int src_w, int src_h, int dst_w, int dst_h) {
#pragma clang fp contract(off)
    Bilin b;
    b.sx = ((float)dx + 0.5f) * src_w / dst_w - 0.5f;
    b.sy = ((float)dy + 0.5f) * src_h / dst_h - 0.5f;
    b.x0 = (int)floorf(b.sx);
    b.y0 = (int)floorf(b.sy);
    b.wx = b.sx - b.x0;
    b.wy = b.sy - b.y0;
    b.x1 = min(b.x0 + 1, src_w - 1);
    b.y1 = min(b.y0 + 1, src_h - 1);
    b.x0 = max(b.x0, 0);
    b.y0 = max(b.y0, 0);
    return b;
}

__device__ __forceinline__ float lerp2(const Bilin& b, float v00, float v01, float v10, float v11) {
#pragma clang fp contract(off)
    return (1 - b.wy) * ((1 - b.wx) * v00 + b.wx * v01) + b.wy * ((1 - b.wx) * v10 + b.wx * v11);
}

// BT.709 YUV (offset chroma) to clamped BGR (main.cu:976-984)
__device__ __forceinline__ void yuv_to_bgr(float Y, float U, float V, float* o) {
#pragma clang fp contract(off)
    const float R = Y + 1.5748f * V;
    const float G = Y - 0.1873f * U - 0.4681f * V;
    const float B = Y + 1.8556f * U;
    o[0] = fminf(fmaxf(B, 0.0f), 255.0f);
    o[1] = fminf(fmaxf(G, 0.0f), 255.0f);
    o[2] = fminf(fmaxf(R, 0.0f), 255.0f);
}

// nearest chroma sample of a half-resolution interleaved UV plane
// (main.cu:967-971)
__device__ __forceinline__ void uv_index(const Bilin& b, int src_w, int src_h, int* ux, int* uy) {
    int x = ((int)(b.sx + 0.5f) / 2) * 2;
    int y = (int)(b.sy + 0.5f) / 2;
    *ux = max(0, min(x, src_w - 2));
    *uy = max(0, min(y, src_h / 2 - 1));
}

// NV12 (8-bit Y plane + interleaved UV) -> float BGR HWC, bilinear Y and
// nearest UV (nv12_to_bgr_resize_kernel, main.cu:947-985)
__global__ void k_nv12_to_bgr(const uint8_t* yp, const uint8_t* uvp, float* out, int src_w,
                              int src_h, int y_stride, int uv_stride, int dst_w, int dst_h) {
#pragma clang fp contract(off)
    const int dx = blockIdx.x * blockDim.x + threadIdx.x;
    const int dy = blockIdx.y * blockDim.y + threadIdx.y;
    if (dx >= dst_w || dy >= dst_h) return;
    const Bilin b = bilin(dx, dy, src_w, src_h, dst_w, dst_h);
    auto Yv = [&](int r, int c) { return (float)yp[(long)r * y_stride + c]; };
    const float Y = lerp2(b, Yv(b.y0, b.x0), Yv(b.y0, b.x1), Yv(b.y1, b.x0), Yv(b.y1, b.x1));
    int ux, uy;
    uv_index(b, src_w, src_h, &ux, &uy);
    const float U = (float)uvp[(long)uy * uv_stride + ux] - 128.0f;
    const float V = (float)uvp[(long)uy * uv_stride + ux + 1] - 128.0f;
    yuv_to_bgr(Y, U, V, out + ((long)dy * dst_w + dx) * 3);
}

// P010 (10 significant bits at the top of 16) -> float BGR, scaled to the
// 8-bit range (p010_to_bgr_resize_kernel, main.cu:988-1027); strides in bytes
__global__ void k_p010_to_bgr(const uint16_t* yp, const uint16_t* uvp, float* out, int src_w,
                              int src_h, int y_stride_b, int uv_stride_b, int dst_w, int dst_h) {
#pragma clang fp contract(off)
    const int dx = blockIdx.x * blockDim.x + threadIdx.x;
    const int dy = blockIdx.y * blockDim.y + threadIdx.y;
    if (dx >= dst_w || dy >= dst_h) return;
    const int ys = y_stride_b / 2, uvs = uv_stride_b / 2;
    const Bilin b = bilin(dx, dy, src_w, src_h, dst_w, dst_h);
    auto Yv = [&](int r, int c) { return (float)(yp[(long)r * ys + c] >> 6) / 4.0f; };
    const float Y = lerp2(b, Yv(b.y0, b.x0), Yv(b.y0, b.x1), Yv(b.y1, b.x0), Yv(b.y1, b.x1));
    int ux, uy;
    uv_index(b, src_w, src_h, &ux, &uy);
    const float U = (float)(uvp[(long)uy * uvs + ux] >> 6) / 4.0f - 128.0f;
    const float V = (float)(uvp[(long)uy * uvs + ux + 1] >> 6) / 4.0f - 128.0f;
    yuv_to_bgr(Y, U, V, out + ((long)dy * dst_w + dx) * 3);
}

// 8-bit BGR (CPU-decoded) -> float BGR with bilinear resize
// (bgr8_to_bgrf_resize_kernel, main.cu:1030-1058); stride in bytes
__global__ void k_bgr8_to_bgrf(const uint8_t* in, float* out, int src_w, int src_h, int stride,
                               int dst_w, int dst_h) {
#pragma clang fp contract(off)
    const int dx = blockIdx.x * blockDim.x + threadIdx.x;
    const int dy = blockIdx.y * blockDim.y + threadIdx.y;
    if (dx >= dst_w || dy >= dst_h) return;
    const Bilin b = bilin(dx, dy, src_w, src_h, dst_w, dst_h);
    float* o = out + ((long)dy * dst_w + dx) * 3;
    for (int c = 0; c < 3; c++) {
        auto v = [&](int r, int x) { return (float)in[(long)r * stride + x * 3 + c]; };
        o[c] = lerp2(b, v(b.y0, b.x0), v(b.y0, b.x1), v(b.y1, b.x0), v(b.y1, b.x1));
    }
}

// BGR HWC (0..255) -> normalised RGB NCHW (preprocess_image_kernel,
// main.cu:1062-1075)
__global__ void k_preprocess(const float* bgr, float* rgb, int hw) {
    const int p = blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= hw) return;
    const float mean[3] = {0.406f, 0.456f, 0.485f};  // B, G, R
    const float sd[3] = {0.225f, 0.224f, 0.229f};
    for (int c = 0; c < 3; c++) rgb[(long)(2 - c) * hw + p] = (bgr[(long)p * 3 + c] / 255.0f - mean[c]) / sd[c];
}

int check_resize(const void* a, const void* b, const void* c, int src_w, int src_h, int dst_w,
                 int dst_h, const char* what) {
    if (!a || !b || !c || src_w < 2 || src_h < 2 || dst_w < 1 || dst_h < 1)
        return fail(SLK_E_ARG, std::string(what) + ": null pointer or sizes below 2x2 / 1x1");
    return SLK_OK;
}

const dim3 kBlock(32, 8);
dim3 grid_of(int w, int h) { return dim3((w + 31) / 32, (h + 7) / 8); }

}  // namespace
}  // namespace slk

using namespace slk;

extern "C" int slk_nv12_to_bgr(const uint8_t* y_plane, const uint8_t* uv_plane, float* bgr_out,
                               int src_w, int src_h, int y_stride, int uv_stride, int dst_w,
                               int dst_h, hipStream_t stream) {
    SLK_TRY(check_resize(y_plane, uv_plane, bgr_out, src_w, src_h, dst_w, dst_h, "nv12_to_bgr"));
    if (y_stride < src_w || uv_stride < src_w || src_w % 2 || src_h % 2)
        return fail(SLK_E_ARG, "nv12_to_bgr: strides below the width or odd source sides");
    hipLaunchKernelGGL(k_nv12_to_bgr, grid_of(dst_w, dst_h), kBlock, 0, stream, y_plane, uv_plane,
                       bgr_out, src_w, src_h, y_stride, uv_stride, dst_w, dst_h);
    SLK_HIP(hipGetLastError());
    return SLK_OK;
}

extern "C" int slk_p010_to_bgr(const uint16_t* y_plane, const uint16_t* uv_plane, float* bgr_out,
                               int src_w, int src_h, int y_stride_bytes, int uv_stride_bytes,
                               int dst_w, int dst_h, hipStream_t stream) {
    SLK_TRY(check_resize(y_plane, uv_plane, bgr_out, src_w, src_h, dst_w, dst_h, "p010_to_bgr"));
    if (y_stride_bytes < 2 * src_w || uv_stride_bytes < 2 * src_w || (y_stride_bytes | uv_stride_bytes) & 1 ||
        src_w % 2 || src_h % 2)
        return fail(SLK_E_ARG, "p010_to_bgr: strides below 2*width, odd strides or odd sides");
    hipLaunchKernelGGL(k_p010_to_bgr, grid_of(dst_w, dst_h), kBlock, 0, stream, y_plane, uv_plane,
                       bgr_out, src_w, src_h, y_stride_bytes, uv_stride_bytes, dst_w, dst_h);
    SLK_HIP(hipGetLastError());
    return SLK_OK;
}

extern "C" int slk_bgr8_to_bgrf(const uint8_t* bgr_in, float* bgr_out, int src_w, int src_h,
                                int src_stride, int dst_w, int dst_h, hipStream_t stream) {
    SLK_TRY(check_resize(bgr_in, bgr_out, bgr_out, src_w, src_h, dst_w, dst_h, "bgr8_to_bgrf"));
    if (src_stride < 3 * src_w) return fail(SLK_E_ARG, "bgr8_to_bgrf: stride below 3*width");
    hipLaunchKernelGGL(k_bgr8_to_bgrf, grid_of(dst_w, dst_h), kBlock, 0, stream, bgr_in, bgr_out,
                       src_w, src_h, src_stride, dst_w, dst_h);
    SLK_HIP(hipGetLastError());
    return SLK_OK;
}

extern "C" int slk_preprocess_image(const float* bgr_hwc, float* rgb_nchw, int H, int W,
                                    hipStream_t stream) {
    if (!bgr_hwc || !rgb_nchw || H < 1 || W < 1)
        return fail(SLK_E_ARG, "preprocess_image: bad argument");
    const int hw = H * W;
    hipLaunchKernelGGL(k_preprocess, dim3((hw + 255) / 256), dim3(256), 0, stream, bgr_hwc,
                       rgb_nchw, hw);
    SLK_HIP(hipGetLastError());
    return SLK_OK;
}

// world->camera to camera->world of one pose, in the reference's float
// arithmetic (main.cu:2896-2914): q^-1 = conjugate, t^-1 = -(q^-1 * t)
static void invert_pose(float* p) {
#pragma clang fp contract(off)
    const float qi[4] = {-p[3], -p[4], -p[5], p[6]};
    const float t[3] = {-p[0], -p[1], -p[2]};
    float uv[3];
    uv[0] = 2.0f * (qi[1] * t[2] - qi[2] * t[1]);
    uv[1] = 2.0f * (qi[2] * t[0] - qi[0] * t[2]);
    uv[2] = 2.0f * (qi[0] * t[1] - qi[1] * t[0]);
    p[0] = t[0] + qi[3] * uv[0] + (qi[1] * uv[2] - qi[2] * uv[1]);
    p[1] = t[1] + qi[3] * uv[1] + (qi[2] * uv[0] - qi[0] * uv[2]);
    p[2] = t[2] + qi[3] * uv[2] + (qi[0] * uv[1] - qi[1] * uv[0]);
    p[3] = qi[0];
    p[4] = qi[1];
    p[5] = qi[2];
    p[6] = qi[3];
}

extern "C" int slk_write_poses_bin(const char* path, int num_keyframes, const int* timestamps,
                                   const float* poses, int cam_to_world) {
    if (!path || num_keyframes < 0 || (num_keyframes > 0 && (!timestamps || !poses)))
        return fail(SLK_E_ARG, "write_poses_bin: bad argument");
    std::vector<float> p(poses, poses + (size_t)num_keyframes * 7);
    if (cam_to_world)
        for (int i = 0; i < num_keyframes; i++) invert_pose(&p[(size_t)i * 7]);
    FILE* f = std::fopen(path, "wb");
    if (!f) return fail(SLK_E_ARG, std::string("write_poses_bin: cannot open ") + path);
    bool ok = std::fwrite(&num_keyframes, sizeof(int), 1, f) == 1;
    if (num_keyframes > 0) {
        ok = ok && std::fwrite(timestamps, sizeof(int), num_keyframes, f) == (size_t)num_keyframes;
        ok = ok && std::fwrite(p.data(), sizeof(float), p.size(), f) == p.size();
    }
    ok = std::fclose(f) == 0 && ok;
    if (!ok) return fail(SLK_E_ARG, std::string("write_poses_bin: write failed on ") + path);
    return SLK_OK;
}
