// The DROID-SLAM feature and context encoders for gfx950: HalfBasicEncoder
// with its HalfResBlocks (cuda_slam/main.cu:236-381) and the encode step of
// CudaDroid::encode_frame (main.cu:1465-1497).
//
// Numerics of the reference restated:
//  * every convolution is a cuDNN fp16 convolution with fp32 accumulation
//    (HalfConvLayer, nn.cuh:668-791): weights rounded to fp16, the fp32 sum
//    written as fp16, then the fp32 bias added and rounded again
//    (bias_add_half_kernel, nn.cuh:657-665). Here the sum is formed by
//    v_mfma_f32_32x32x16_f16 and the epilogue applies both roundings;
//  * instance norm (instance_norm_half_kernel, nn.cuh:609-654): mean and
//    variance over the h*w pixels of one channel of fp16 data in fp32, eps
//    1e-5, result rounded to fp16. Here a statistics kernel writes per-split
//    (mean, M2) pairs and the normalising kernel combines them (the total
//    mean from the split means, then M2 = sum of the splits' M2 plus their
//    count-weighted squared mean offsets) before it applies the norm, the
//    ReLU and the residual add of the block in one pass;
//  * ReLU and the residual add of fp16 values (relu_half_kernel,
//    add_half_kernel, nn.cuh:588-607) are exact / one rounding.
//
// Activations use the update operator's "CK" layout, [image][C/16][h*w][16]
// fp16, so a 16-channel chunk of a patch of pixels is a few contiguous rows.
// The input image is [h*w][4] fp16 (R, G, B, 0), read by a stem kernel
// whose K steps pack 4 taps x 4 channels.

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "slk_internal.hpp"

namespace slk {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

constexpr int kTW = 32;  // output columns per tile: one MFMA column block

__device__ __forceinline__ float r16(float x) { return (float)(_Float16)x; }

enum EncEpi {
    kEpRaw = 0,      // y = round16(round16(conv) + b)
    kEpRelu = 1,     // relu(y)
    kEpAddRelu = 2,  // relu(round16(relu(y) + res)), res a CK tensor of the output shape
    kEpNchw = 3,     // y to an NCHW fp16 output (the encoder's result)
    kEpNetInp = 4,   // channels < 128: net = tanh(y); the rest: inp = relu(y), NCHW fp32
};

struct EncArgs {
    const _Float16* in;  // CK input
    long in_nstride;
    int nchunk, ih, iw;
    const _Float16* wt;  // [taps][nchunk][co_pad][16]
    const float* bias;   // [co_pad]
    int co_pad, Co;
    int oh, ow, tiles_x;
    _Float16* out;  // CK output, or NCHW fp16 for kEpNchw
    long out_nstride;
    const _Float16* res;  // kEpAddRelu
    long res_nstride;
    float* net;  // kEpNetInp
    float* inp;
    long ni_nstride;
};

// The epilogue of one lane's accumulator block: register v holds output
// channel co0 + 8*(v/4) + v%4 (co0 includes the lane's 4*lhi) at pixel p.
template <int EPI>
__device__ __forceinline__ void enc_epilogue(const EncArgs& a, const f32x16& acc, int n, int co0,
                                             int p, int ohw) {
#pragma unroll
    for (int g = 0; g < 4; g++) {
        const int co = co0 + 8 * g;
        if (co >= a.Co) continue;
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = r16(r16(acc[4 * g + i]) + a.bias[co + i]);
        const long ck = ((long)(co >> 4) * ohw + p) * 16 + (co & 15);
        if constexpr (EPI == kEpRaw || EPI == kEpRelu) {
            f16x4 o;
#pragma unroll
            for (int i = 0; i < 4; i++) o[i] = (_Float16)(EPI == kEpRelu ? fmaxf(v[i], 0.0f) : v[i]);
            *reinterpret_cast<f16x4*>(a.out + (long)n * a.out_nstride + ck) = o;
        } else if constexpr (EPI == kEpAddRelu) {
            const f16x4 rs = *reinterpret_cast<const f16x4*>(a.res + (long)n * a.res_nstride + ck);
            f16x4 o;
#pragma unroll
            for (int i = 0; i < 4; i++)
                o[i] = (_Float16)fmaxf(r16(fmaxf(v[i], 0.0f) + (float)rs[i]), 0.0f);
            *reinterpret_cast<f16x4*>(a.out + (long)n * a.out_nstride + ck) = o;
        } else if constexpr (EPI == kEpNchw) {
#pragma unroll
            for (int i = 0; i < 4; i++)
                a.out[(long)n * a.out_nstride + (long)(co + i) * ohw + p] = (_Float16)v[i];
        } else {  // kEpNetInp
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int cc = co + i;
                if (cc < 128)
                    a.net[(long)n * a.ni_nstride + (long)cc * ohw + p] = tanhf(v[i]);
                else
                    a.inp[(long)n * a.ni_nstride + (long)(cc - 128) * ohw + p] = fmaxf(v[i], 0.0f);
            }
        }
    }
}

// 3x3 and 1x1 convolutions. One workgroup: 4 waves in a WM x WN grid, wave
// (wm, wn) computing output channels cot*CO_T + wm*32 .. +31 of output row
// ty0 + wn, 32 consecutive columns. The layers are small (at most 8 input
// chunks, a few KB of patch per chunk), so a workgroup stages the input
// patches of up to NCH chunks at once: every global load of the group is
// issued before the first is stored to LDS, one barrier, then the MFMAs of
// all NCH chunks. The weight fragments of chunk c+1 (all taps) are loaded
// during chunk c's MFMAs (two register sets).
template <int KS, int S, int WM, int NCH, int EPI>
__global__ __launch_bounds__(256) void k_enc_conv(EncArgs a) {
    static_assert(NCH % 2 == 0, "register sets alternate by chunk parity");
    constexpr int WN = 4 / WM, TH = WN, CO_T = WM * 32;
    constexpr int P = KS / 2;
    constexpr int PH = S * (TH - 1) + KS, PW = S * (kTW - 1) + KS;
    constexpr int UNITS = PH * PW * 2;  // 16-byte units of one chunk's patch
    constexpr int UPT = (UNITS + 255) / 256;
    constexpr int TAPS = KS * KS;
    __shared__ __attribute__((aligned(16))) _Float16 patch[NCH][PH * PW * 16];
    const int ihw = a.ih * a.iw;
    const int cot = blockIdx.x, tile = blockIdx.y, n = blockIdx.z;
    const int ty0 = (tile / a.tiles_x) * TH, tx0 = (tile % a.tiles_x) * kTW;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave % WM, wn = wave / WM;
    const int l32 = lane & 31, lhi = lane >> 5;
    const int iy0 = S * ty0 - P, ix0 = S * tx0 - P;

    const _Float16* wbase = a.wt + ((long)cot * CO_T + wm * 32 + l32) * 16 + lhi * 8;
    const long tap_stride = (long)a.nchunk * a.co_pad * 16;
    f16x8 A[2][TAPS];
    auto load_a = [&](int c, f16x8* dst) {
#pragma unroll
        for (int t = 0; t < TAPS; t++)
            dst[t] = *reinterpret_cast<const f16x8*>(wbase + t * tap_stride + (long)c * a.co_pad * 16);
    };
    load_a(0, A[0]);
    f32x16 acc = {};
    for (int g0 = 0; g0 < a.nchunk; g0 += NCH) {
        const int ng = min(NCH, a.nchunk - g0);
        if (g0 > 0) __syncthreads();  // the previous group's patches are consumed
        f16x8 reg[NCH][UPT];
#pragma unroll
        for (int q = 0; q < NCH; q++) {
            const _Float16* base = a.in + (long)n * a.in_nstride + (long)(g0 + q) * ihw * 16;
#pragma unroll
            for (int u = 0; u < UPT; u++) {
                const int unit = tid + 256 * u;
                const int pix = unit >> 1, half = unit & 1;
                const int py = pix / PW, px = pix - (pix / PW) * PW;
                const int y = iy0 + py, x = ix0 + px;
                const bool ok = q < ng && unit < UNITS && y >= 0 && y < a.ih && x >= 0 && x < a.iw;
                f16x8 v = {};
                if (ok) v = *reinterpret_cast<const f16x8*>(base + ((long)y * a.iw + x) * 16 + half * 8);
                reg[q][u] = v;
            }
        }
#pragma unroll
        for (int q = 0; q < NCH; q++)
#pragma unroll
            for (int u = 0; u < UPT; u++) {
                const int unit = tid + 256 * u;
                if (q < ng && unit < UNITS) *reinterpret_cast<f16x8*>(&patch[q][unit * 8]) = reg[q][u];
            }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < NCH; q++) {
            if (q < ng) {
                const int c = g0 + q;
                if (c + 1 < a.nchunk) load_a(c + 1, A[(q + 1) & 1]);
                const _Float16* pb = &patch[q][0];
#pragma unroll
                for (int t = 0; t < TAPS; t++) {
                    const int ky = t / KS, kx = t - (t / KS) * KS;
                    const f16x8 b = *reinterpret_cast<const f16x8*>(
                        pb + (((S * wn + ky) * PW + S * l32 + kx) * 16 + lhi * 8));
                    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[q & 1][t], b, acc, 0, 0, 0);
                }
            }
        }
    }
    const int y = ty0 + wn, x = tx0 + l32;
    if (y < a.oh && x < a.ow)
        enc_epilogue<EPI>(a, acc, n, cot * CO_T + wm * 32 + 4 * lhi, y * a.ow + x, a.oh * a.ow);
}

// conv1 (7x7, stride 2, 3 -> 32 channels) with the taps packed into K: the
// image is [image][h*w][4] fp16 (R, G, B, 0) and K step ks covers taps
// 4*ks .. 4*ks+3 with their 4 channels (k = 4*(t - 4*ks) + c), 13 steps for
// the 49 taps (taps 49..51 have zero weights). Lane (l32, lhi) reads two
// 8-byte pixels of the LDS patch per step. Workgroup: 32 channels x 4 output
// rows x 32 columns, wave wn = one row.
template <int EPI>
__global__ __launch_bounds__(256) void k_enc_stem(EncArgs a) {
    constexpr int KS = 7, S = 2, P = 3, TH = 4, KSTEPS = 13;
    constexpr int PH = S * (TH - 1) + KS, PW = S * (kTW - 1) + KS;
    constexpr int UNITS = PH * PW;  // 8-byte pixels of the patch
    constexpr int UPT = (UNITS + 255) / 256;
    __shared__ __attribute__((aligned(16))) _Float16 patch[PH * PW * 4];
    const int tile = blockIdx.y, n = blockIdx.z;
    const int ty0 = (tile / a.tiles_x) * TH, tx0 = (tile % a.tiles_x) * kTW;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wn = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, lhi = lane >> 5;
    const int iy0 = S * ty0 - P, ix0 = S * tx0 - P;
    const _Float16* img = a.in + (long)n * a.in_nstride;
    f16x4 reg[UPT];
#pragma unroll
    for (int u = 0; u < UPT; u++) {
        const int pix = tid + 256 * u;
        const int py = pix / PW, px = pix - (pix / PW) * PW;
        const int y = iy0 + py, x = ix0 + px;
        f16x4 v = {};
        if (pix < UNITS && y >= 0 && y < a.ih && x >= 0 && x < a.iw)
            v = *reinterpret_cast<const f16x4*>(img + ((long)y * a.iw + x) * 4);
        reg[u] = v;
    }
    f16x8 A[KSTEPS];
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ks++)
        A[ks] = *reinterpret_cast<const f16x8*>(a.wt + ((long)ks * 32 + l32) * 16 + lhi * 8);
#pragma unroll
    for (int u = 0; u < UPT; u++) {
        const int pix = tid + 256 * u;
        if (pix < UNITS) *reinterpret_cast<f16x4*>(&patch[pix * 4]) = reg[u];
    }
    __syncthreads();
    f32x16 acc = {};
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ks++) {
        const int t0 = min(4 * ks + 2 * lhi, 48), t1 = min(4 * ks + 2 * lhi + 1, 48);
        const int ky0 = t0 / KS, kx0 = t0 - ky0 * KS, ky1 = t1 / KS, kx1 = t1 - ky1 * KS;
        const f16x4 b0 = *reinterpret_cast<const f16x4*>(
            &patch[((S * wn + ky0) * PW + S * l32 + kx0) * 4]);
        const f16x4 b1 = *reinterpret_cast<const f16x4*>(
            &patch[((S * wn + ky1) * PW + S * l32 + kx1) * 4]);
        const f16x8 b = {b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[ks], b, acc, 0, 0, 0);
    }
    const int y = ty0 + wn, x = tx0 + l32;
    if (y < a.oh && x < a.ow) enc_epilogue<EPI>(a, acc, n, 4 * lhi, y * a.ow + x, a.oh * a.ow);
}

constexpr int kSplit = 256;  // pixels per statistics split (2 per thread pair)

// Per-split statistics of one 16-channel chunk of a CK tensor: pixels
// [s*kSplit, min(hw, (s+1)*kSplit)) of image n; part[(n*nsplit + s)*C + c] =
// (mean, sum of squared deviations from that mean), both in fp32. Thread t
// holds channels 8*(t&1) .. +7 of pixels s*kSplit + (t>>1) + 128*i.
__global__ __launch_bounds__(256) void k_in_stats(const _Float16* y, long nstride, int hw,
                                                  int C, int nsplit, float2* part) {
    __shared__ float red[4][2][8];
    __shared__ float tot_s[16], mean_s[16], m2_s[16];
    const int ch = blockIdx.x, s = blockIdx.y, n = blockIdx.z;
    const int t = threadIdx.x, half = t & 1, pl = t >> 1;
    const int lane = t & 63, wave = t >> 6;
    const int p0 = s * kSplit, p1 = min(hw, p0 + kSplit);
    const _Float16* base = y + (long)n * nstride + (long)ch * hw * 16 + half * 8;
    constexpr int kIt = kSplit / 128;
    f16x8 v[kIt];
    float acc[8];
#pragma unroll
    for (int k = 0; k < 8; k++) acc[k] = 0.0f;
#pragma unroll
    for (int i = 0; i < kIt; i++) {
        const int p = p0 + pl + 128 * i;
        v[i] = f16x8{};
        if (p < p1) v[i] = *reinterpret_cast<const f16x8*>(base + (long)p * 16);
#pragma unroll
        for (int k = 0; k < 8; k++) acc[k] += (float)v[i][k];
    }
    // sum over the 128 threads of one half: lanes of equal parity, then waves
    auto reduce = [&](float* vals, float* outv) {
#pragma unroll
        for (int k = 0; k < 8; k++) {
            float x = vals[k];
#pragma unroll
            for (int off = 2; off < 64; off <<= 1) x += __shfl_xor(x, off);
            vals[k] = x;
        }
        if (lane < 2) {
#pragma unroll
            for (int k = 0; k < 8; k++) red[wave][lane][k] = vals[k];
        }
        __syncthreads();
        if (t < 16) {
            const int hh = t >> 3, k = t & 7;
            outv[t] = ((red[0][hh][k] + red[1][hh][k]) + red[2][hh][k]) + red[3][hh][k];
        }
        __syncthreads();
    };
    reduce(acc, tot_s);
    const float cnt = (float)(p1 - p0);
    if (t < 16) mean_s[t] = tot_s[t] / cnt;
    __syncthreads();
    float m[8];
#pragma unroll
    for (int k = 0; k < 8; k++) m[k] = mean_s[half * 8 + k];
#pragma unroll
    for (int k = 0; k < 8; k++) acc[k] = 0.0f;
#pragma unroll
    for (int i = 0; i < kIt; i++) {
        if (p0 + pl + 128 * i < p1) {
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const float d = (float)v[i][k] - m[k];
                acc[k] += d * d;
            }
        }
    }
    reduce(acc, m2_s);
    if (t < 16) part[((long)n * nsplit + s) * C + ch * 16 + t] = make_float2(mean_s[t], m2_s[t]);
}

// (mean, 1/sqrt(var + 1e-5)) of the 16 channels of chunk ch of image n from
// their nsplit partials, into mom[16]: 16 threads per channel (all 256 of
// the workgroup take part), the total mean from the count-weighted split
// means, then the sum of squared deviations as sum_s M2_s + n_s (mean_s -
// mean)^2, each a fixed-order sum per thread and a fixed butterfly over
// the 16 threads.
__device__ void in_moments16(const float2* part, int n, int nsplit, int C, int ch, int hw,
                             float2* mom) {
    const int t = threadIdx.x, c = t >> 4, j = t & 15;
    const float2* q = part + (long)n * nsplit * C + ch * 16 + c;
    float s1 = 0.0f;
    for (int s = j; s < nsplit; s += 16) s1 += (float)min(kSplit, hw - s * kSplit) * q[(long)s * C].x;
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) s1 += __shfl_xor(s1, off);
    const float mean = s1 / (float)hw;
    float s2 = 0.0f;
    for (int s = j; s < nsplit; s += 16) {
        const float2 v = q[(long)s * C];
        const float d = v.x - mean;
        s2 += v.y + (float)min(kSplit, hw - s * kSplit) * d * d;
    }
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) s2 += __shfl_xor(s2, off);
    if (j == 0) mom[c] = make_float2(mean, 1.0f / sqrtf(s2 / (float)hw + 1e-5f));
}

enum InMode {
    kInRelu = 0,     // y = relu(round16(norm(y)))
    kInAddRelu = 1,  // out = relu(round16(relu(round16(norm(y))) + res))
    kInAddNorm = 2,  // out = relu(round16(relu(round16(norm(y))) + round16(norm2(res))))
};

// Normalises one CK tensor in place (or into out), fused with the block's
// ReLU and residual add: grid (ceil(hw/128), C/16, images), thread = 8
// channels of one pixel.
template <int MODE>
__global__ __launch_bounds__(256) void k_in_apply(_Float16* y, const float2* part,
                                                  const _Float16* res, const float2* part2,
                                                  _Float16* out, long nstride, int hw, int C,
                                                  int nsplit) {
    __shared__ float2 mom[2][16];
    const int ch = blockIdx.y, n = blockIdx.z, t = threadIdx.x;
    in_moments16(part, n, nsplit, C, ch, hw, mom[0]);
    if constexpr (MODE == kInAddNorm) in_moments16(part2, n, nsplit, C, ch, hw, mom[1]);
    __syncthreads();
    const int p = blockIdx.x * 128 + (t >> 1), half = t & 1;
    if (p >= hw) return;
    const long off = (long)n * nstride + ((long)ch * hw + p) * 16 + half * 8;
    const f16x8 v = *reinterpret_cast<const f16x8*>(y + off);
    f16x8 rs = {};
    if constexpr (MODE != kInRelu) rs = *reinterpret_cast<const f16x8*>(res + off);
    f16x8 o;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const float2 m = mom[0][half * 8 + k];
        const float nv = fmaxf(r16(((float)v[k] - m.x) * m.y), 0.0f);
        if constexpr (MODE == kInRelu) {
            o[k] = (_Float16)nv;
        } else {
            float r = (float)rs[k];
            if constexpr (MODE == kInAddNorm) {
                const float2 m2 = mom[1][half * 8 + k];
                r = r16((r - m2.x) * m2.y);
            }
            o[k] = (_Float16)fmaxf(r16(nv + r), 0.0f);
        }
    }
    *reinterpret_cast<f16x8*>((MODE == kInRelu ? y : out) + off) = o;
}

// The encoder input as [image][h*w][4] fp16 (R, G, B, 0). From the caller's BGR frame (H x W x 3,
// 0..255; preprocess_image_kernel, main.cu:1062-1075: BGR -> RGB, x/255,
// minus the ImageNet mean, over its std, then float_to_half) or from an
// NCHW fp32 3-channel image (float_to_half only, HalfBasicEncoder::forward).
__global__ void k_image_to_px4(const float* src, int from_bgr, long src_nstride, int hw,
                              _Float16* out, long out_nstride) {
    const int p = blockIdx.x * blockDim.x + threadIdx.x, n = blockIdx.y;
    if (p >= hw) return;
    const float* s = src + (long)n * src_nstride;
    float rgb[3];
    if (from_bgr) {
        const float mean[3] = {0.406f, 0.456f, 0.485f};  // B, G, R
        const float sd[3] = {0.225f, 0.224f, 0.229f};
#pragma unroll
        for (int c = 0; c < 3; c++) rgb[2 - c] = (s[(long)p * 3 + c] / 255.0f - mean[c]) / sd[c];
    } else {
#pragma unroll
        for (int c = 0; c < 3; c++) rgb[c] = s[(long)c * hw + p];
    }
    const f16x4 v = {(_Float16)rgb[0], (_Float16)rgb[1], (_Float16)rgb[2], (_Float16)0.0f};
    *reinterpret_cast<f16x4*>(out + (long)n * out_nstride + (long)p * 4) = v;
}

// ---------------------------------------------------------------- host side
constexpr int kEncLayers = 16;
struct EncLayer {
    const char* suffix;
    int co, ci, k, s;  // co of the last layer is the encoder's output_dim
};
constexpr EncLayer kEnc[kEncLayers] = {
    {"conv1", 32, 3, 7, 2},
    {"layer1_0_conv1", 32, 32, 3, 1},          {"layer1_0_conv2", 32, 32, 3, 1},
    {"layer1_1_conv1", 32, 32, 3, 1},          {"layer1_1_conv2", 32, 32, 3, 1},
    {"layer2_0_conv1", 64, 32, 3, 2},          {"layer2_0_conv2", 64, 64, 3, 1},
    {"layer2_0_downsample_0", 64, 32, 1, 2},   {"layer2_1_conv1", 64, 64, 3, 1},
    {"layer2_1_conv2", 64, 64, 3, 1},          {"layer3_0_conv1", 128, 64, 3, 2},
    {"layer3_0_conv2", 128, 128, 3, 1},        {"layer3_0_downsample_0", 128, 64, 1, 2},
    {"layer3_1_conv1", 128, 128, 3, 1},        {"layer3_1_conv2", 128, 128, 3, 1},
    {"conv2", 0, 128, 1, 1},
};
// output-channel tile of a layer with co channels (the kernel's CO_T)
int co_tile(int co) { return co <= 32 ? 32 : co <= 64 ? 64 : 128; }

struct EncPacked {
    int k = 1, s = 1, nchunk = 0, co_pad = 0, Co = 0;
    DevBuf wt, bias;
};

}  // namespace

struct slk_encoder_state {
    int in_h = 0, in_w = 0, out_dim = 0, norm = 0, max_batch = 0;
    std::vector<float> hw_[kEncLayers], hb_[kEncLayers];
    bool have[kEncLayers] = {};
    bool packed = false;
    EncPacked pk[kEncLayers];
    DevBuf img, A, B, T, D, part1, part2;
    // encode_frame runs the context encoder on this stream (non-blocking,
    // default priority) beside the feature encoder on the caller's, forked
    // and joined by the two events; created on the first such call
    hipStream_t side = nullptr;
    hipEvent_t ev_fork = nullptr, ev_join = nullptr;
};

namespace {

int layer_co(const slk_encoder_state& e, int L) { return L == kEncLayers - 1 ? e.out_dim : kEnc[L].co; }

int pack_layer(slk_encoder_state& e, int L) {
    EncPacked& pc = e.pk[L];
    const int co = layer_co(e, L), ci = kEnc[L].ci, k = kEnc[L].k, taps = k * k;
    pc.k = k;
    pc.s = kEnc[L].s;
    pc.Co = co;
    pc.nchunk = (ci + 15) / 16;
    const int cot = co_tile(co);
    pc.co_pad = (co + cot - 1) / cot * cot;
    std::vector<_Float16> w;
    std::vector<float> b(pc.co_pad, 0.0f);
    const std::vector<float>& src = e.hw_[L];
    if (L == 0) {
        // the stem's tap-packed K: [13 steps][32][16], k = 4*(t - 4*step) + c
        w.assign((size_t)13 * 32 * 16, (_Float16)0.0f);
        for (int o = 0; o < co; o++)
            for (int c = 0; c < ci; c++)
                for (int t = 0; t < taps; t++)
                    w[((size_t)(t / 4) * 32 + o) * 16 + 4 * (t % 4) + c] =
                        (_Float16)src[((size_t)o * ci + c) * taps + t];
    } else {
        w.assign((size_t)taps * pc.nchunk * pc.co_pad * 16, (_Float16)0.0f);
        for (int o = 0; o < co; o++)
            for (int c = 0; c < ci; c++)
                for (int t = 0; t < taps; t++)
                    w[(((size_t)t * pc.nchunk + c / 16) * pc.co_pad + o) * 16 + c % 16] =
                        (_Float16)src[((size_t)o * ci + c) * taps + t];
    }
    for (int o = 0; o < co; o++) b[o] = e.hb_[L][o];
    SLK_TRY(pc.wt.ensure(w.size() * sizeof(_Float16)));
    SLK_TRY(pc.bias.ensure(b.size() * sizeof(float)));
    SLK_HIP(hipMemcpy(pc.wt.ptr, w.data(), w.size() * sizeof(_Float16), hipMemcpyHostToDevice));
    SLK_HIP(hipMemcpy(pc.bias.ptr, b.data(), b.size() * sizeof(float), hipMemcpyHostToDevice));
    return SLK_OK;
}

int pack_encoder(slk_encoder_state& e) {
    for (int L = 0; L < kEncLayers; L++) {
        if (!e.have[L])
            return fail(SLK_E_STATE, std::string("encoder: weights of ") + kEnc[L].suffix + " not set");
        SLK_TRY(pack_layer(e, L));
    }
    SLK_HIP(hipDeviceSynchronize());
    e.packed = true;
    return SLK_OK;
}

// an activation: buffer, chunk count, map size and elements per image
// (nch*h*w*16 for a CK tensor; 4*h*w for the [h*w][4] input image)
struct Act {
    _Float16* p;
    int nch, h, w;
    long ns;
};
Act ck_act(_Float16* p, int nch, int h, int w) { return Act{p, nch, h, w, (long)nch * h * w * 16}; }

template <int KS, int S, int WM, int NCH, int EPI>
void launch_cfg(const EncArgs& a, int N, hipStream_t stream) {
    constexpr int TH = 4 / WM, CO_T = WM * 32;
    const int tiles_y = (a.oh + TH - 1) / TH;
    EncArgs b = a;
    b.tiles_x = (a.ow + kTW - 1) / kTW;
    hipLaunchKernelGGL((k_enc_conv<KS, S, WM, NCH, EPI>), dim3(a.co_pad / CO_T, b.tiles_x * tiles_y, N),
                       dim3(256), 0, stream, b);
}

template <int EPI>
int launch_layer(const EncPacked& pc, EncArgs a, int N, hipStream_t stream) {
    a.nchunk = pc.nchunk;
    a.wt = pc.wt.as<_Float16>();
    a.bias = pc.bias.as<float>();
    a.co_pad = pc.co_pad;
    a.Co = pc.Co;
    a.oh = (a.ih + 2 * (pc.k / 2) - pc.k) / pc.s + 1;
    a.ow = (a.iw + 2 * (pc.k / 2) - pc.k) / pc.s + 1;
    const int cot = co_tile(pc.Co);
    // tiles: 32 channels x 4 rows, 64 x 2, 128 x 1 (x 32 columns); NCH covers
    // the layer's input chunks (larger inputs run in groups of NCH)
    if (pc.k == 7 && pc.s == 2 && cot == 32) {
        a.tiles_x = (a.ow + kTW - 1) / kTW;
        hipLaunchKernelGGL((k_enc_stem<EPI>), dim3(1, a.tiles_x * ((a.oh + 3) / 4), N), dim3(256),
                           0, stream, a);
    } else if (cot == 32 && pc.k == 3 && pc.s == 1) launch_cfg<3, 1, 1, 2, EPI>(a, N, stream);
    else if (cot == 64 && pc.k == 3 && pc.s == 2) launch_cfg<3, 2, 2, 2, EPI>(a, N, stream);
    else if (cot == 64 && pc.k == 3 && pc.s == 1) launch_cfg<3, 1, 2, 4, EPI>(a, N, stream);
    else if (cot == 64 && pc.k == 1 && pc.s == 2) launch_cfg<1, 2, 2, 2, EPI>(a, N, stream);
    else if (cot == 128 && pc.k == 3 && pc.s == 2) launch_cfg<3, 2, 4, 4, EPI>(a, N, stream);
    else if (cot == 128 && pc.k == 3 && pc.s == 1) launch_cfg<3, 1, 4, 8, EPI>(a, N, stream);
    else if (cot == 128 && pc.k == 1 && pc.s == 2) launch_cfg<1, 2, 4, 4, EPI>(a, N, stream);
    else if (cot == 128 && pc.k == 1 && pc.s == 1) launch_cfg<1, 1, 4, 8, EPI>(a, N, stream);
    else return fail(SLK_E_ARG, "encoder: no kernel for this layer shape");
    SLK_HIP(hipGetLastError());
    return SLK_OK;
}

// conv of layer L from x into a new activation at `dst`
template <int EPI>
int conv(const slk_encoder_state& e, int L, const Act& x, _Float16* dst, Act* y, int N,
         hipStream_t stream, const Act* res = nullptr) {
    const EncPacked& pc = e.pk[L];
    EncArgs a{};
    a.in = x.p;
    a.in_nstride = x.ns;
    a.ih = x.h;
    a.iw = x.w;
    const int oh = (x.h + 2 * (pc.k / 2) - pc.k) / pc.s + 1;
    const int ow = (x.w + 2 * (pc.k / 2) - pc.k) / pc.s + 1;
    *y = ck_act(dst, (pc.Co + 15) / 16, oh, ow);
    a.out = dst;
    a.out_nstride = y->ns;
    if (res) {
        a.res = res->p;
        a.res_nstride = res->ns;
    }
    return launch_layer<EPI>(pc, a, N, stream);
}

int nsplit_of(int hw) { return (hw + kSplit - 1) / kSplit; }

void in_stats(const Act& y, float2* part, int N, hipStream_t stream) {
    const int hw = y.h * y.w;
    hipLaunchKernelGGL(k_in_stats, dim3(y.nch, nsplit_of(hw), N), dim3(256), 0, stream, y.p,
                       y.ns, hw, y.nch * 16, nsplit_of(hw), part);
}

template <int MODE>
void in_apply(const Act& y, const float2* part, const Act* res, const float2* part2, _Float16* out,
              int N, hipStream_t stream) {
    const int hw = y.h * y.w;
    hipLaunchKernelGGL((k_in_apply<MODE>), dim3((hw + 127) / 128, y.nch, N), dim3(256), 0, stream,
                       y.p, part, res ? res->p : nullptr, part2, out, y.ns, hw, y.nch * 16,
                       nsplit_of(hw));
}

// HalfBasicEncoder::forward from a CK image to the last layer,
// whose epilogue `finish` writes the caller's output.
template <typename Finish>
int encoder_run(slk_encoder_state& e, const _Float16* image, int N, hipStream_t stream,
                Finish finish) {
    float2* p1 = e.part1.as<float2>();
    float2* p2 = e.part2.as<float2>();
    Act img{const_cast<_Float16*>(image), 1, e.in_h, e.in_w, 4L * e.in_h * e.in_w};
    Act x, y, t, d;
    _Float16* bufA = e.A.as<_Float16>();
    _Float16* bufB = e.B.as<_Float16>();
    // conv1 (7x7, stride 2) + norm + relu (main.cu:363-365)
    if (e.norm) {
        SLK_TRY(conv<kEpRaw>(e, 0, img, bufA, &x, N, stream));
        in_stats(x, p1, N, stream);
        in_apply<kInRelu>(x, p1, nullptr, nullptr, nullptr, N, stream);
    } else {
        SLK_TRY(conv<kEpRelu>(e, 0, img, bufA, &x, N, stream));
    }
    // six residual blocks (HalfResBlock::forward, main.cu:268-290)
    for (int blk = 0; blk < 6; blk++) {
        const int c1 = blk == 0 ? 1 : blk == 1 ? 3 : blk == 2 ? 5 : blk == 3 ? 8 : blk == 4 ? 10 : 13;
        const bool ds = blk == 2 || blk == 4;
        _Float16* out = x.p == bufA ? bufB : bufA;
        if (e.norm) {
            SLK_TRY(conv<kEpRaw>(e, c1, x, e.T.as<_Float16>(), &t, N, stream));
            in_stats(t, p1, N, stream);
            in_apply<kInRelu>(t, p1, nullptr, nullptr, nullptr, N, stream);
            if (ds) {
                SLK_TRY(conv<kEpRaw>(e, c1 + 2, x, e.D.as<_Float16>(), &d, N, stream));
                in_stats(d, p2, N, stream);
            }
            SLK_TRY(conv<kEpRaw>(e, c1 + 1, t, out, &y, N, stream));
            in_stats(y, p1, N, stream);
            if (ds)
                in_apply<kInAddNorm>(y, p1, &d, p2, out, N, stream);
            else
                in_apply<kInAddRelu>(y, p1, &x, nullptr, out, N, stream);
        } else {
            SLK_TRY(conv<kEpRelu>(e, c1, x, e.T.as<_Float16>(), &t, N, stream));
            if (ds) SLK_TRY(conv<kEpRaw>(e, c1 + 2, x, e.D.as<_Float16>(), &d, N, stream));
            SLK_TRY(conv<kEpAddRelu>(e, c1 + 1, t, out, &y, N, stream, ds ? &d : &x));
        }
        SLK_HIP(hipGetLastError());
        x = y;
    }
    return finish(x);
}

int check_encoder(slk_encoder_state* e, int batch, const char* what) {
    if (!e) return fail(SLK_E_ARG, std::string(what) + ": null encoder");
    if (batch < 1 || batch > e->max_batch)
        return fail(SLK_E_ARG, std::string(what) + ": batch outside [1, max_batch]");
    if (!e->packed) SLK_TRY(pack_encoder(*e));
    return SLK_OK;
}

}  // namespace
}  // namespace slk

using namespace slk;

struct slk_encoder {
    slk_encoder_state s;
};

extern "C" int slk_encoder_create(slk_encoder** out, int in_h, int in_w, int out_dim, int use_norm,
                                  int max_batch) {
    if (!out) return fail(SLK_E_ARG, "encoder_create: null output");
    *out = nullptr;
    if (in_h < 8 || in_w < 8 || in_h % 8 || in_w % 8 || (long)in_h * in_w > (1L << 24))
        return fail(SLK_E_ARG, "encoder_create: image sides must be multiples of 8, h*w <= 2^24");
    if (out_dim < 16 || out_dim > 256 || out_dim % 16 || max_batch < 1)
        return fail(SLK_E_ARG, "encoder_create: need out_dim a multiple of 16 in [16, 256] and "
                               "max_batch >= 1");
    slk_encoder* enc = new slk_encoder();
    slk_encoder_state& e = enc->s;
    e.in_h = in_h;
    e.in_w = in_w;
    e.out_dim = out_dim;
    e.norm = use_norm ? 1 : 0;
    e.max_batch = max_batch;
    const size_t N = max_batch, hw = (size_t)in_h * in_w, h2 = hw / 4;
    // the largest activation: 32 channels at half resolution (= 64 at a
    // quarter, 128 at an eighth)
    const size_t act = N * 32 * h2 * sizeof(_Float16);
    const size_t parts = N * (size_t)nsplit_of((int)h2) * 128 * sizeof(float2);
    int st = e.img.ensure(N * hw * 4 * sizeof(_Float16));
    for (DevBuf* b : {&e.A, &e.B, &e.T, &e.D})
        if (st == SLK_OK) st = b->ensure(act);
    if (st == SLK_OK) st = e.part1.ensure(parts);
    if (st == SLK_OK) st = e.part2.ensure(parts);
    if (st != SLK_OK) {
        slk_encoder_destroy(enc);
        return st;
    }
    *out = enc;
    return SLK_OK;
}

extern "C" int slk_encoder_destroy(slk_encoder* enc) {
    if (!enc) return SLK_OK;
    slk_encoder_state& e = enc->s;
    for (EncPacked& pc : e.pk) {
        pc.wt.release();
        pc.bias.release();
    }
    for (DevBuf* b : {&e.img, &e.A, &e.B, &e.T, &e.D, &e.part1, &e.part2}) b->release();
    if (e.side) {
        // the side stream's work is finished before its resources go
        (void)hipStreamSynchronize(e.side);
        (void)hipStreamDestroy(e.side);
    }
    if (e.ev_fork) (void)hipEventDestroy(e.ev_fork);
    if (e.ev_join) (void)hipEventDestroy(e.ev_join);
    delete enc;
    return SLK_OK;
}

extern "C" int slk_encoder_num_layers(void) { return kEncLayers; }

extern "C" const char* slk_encoder_layer_suffix(int layer) {
    return layer >= 0 && layer < kEncLayers ? kEnc[layer].suffix : nullptr;
}

extern "C" int slk_encoder_layer_shape(const slk_encoder* enc, int layer, int* co, int* ci, int* k,
                                       int* stride) {
    if (!enc || layer < 0 || layer >= kEncLayers)
        return fail(SLK_E_ARG, "encoder_layer_shape: bad argument");
    if (co) *co = layer_co(enc->s, layer);
    if (ci) *ci = kEnc[layer].ci;
    if (k) *k = kEnc[layer].k;
    if (stride) *stride = kEnc[layer].s;
    return SLK_OK;
}

extern "C" int slk_encoder_set_conv(slk_encoder* enc, int layer, const float* weight_host,
                                    const float* bias_host) {
    if (!enc || layer < 0 || layer >= kEncLayers || !weight_host || !bias_host)
        return fail(SLK_E_ARG, "encoder_set_conv: bad argument");
    slk_encoder_state& e = enc->s;
    const int co = layer_co(e, layer), ci = kEnc[layer].ci, k = kEnc[layer].k;
    e.hw_[layer].assign(weight_host, weight_host + (size_t)co * ci * k * k);
    e.hb_[layer].assign(bias_host, bias_host + co);
    e.have[layer] = true;
    e.packed = false;
    return SLK_OK;
}

extern "C" int slk_encoder_load_dir(slk_encoder* enc, const char* dir, const char* prefix) {
    if (!enc || !dir || !prefix) return fail(SLK_E_ARG, "encoder_load_dir: bad argument");
    for (int L = 0; L < kEncLayers; L++) {
        const int co = layer_co(enc->s, L), ci = kEnc[L].ci, k = kEnc[L].k;
        std::vector<float> wb[2];
        for (int part = 0; part < 2; part++) {
            const std::string path = std::string(dir) + "/" + prefix + "_" + kEnc[L].suffix +
                                     (part ? "_bias.bin" : "_weight.bin");
            FILE* f = std::fopen(path.c_str(), "rb");
            if (!f) return fail(SLK_E_ARG, "encoder_load_dir: cannot open " + path);
            int nd = 0;
            bool ok = std::fread(&nd, sizeof(int), 1, f) == 1 && nd >= 1 && nd <= 4;
            size_t total = 1;
            for (int dd = 0; ok && dd < nd; dd++) {
                int dim = 0;
                ok = std::fread(&dim, sizeof(int), 1, f) == 1 && dim > 0;
                total *= ok ? (size_t)dim : 0;
            }
            const size_t want = part ? (size_t)co : (size_t)co * ci * k * k;
            ok = ok && total == want;
            if (ok) {
                wb[part].resize(total);
                ok = std::fread(wb[part].data(), sizeof(float), total, f) == total;
            }
            std::fclose(f);
            if (!ok) return fail(SLK_E_ARG, "encoder_load_dir: bad tensor file " + path);
        }
        SLK_TRY(slk_encoder_set_conv(enc, L, wb[0].data(), wb[1].data()));
    }
    return SLK_OK;
}

extern "C" int slk_encoder_forward(slk_encoder* enc, const float* input, void* output, int batch,
                                   hipStream_t stream) {
    SLK_TRY(check_encoder(enc ? &enc->s : nullptr, batch, "encoder_forward"));
    if (!input || !output) return fail(SLK_E_ARG, "encoder_forward: null argument");
    slk_encoder_state& e = enc->s;
    const int hw = e.in_h * e.in_w;
    hipLaunchKernelGGL(k_image_to_px4, dim3((hw + 255) / 256, batch), dim3(256), 0, stream, input,
                       0, 3L * hw, hw, e.img.as<_Float16>(), 4L * hw);
    SLK_HIP(hipGetLastError());
    return encoder_run(e, e.img.as<_Float16>(), batch, stream, [&](const Act& x) {
        const EncPacked& pc = e.pk[kEncLayers - 1];
        EncArgs a{};
        a.in = x.p;
        a.in_nstride = x.ns;
        a.ih = x.h;
        a.iw = x.w;
        a.out = static_cast<_Float16*>(output);
        a.out_nstride = (long)pc.Co * x.h * x.w;
        return launch_layer<kEpNchw>(pc, a, batch, stream);
    });
}

extern "C" int slk_encode_frame(slk_encoder* fnet, slk_encoder* cnet, const float* bgr_hwc,
                                void* fmap, float* net, float* inp, hipStream_t stream) {
    SLK_TRY(check_encoder(fnet ? &fnet->s : nullptr, 1, "encode_frame"));
    SLK_TRY(check_encoder(cnet ? &cnet->s : nullptr, 1, "encode_frame"));
    if (!bgr_hwc || !fmap || !net || !inp) return fail(SLK_E_ARG, "encode_frame: null argument");
    slk_encoder_state& f = fnet->s;
    slk_encoder_state& c = cnet->s;
    if (f.in_h != c.in_h || f.in_w != c.in_w || f.out_dim != 128 || c.out_dim != 256)
        return fail(SLK_E_ARG, "encode_frame: need fnet (out 128) and cnet (out 256) of one size");
    const int hw = f.in_h * f.in_w;
    if (!c.side) {
        SLK_HIP(hipStreamCreateWithFlags(&c.side, hipStreamNonBlocking));
        SLK_HIP(hipEventCreateWithFlags(&c.ev_fork, hipEventDisableTiming));
        SLK_HIP(hipEventCreateWithFlags(&c.ev_join, hipEventDisableTiming));
    }
    hipLaunchKernelGGL(k_image_to_px4, dim3((hw + 255) / 256, 1), dim3(256), 0, stream, bgr_hwc, 1,
                       3L * hw, hw, f.img.as<_Float16>(), 4L * hw);
    SLK_HIP(hipGetLastError());
    // both encoders read the one preprocessed image: the context encoder on
    // the side stream once the image is written, the feature encoder on the
    // caller's stream, which then waits for the side stream (the two
    // encoders' launches are latency-bound at one frame and overlap)
    SLK_HIP(hipEventRecord(c.ev_fork, stream));
    SLK_HIP(hipStreamWaitEvent(c.side, c.ev_fork, 0));
    SLK_TRY(encoder_run(f, f.img.as<_Float16>(), 1, stream, [&](const Act& x) {
        const EncPacked& pc = f.pk[kEncLayers - 1];
        EncArgs a{};
        a.in = x.p;
        a.in_nstride = x.ns;
        a.ih = x.h;
        a.iw = x.w;
        a.out = static_cast<_Float16*>(fmap);
        a.out_nstride = 128L * x.h * x.w;
        return launch_layer<kEpNchw>(pc, a, 1, stream);
    }));
    hipStream_t side = c.side;
    SLK_TRY(encoder_run(c, f.img.as<_Float16>(), 1, side, [&](const Act& x) {
        const EncPacked& pc = c.pk[kEncLayers - 1];
        EncArgs a{};
        a.in = x.p;
        a.in_nstride = x.ns;
        a.ih = x.h;
        a.iw = x.w;
        a.net = net;
        a.inp = inp;
        a.ni_nstride = 128L * x.h * x.w;
        return launch_layer<kEpNetInp>(pc, a, 1, side);
    }));
    SLK_HIP(hipEventRecord(c.ev_join, side));
    SLK_HIP(hipStreamWaitEvent(stream, c.ev_join, 0));
    return SLK_OK;
}
