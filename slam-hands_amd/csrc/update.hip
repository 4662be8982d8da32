// The DROID-SLAM update operator for gfx950: UpdateModule::forward with its
// ConvGRU, and UpdateModule::compute_eta (cuda_slam/main.cu:385-667).
//
// Every convolution runs as an implicit GEMM on v_mfma_f32_32x32x16_f16:
// output channels are the GEMM rows, pixels its columns, and K walks
// 16-channel chunks of the input times the kernel taps. The reference's
// convolutions are cuDNN tensor-op convolutions of fp32 tensors
// (CUDNN_TENSOR_OP_MATH, nn.cuh:146): products of operands rounded to a
// 10-bit mantissa, accumulated in fp32. fp16 operands carry the same 10-bit
// mantissa, so weights and activations are rounded to fp16 once and the
// MFMA accumulates in fp32. Every activation the reference rounds to fp16
// (round_to_fp16, nn.cuh:563-569) is stored as fp16 here, so nothing is lost
// by keeping the intermediates in half the bytes.
//
// Activation layout "CK": [image][C/16][h*w][16] fp16: a 16-channel chunk of
// consecutive pixels is contiguous, so a workgroup's input patch of one chunk
// is a few contiguous rows, and every MFMA operand read is 16 bytes.
// Concatenations of the reference (concat4_kernel, nn.cuh:497) are chunk
// ranges of one CK buffer, written in place by their producers.
//
// The GRU's elementwise steps are epilogues of the convolutions that produce
// their inputs: z and r (sigmoid of conv + global term, rounded) and r*net
// in the epilogue of the fused convz|convr GEMM, the gated global pooling
// input in the epilogue of w, q and the state update (1-z) net + z q in the
// epilogue of convq, and the three 128-channel heads of the new state
// (delta_0 | weight_0 | agg_conv1) as one 384-row GEMM.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "lds_dma.hpp"
#include "slk_internal.hpp"

namespace slk {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kTH = 8;    // output rows per workgroup tile
constexpr int kTW = 32;   // output columns per workgroup tile (one MFMA column block)
constexpr int kCoT = 128; // output channels per workgroup tile

__device__ __forceinline__ float r16(float x) { return (float)(_Float16)x; }
__device__ __forceinline__ float sigm(float x) { return 1.0f / (1.0f + expf(-x)); }

// One input source of a convolution: chunks of a CK buffer.
struct CkSrc {
    const _Float16* p;  // chunk 0 of image 0
    int nchunk;         // chunks taken from this source
    long nstride;       // elements between images
};

enum Epi {
    kEpiRelu = 0,   // out16 = round16(relu(conv + b))
    kEpiGate = 1,   // out16 = round16(round16(sigmoid(round16(conv + b))) * net)
    kEpiZR = 2,     // rows < 128: z; rows >= 128: r and out r*net (see below)
    kEpiQ = 3,      // q and the state update
    kEpiHeads = 4,  // rows < 256: out16 = round16(relu(conv + b)); rows >= 256: out32
};

struct ConvArgs {
    CkSrc s0, s1;         // input chunks [0, s0.nchunk) from s0, the rest from s1
    int nchunk;           // input chunks in total
    const _Float16* wt;   // [taps][nchunk][co_tot][16]
    const float* bias;    // [co_tot]
    int co_tot, Co;       // padded / real output channels
    int h, w, tiles_x;
    // epilogue operands (CK buffers are [image][chunks][hw][16] with nstride)
    _Float16* out16;      // kEpiRelu/kEpiGate/kEpiHeads: output chunks
    long out16_nstride;
    _Float16* zbuf;       // kEpiZR: z (8 chunks); kEpiQ: z input
    _Float16* rnet;       // kEpiZR: r * net (8 chunks)
    long zr_nstride;
    _Float16* net16;      // 8 chunks of the state (read by Gate/ZR/Q; Q writes it)
    long net_nstride;
    const float* gterm;   // [image][384] rounded global terms (zg | rg | qg)
    float* out32;         // kEpiQ: the new state; kEpiHeads: agg_conv1, NCHW fp32
    long out32_nstride;
    const _Float16* zero16;  // 16 zero bytes: the source of staged units outside the image
};

// The epilogue of one pixel's two 32-row accumulator blocks: acc0/acc1
// register v holds output channel co0 + mb*32 + 8*(v/4) + v%4 (co0 includes
// the lane's 4*lhi), so each group of four registers is four consecutive
// channels of the CK layout. bias[co] is the channel's bias and, for kEpiZR
// and kEpiQ, gts[co] its global term of image n (the 3x3 kernels stage
// their tile's in LDS). Every memory read of the epilogue is
// issued before its first store, from a clamped channel where the group is
// past Co: vector memory counts loads and stores together, in order, so a
// load issued after a store would wait for that store.
template <int EPI>
__device__ __forceinline__ void epi_block(const ConvArgs& a, const f32x16& acc0,
                                          const f32x16& acc1, int n, int co0, int p, int HW,
                                          const float* bias, const float* gts) {
    // the state operands of each group: s0 (net, or for kEpiQ z), s1 (kEpiQ: net)
    f16x4 s0[2][4], s1[2][4];
#pragma unroll
    for (int mb = 0; mb < 2; mb++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int co = co0 + mb * 32 + 8 * g;
            const int cc = co < a.Co ? co : 0;
            if constexpr (EPI == kEpiGate) {
                s0[mb][g] = *reinterpret_cast<const f16x4*>(
                    a.net16 + (long)n * a.net_nstride + ((long)(cc >> 4) * HW + p) * 16 + (cc & 15));
            } else if constexpr (EPI == kEpiZR) {
                const int cr = cc >= 128 ? cc - 128 : 0;
                s0[mb][g] = *reinterpret_cast<const f16x4*>(
                    a.net16 + (long)n * a.net_nstride + ((long)(cr >> 4) * HW + p) * 16 + (cr & 15));
            } else if constexpr (EPI == kEpiQ) {
                const long off = ((long)(cc >> 4) * HW + p) * 16 + (cc & 15);
                s0[mb][g] = *reinterpret_cast<const f16x4*>(a.zbuf + (long)n * a.zr_nstride + off);
                s1[mb][g] = *reinterpret_cast<const f16x4*>(a.net16 + (long)n * a.net_nstride + off);
            }
        }
#pragma unroll
    for (int mb = 0; mb < 2; mb++) {
        const f32x16& acc = mb ? acc1 : acc0;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int co = co0 + mb * 32 + 8 * g;
            if (co >= a.Co) continue;
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; i++) v[i] = acc[4 * g + i] + bias[co + i];
            if constexpr (EPI == kEpiRelu) {
                f16x4 o;
#pragma unroll
                for (int i = 0; i < 4; i++) o[i] = (_Float16)fmaxf(v[i], 0.0f);
                *reinterpret_cast<f16x4*>(a.out16 + (long)n * a.out16_nstride +
                                          ((long)(co >> 4) * HW + p) * 16 + (co & 15)) = o;
            } else if constexpr (EPI == kEpiGate) {
                const f16x4 nt = s0[mb][g];
                f16x4 o;
#pragma unroll
                for (int i = 0; i < 4; i++) o[i] = (_Float16)(r16(sigm(r16(v[i]))) * (float)nt[i]);
                *reinterpret_cast<f16x4*>(a.out16 + (long)n * a.out16_nstride +
                                          ((long)(co >> 4) * HW + p) * 16 + (co & 15)) = o;
            } else if constexpr (EPI == kEpiZR) {
                f16x4 sg;
#pragma unroll
                for (int i = 0; i < 4; i++) sg[i] = (_Float16)sigm(r16(v[i]) + gts[co + i]);
                if (co < 128) {
                    *reinterpret_cast<f16x4*>(a.zbuf + (long)n * a.zr_nstride +
                                              ((long)(co >> 4) * HW + p) * 16 + (co & 15)) = sg;
                } else {
                    const int cr = co - 128;
                    const long off = ((long)(cr >> 4) * HW + p) * 16 + (cr & 15);
                    const f16x4 nt = s0[mb][g];
                    f16x4 o;
#pragma unroll
                    for (int i = 0; i < 4; i++) o[i] = (_Float16)((float)nt[i] * (float)sg[i]);
                    *reinterpret_cast<f16x4*>(a.rnet + (long)n * a.zr_nstride + off) = o;
                }
            } else if constexpr (EPI == kEpiQ) {
                const long off = ((long)(co >> 4) * HW + p) * 16 + (co & 15);
                const f16x4 z = s0[mb][g], nt = s1[mb][g];
                f16x4 o;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float q = r16(tanhf(r16(v[i]) + gts[co + i]));
                    const float zi = (float)z[i];
                    const float nn = (1.0f - zi) * (float)nt[i] + zi * q;
                    o[i] = (_Float16)nn;
                    a.out32[(long)n * a.out32_nstride + (long)(co + i) * HW + p] = (float)o[i];
                }
                *reinterpret_cast<f16x4*>(a.net16 + (long)n * a.net_nstride + off) = o;
            } else {  // kEpiHeads
                if (co < 256) {
                    f16x4 o;
#pragma unroll
                    for (int i = 0; i < 4; i++) o[i] = (_Float16)fmaxf(v[i], 0.0f);
                    *reinterpret_cast<f16x4*>(a.out16 + (long)n * a.out16_nstride +
                                              ((long)(co >> 4) * HW + p) * 16 + (co & 15)) = o;
                } else {
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        a.out32[(long)n * a.out32_nstride + (long)(co - 256 + i) * HW + p] =
                            r16(fmaxf(v[i], 0.0f));
                }
            }
        }
    }
}

// 1x1 convolutions as a plain GEMM with register-direct operands (no halo,
// so nothing is staged in LDS): tile kCoT output channels x 256 consecutive
// pixels, wave (wm, wn) = 64 channels x 128 pixels; every lane loads its
// 16-byte A (weights) and B (8 channels of one pixel) fragments straight from
// global memory, two chunks ahead of their MFMAs.
template <int EPI>
__global__ __launch_bounds__(256) void k_conv1x1(ConvArgs a) {
    __shared__ float bsh[kCoT];  // the tile's biases
    const int HW = a.h * a.w;
    const int cot = blockIdx.x, n = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63;
    if (tid < kCoT) bsh[tid] = a.bias[cot * kCoT + tid];
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave & 1, wn = wave >> 1;
    const int l32 = lane & 31, lhi = lane >> 5;
    const int p0 = blockIdx.y * 256 + wn * 128;
    const _Float16* wbase = a.wt + ((long)cot * kCoT + wm * 64 + l32) * 16 + lhi * 8;
    f16x8 A[3][2], B[3][4];
    // every load unconditional, from a clamped chunk and pixel (a chunk past
    // the last goes to a slot no step multiplies; a pixel past the map only
    // reaches accumulator columns never stored), so the waits count loads
    // along one straight path and the next two chunks stay in flight
    auto load = [&](int c, int slot) {
        c = min(c, a.nchunk - 1);
        const _Float16* wc = wbase + (long)c * a.co_tot * 16;
        A[slot][0] = *reinterpret_cast<const f16x8*>(wc);
        A[slot][1] = *reinterpret_cast<const f16x8*>(wc + 32 * 16);
        const bool first = c < a.s0.nchunk;  // uniform
        const _Float16* sp = first ? a.s0.p + (long)n * a.s0.nstride + (long)c * HW * 16
                                   : a.s1.p + (long)n * a.s1.nstride +
                                         (long)(c - a.s0.nchunk) * HW * 16;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int p = min(p0 + r * 32 + l32, HW - 1);
            B[slot][r] = *reinterpret_cast<const f16x8*>(sp + (long)p * 16 + lhi * 8);
        }
    };
    f32x16 acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = f32x16{};
    // three register slots, so every slot index below is a compile-time constant
    auto step = [&](int c, int slot) {
        load(c + 2, slot == 0 ? 2 : slot - 1);
        if (c < a.nchunk) {  // uniform
#pragma unroll
            for (int r = 0; r < 4; r++) {
                acc[0][r] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[slot][0], B[slot][r],
                                                                   acc[0][r], 0, 0, 0);
                acc[1][r] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[slot][1], B[slot][r],
                                                                   acc[1][r], 0, 0, 0);
            }
        }
    };
    load(0, 0);
    load(1, 1);
    for (int c = 0; c < a.nchunk; c += 3) {
        step(c, 0);
        step(c + 1, 1);
        step(c + 2, 2);
    }
    __syncthreads();  // bsh
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int p = p0 + r * 32 + l32;
        if (p < HW)
            epi_block<EPI>(a, acc[0][r], acc[1][r], n, cot * kCoT + wm * 64 + 4 * lhi, p, HW,
                           bsh - cot * kCoT, nullptr);
    }
}

// The flow encoder's 7x7 stem (4 input channels) with its taps packed into
// K: K step ks covers taps 4 ks .. 4 ks + 3 with their 4 channels (k =
// 4 (t - 4 ks) + c), 13 steps for the 49 taps (taps 49..51 have zero
// weights), where a chunked K would take 49 steps of 16 channels, 12 of them
// zero. One conv tile: kCoT output channels x (kTH x kTW) pixels of one image,
// four waves, wave (wm, wn) taking 64 channels (two 32-row MFMA blocks) of
// image rows wn*4 .. wn*4+3 (four 32-pixel column blocks); the patch holds
// each pixel's 4 channels (8 bytes), and lane (l32, lhi) reads two patch
// pixels per K step, those of
// taps 4 ks + 2 lhi and 4 ks + 2 lhi + 1. The tile's weights of all 13 K
// steps ([13][co_tot][16] in memory, 52 KB) are staged in LDS by
// direct-to-LDS loads beside the patch's loads, every 32-byte row's halves
// swapped when bit 3 of its channel is set (as in k_conv3).
template <int EPI>
__global__ __launch_bounds__(256, 2) void k_conv7p(ConvArgs a) {
    constexpr int KS = 7, P = 3, KSTEPS = 13;
    constexpr int PH = kTH + KS - 1, PW = kTW + KS - 1;
    constexpr int UNITS = PH * PW;  // 8-byte pixels of the patch
    constexpr int UPT = (UNITS + 255) / 256;
    __shared__ __attribute__((aligned(16))) _Float16 patch[UNITS * 4];
    __shared__ __attribute__((aligned(16))) _Float16 wsh[KSTEPS * kCoT * 16];
    __shared__ float bsh[kCoT];  // the tile's biases
    const int HW = a.h * a.w;
    const int cot = blockIdx.x, tile = blockIdx.y, n = blockIdx.z;
    const int ty0 = (tile / a.tiles_x) * kTH, tx0 = (tile % a.tiles_x) * kTW;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave & 1, wn = wave >> 1;
    const int l32 = lane & 31, lhi = lane >> 5;
    // the weights: 16-byte unit u = 256 r + tid is physical half u & 1 of row
    // u / 2 = (ks, co); the thread loads the logical half that lands there
#pragma unroll
    for (int r = 0; r < KSTEPS; r++) {
        const int unit = r * 256 + tid, row = unit >> 1;
        const int ks = row / kCoT, co = row - (row / kCoT) * kCoT;
        const int half = (unit & 1) ^ ((co >> 3) & 1);
        dma_x4(a.wt + ((long)ks * a.co_tot + cot * kCoT + co) * 16 + half * 8,
               lds_addr(&wsh[(r * 256 + wave * 64) * 8]));
    }
    if (tid < kCoT) bsh[tid] = a.bias[cot * kCoT + tid];
    // channels 0..3 of chunk 0 of the input
    const _Float16* img = a.s0.p + (long)n * a.s0.nstride;
    f16x4 reg[UPT];
#pragma unroll
    for (int u = 0; u < UPT; u++) {
        const int pix = tid + 256 * u;
        const int py = pix / PW, px = pix - (pix / PW) * PW;
        const int y = ty0 - P + py, x = tx0 - P + px;
        f16x4 v = {};
        if (pix < UNITS && y >= 0 && y < a.h && x >= 0 && x < a.w)
            v = *reinterpret_cast<const f16x4*>(img + ((long)y * a.w + x) * 16);
        reg[u] = v;
    }
#pragma unroll
    for (int u = 0; u < UPT; u++) {
        const int pix = tid + 256 * u;
        if (pix < UNITS) *reinterpret_cast<f16x4*>(&patch[pix * 4]) = reg[u];
    }
    __builtin_amdgcn_s_waitcnt(kWaitVm0Lgkm0);  // the weights' direct-to-LDS loads
    __syncthreads();
    f32x16 acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = f32x16{};
    // A rows co = wm*64 + mb*32 + l32 (bit 3 of co is bit 3 of l32)
    const int aoff = ((wm * 64 + l32) * 2 + (lhi ^ ((l32 >> 3) & 1))) * 8;
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ks++) {
        const f16x8 a0 = *reinterpret_cast<const f16x8*>(&wsh[ks * kCoT * 16 + aoff]);
        const f16x8 a1 = *reinterpret_cast<const f16x8*>(&wsh[ks * kCoT * 16 + aoff + 32 * 16]);
        // (taps past 48 have zero weights; their reads stay in the patch)
        const int t0 = min(4 * ks + 2 * lhi, 48), t1 = min(4 * ks + 2 * lhi + 1, 48);
        const int ky0 = t0 / KS, kx0 = t0 - ky0 * KS, ky1 = t1 / KS, kx1 = t1 - ky1 * KS;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int prow = wn * 4 + r;
            const f16x4 b0 = *reinterpret_cast<const f16x4*>(&patch[((prow + ky0) * PW + l32 + kx0) * 4]);
            const f16x4 b1 = *reinterpret_cast<const f16x4*>(&patch[((prow + ky1) * PW + l32 + kx1) * 4]);
            const f16x8 b = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
            acc[0][r] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, b, acc[0][r], 0, 0, 0);
            acc[1][r] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, b, acc[1][r], 0, 0, 0);
        }
    }
    const int x = tx0 + l32;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int y = ty0 + wn * 4 + r;
        if (y >= a.h || x >= a.w) continue;
        epi_block<EPI>(a, acc[0][r], acc[1][r], n, cot * kCoT + wm * 64 + 4 * lhi, y * a.w + x,
                       HW, bsh - cot * kCoT, nullptr);
    }
}

// The 3x3 convolutions: the tile of k_conv7p (kCoT output channels x kTH x kTW
// pixels, four waves, wave (wm, wn) = 64 channels x image rows wn*4..+3), with
// both operands staged in LDS by direct-to-LDS loads, so that the four waves
// share one copy of the weights. Per input chunk c: the (kTH + 2) x (kTW + 2) patch (double
// buffered), and the weights of taps 0-4 (WA) and 5-8 (WB) of the tile's
// kCoT channels, one buffer each: WB(c) and the patch of chunk c + 1 are
// loaded after the barrier that starts chunk c, WA(c + 1) after the barrier
// between its taps 4 and 5, so each half has about half a chunk of MFMAs to
// land. 60 KB of LDS: two workgroups a CU. Every staged 32-byte row (a pixel
// of the patch, an output channel of the weights) has its two 16-byte halves
// swapped when bit 3 of the row is set, so the 16 lanes of one pass of a
// 128-bit operand read touch 64 distinct banks.
constexpr int kTH3 = 6;            // output rows of a k_conv3 tile
constexpr int kPatchUnits = 768;  // 16-byte units of a patch buffer: (kTH + 2) x (kTW + 2) x 2 = 680, padded
constexpr int kWaTaps = 5, kWbTaps = 4;
static_assert(kPatchUnits >= (kTH + 2) * (kTW + 2) * 2 && kPatchUnits % 256 == 0, "patch units");
static_assert(kCoT * 2 == 256, "one 256-unit round per weight tap");

template <int EPI, int TH>
__global__ __launch_bounds__(256, 2) void k_conv3(ConvArgs a) {
    constexpr int PW = kTW + 2;
    constexpr int RW = TH / 2;  // output rows of a wave
    static_assert(TH % 2 == 0 && (TH + 2) * PW * 2 <= kPatchUnits, "conv3 tile height");
    __shared__ __attribute__((aligned(16))) _Float16 sp[2][kPatchUnits * 8];
    __shared__ __attribute__((aligned(16))) _Float16 swa[kWaTaps * 256 * 8];
    __shared__ __attribute__((aligned(16))) _Float16 swb[kWbTaps * 256 * 8];
    // the tile's biases and (kEpiZR, kEpiQ) global terms, in LDS by the first
    // chunk's barrier
    __shared__ float bsh[kCoT], gsh[kCoT];
    const int HW = a.h * a.w;
    const int cot = blockIdx.x, tile = blockIdx.y, n = blockIdx.z;
    const int ty0 = (tile / a.tiles_x) * TH, tx0 = (tile % a.tiles_x) * kTW;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave & 1, wn = wave >> 1;
    const int l32 = lane & 31, lhi = lane >> 5;
    const int nch = a.nchunk;
    const long tap_stride = (long)nch * a.co_tot * 16;
    // weight unit tid of a tap: output channel co = tid / 2, physical half tid & 1
    const int wco = tid >> 1;
    const int whalf = (tid & 1) ^ ((wco >> 3) & 1);
    const _Float16* wsrc = a.wt + ((long)cot * kCoT + wco) * 16 + whalf * 8;
    auto issue_w = [&](int c, int t0, int ntaps, _Float16* dst) {
        for (int t = 0; t < ntaps; t++)  // uniform
            dma_x4(wsrc + (long)(t0 + t) * tap_stride + (long)c * a.co_tot * 16,
                   lds_addr(dst + (t * 256 + wave * 64) * 8));
    };
    auto issue_patch = [&](int c, int buf) {
        const bool first = c < a.s0.nchunk;
        const CkSrc& s = first ? a.s0 : a.s1;
        const int cc = first ? c : c - a.s0.nchunk;
        const _Float16* base = s.p + (long)n * s.nstride + (long)cc * HW * 16;
#pragma unroll
        for (int r = 0; r < kPatchUnits / 256; r++) {
            const int unit = r * 256 + tid;
            const int pix = unit >> 1;
            const int half = (unit & 1) ^ ((pix >> 3) & 1);
            const int py = pix / PW, px = pix - (pix / PW) * PW;
            const int y = ty0 - 1 + py, x = tx0 - 1 + px;
            const bool ok = pix < (TH + 2) * PW && y >= 0 && y < a.h && x >= 0 && x < a.w;
            dma_x4(ok ? base + ((long)y * a.w + x) * 16 + half * 8 : a.zero16,
                   lds_addr(&sp[buf][(r * 256 + wave * 64) * 8]));
        }
    };

    f32x16 acc[2][RW];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < RW; j++) acc[i][j] = f32x16{};
    auto taps = [&](int t0, int nt, const _Float16* wb, const _Float16* pb) {
#pragma unroll
        for (int tt = 0; tt < nt; tt++) {  // the callers' counts are constants
            const int t = t0 + tt, ky = t / 3, kx = t - (t / 3) * 3;
            f16x8 av[2];
#pragma unroll
            for (int mb = 0; mb < 2; mb++) {
                const int co = wm * 64 + mb * 32 + l32;
                av[mb] = *reinterpret_cast<const f16x8*>(
                    wb + ((tt * 256 + co * 2) * 8 + ((lhi ^ ((co >> 3) & 1)) * 8)));
            }
#pragma unroll
            for (int r = 0; r < RW; r++) {
                const int pix = (wn * RW + r + ky) * PW + l32 + kx;
                const f16x8 b = *reinterpret_cast<const f16x8*>(
                    pb + (pix * 16 + ((lhi ^ ((pix >> 3) & 1)) * 8)));
                acc[0][r] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[0], b, acc[0][r], 0, 0, 0);
                acc[1][r] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[1], b, acc[1][r], 0, 0, 0);
            }
        }
    };
    // Issue order (every thread the same count of loads): P(0) WA(0) | WB(0)
    // P(1) | WA(1) | WB(1) P(2) | WA(2) ...; a chunk starts once everything
    // issued before it has landed (its patch and WA), its taps 5-8 once WB
    // has (only the next patch, 3 loads, may still be in flight).
    if (tid < kCoT) bsh[tid] = a.bias[cot * kCoT + tid];
    if constexpr (EPI == kEpiZR || EPI == kEpiQ)
        if (tid < kCoT) gsh[tid] = a.gterm[(long)n * 384 + (EPI == kEpiQ ? 256 : 0) + cot * kCoT + tid];
    issue_patch(0, 0);
    issue_w(0, 0, kWaTaps, swa);
    for (int c = 0; c < nch; c++) {
        __builtin_amdgcn_s_waitcnt(kWaitVm0Lgkm0);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_barrier();  // P(c), WA(c) in; every wave done with chunk c - 1
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        issue_w(c, kWaTaps, kWbTaps, swb);
        const bool more = c + 1 < nch;  // uniform
        if (more) issue_patch(c + 1, (c + 1) & 1);
        taps(0, kWaTaps, swa, &sp[c & 1][0]);
        if (more)
            __builtin_amdgcn_s_waitcnt(kWaitVm0Lgkm0 | (kPatchUnits / 256));
        else
            __builtin_amdgcn_s_waitcnt(kWaitVm0Lgkm0);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_barrier();  // WB(c) in; every wave done with WA(c)
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        if (more) issue_w(c + 1, 0, kWaTaps, swa);
        taps(kWaTaps, kWbTaps, swb, &sp[c & 1][0]);
    }

    const int x = tx0 + l32;
#pragma unroll
    for (int r = 0; r < RW; r++) {
        const int y = ty0 + wn * RW + r;
        if (y >= a.h || x >= a.w) continue;
        epi_block<EPI>(a, acc[0][r], acc[1][r], n, cot * kCoT + wm * 64 + 4 * lhi, y * a.w + x,
                       HW, bsh - cot * kCoT, gsh - cot * kCoT);
    }
}

// NCHW fp32 [image][C][hw] -> CK fp16 chunks [c0 ..) of out; channels past C
// up to the chunk boundary are zero. kWB: the rounded values also replace
// the fp32 source (round_to_fp16 in place, nn.cuh:563-569). The 16 loads of
// a thread are unconditional (channels past C read channel C - 1 and are
// zeroed after), so they are all in flight together.
template <bool kWB>
__global__ __launch_bounds__(256) void k_to_ck(const float* in, long in_nstride, int C,
                                               _Float16* out, long out_nstride, int c0, int hw,
                                               float* writeback) {
    const int n = blockIdx.z, ch = blockIdx.y;  // chunk index within the source
    const int p = blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= hw) return;
    const long base = (long)n * in_nstride + p;
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; i++) x[i] = in[base + (long)min(ch * 16 + i, C - 1) * hw];
    alignas(16) _Float16 v[16];
#pragma unroll
    for (int i = 0; i < 16; i++) v[i] = (_Float16)(ch * 16 + i < C ? x[i] : 0.0f);
    if constexpr (kWB) {
#pragma unroll
        for (int i = 0; i < 16; i++)
            if (ch * 16 + i < C) writeback[base + (long)(ch * 16 + i) * hw] = (float)v[i];
    }
    _Float16* o = out + (long)n * out_nstride + ((long)(c0 + ch) * hw + p) * 16;
    *reinterpret_cast<f16x8*>(o) = *reinterpret_cast<f16x8*>(&v[0]);
    *reinterpret_cast<f16x8*>(o + 8) = *reinterpret_cast<f16x8*>(&v[8]);
}

// global_avg_pool_kernel (nn.cuh:414-431) of the gated state: glo[n][c] =
// sum_p gate[n][c][p] / hw in fp32, one workgroup per (image, chunk), a
// fixed-order tree over the threads.
__global__ __launch_bounds__(256) void k_gate_pool(const _Float16* gate, long nstride, int hw,
                                                   float* glo) {
    __shared__ float red[256][17];
    const int n = blockIdx.y, ch = blockIdx.x;
    const _Float16* g = gate + (long)n * nstride + (long)ch * hw * 16;
    float s[16] = {};
    for (int p = threadIdx.x; p < hw; p += 256) {
        const f16x8 a = *reinterpret_cast<const f16x8*>(g + (long)p * 16);
        const f16x8 b = *reinterpret_cast<const f16x8*>(g + (long)p * 16 + 8);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            s[i] += (float)a[i];
            s[8 + i] += (float)b[i];
        }
    }
#pragma unroll
    for (int i = 0; i < 16; i++) red[threadIdx.x][i] = s[i];
    __syncthreads();
    for (int st = 128; st > 0; st >>= 1) {
        if (threadIdx.x < st)
#pragma unroll
            for (int i = 0; i < 16; i++) red[threadIdx.x][i] += red[threadIdx.x + st][i];
        __syncthreads();
    }
    if (threadIdx.x < 16) glo[(long)n * 128 + ch * 16 + threadIdx.x] = red[0][threadIdx.x] / (float)hw;
}

// The three 1x1 global convolutions of the pooled vector (convz_glo,
// convr_glo, convq_glo, main.cu:492-523): gterm[n][j] = round16(W[j] .
// round16(glo[n]) + b[j]) for j in 0..383, W and b stacked z | r | q.
__global__ __launch_bounds__(384) void k_glo_fc(const float* glo, const float* W, const float* b,
                                                float* gterm) {
    __shared__ float gs[128];
    const int n = blockIdx.x, j = threadIdx.x;
    if (j < 128) gs[j] = r16(glo[(long)n * 128 + j]);
    __syncthreads();
    float s = 0.0f;
    for (int c = 0; c < 128; c++) s += W[(long)j * 128 + c] * gs[c];
    gterm[(long)n * 384 + j] = r16(s + b[j]);
}

// 3x3 convolutions to at most 3 output channels (delta_2, weight_2,
// agg_eta_0) on 8 input chunks, a kTH x kTW pixel tile per workgroup: the
// tile's (kTH + 2) x (kTW + 2) patch of each chunk staged in LDS (double
// buffered through registers). The taps go into M: for 32 patch pixels a
// v_mfma_f32_32x32x16_f16 forms D[t * 3 + o][q] = W[o][.][t] . x[.][q] for
// all 27 (tap, output) rows at once, summed over the chunks in fp32; D goes
// through LDS and each output pixel adds its 9 taps' rows at the shifted
// patch pixels (weights rounded to fp16 on upload, laid out
// [o][chunk][tap][16]).
// mode 0: round16(conv + b) (delta, main.cu:634-635); 1: round16(sigmoid(
// conv + b)) (weight, :641-643); 2: 0.01 * softplus(round16(conv + b)) (eta,
// :663-665). blockIdx.y = image * nheads + head: head h reads chunks
// [8h, 8h + 8) of `in`, weights W + h * wstride and writes out + h * ostride.
struct SmallArgs {
    const _Float16* in;
    long in_nstride;
    const float* W;
    const float* b;
    long wstride;  // floats between the heads' weight blocks (Co * 8 * 9 * 16)
    int Co, h, w, tiles_x, nheads;
    int mode[2];
    float* out[2];
    long out_nstride;
};
__global__ __launch_bounds__(256) void k_conv_small(SmallArgs a) {
    constexpr int PH = kTH + 2, PW = kTW + 2;
    constexpr int NPIX = PH * PW;                 // 340 patch pixels
    constexpr int NB = (NPIX + 31) / 32;          // 11 blocks of 32 patch pixels
    constexpr int UNITS = NPIX * 2;               // 16-byte units of a chunk's patch
    constexpr int UPT = (UNITS + 255) / 256;
    constexpr int NM = 27;                        // rows of D: tap * 3 + output channel
    constexpr int PBUF = NB * 32 * 16;            // halves of one patch buffer (352 pixels)
    // the patch (double-buffered) and A, then D over both
    struct Stage {
        _Float16 patch[2][PBUF];
        _Float16 A[8][32 * 16];  // [chunk][row m][k], rows past the taps' outputs zero
    };
    constexpr int kSmem = sizeof(Stage) > NM * NB * 32 * 4 ? sizeof(Stage) : NM * NB * 32 * 4;
    __shared__ __attribute__((aligned(16))) unsigned char smem[kSmem];
    Stage& st = *reinterpret_cast<Stage*>(smem);
    float* D = reinterpret_cast<float*>(smem);  // [NM][NB * 32], after the chunk loop
    const int n = blockIdx.z, head = blockIdx.y, tile = blockIdx.x;
    const int ty0 = (tile / a.tiles_x) * kTH, tx0 = (tile % a.tiles_x) * kTW;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int Co = a.Co, hw = a.h * a.w;
    // A of every chunk: row m = t * 3 + o holds W[o][chunk][t][0..15] (fp16),
    // zero for o >= Co and m >= 27; 16 values a thread, loads unconditional
    {
        const float* W = a.W + head * a.wstride;
        float wv[16];
#pragma unroll
        for (int u = 0; u < 16; u++) {
            const int i = tid + 256 * u;  // (chunk, m, k)
            const int ch = i >> 9, m = (i >> 4) & 31, k = i & 15;
            const int t = min(m / 3, 8), o = min(m % 3, Co - 1);
            wv[u] = W[((o * 8 + ch) * 9 + t) * 16 + k];
        }
#pragma unroll
        for (int u = 0; u < 16; u++) {
            const int i = tid + 256 * u;
            const int m = (i >> 4) & 31;
            const bool live = m < NM && m % 3 < Co;
            (&st.A[0][0])[i] = (_Float16)(live ? wv[u] : 0.0f);
        }
    }
    const _Float16* base = a.in + (long)n * a.in_nstride + (long)head * 8 * hw * 16;
    // chunk ch's patch units in register slot ch % 3, loaded two chunks ahead,
    // every load unconditional (a pixel clamped into the image; units
    // outside it zeroed when stored)
    f16x8 reg[3][UPT];
    auto load_chunk = [&](int ch, int slot) {
#pragma unroll
        for (int u = 0; u < UPT; u++) {
            const int unit = tid + 256 * u;
            const int pix = min(unit >> 1, NPIX - 1), half = unit & 1;
            const int yy = ty0 - 1 + pix / PW, xx = tx0 - 1 + pix % PW;
            const int yc = min(max(yy, 0), a.h - 1), xc = min(max(xx, 0), a.w - 1);
            reg[slot][u] = *reinterpret_cast<const f16x8*>(
                base + ((long)ch * hw + yc * a.w + xc) * 16 + half * 8);
        }
    };
    auto store_chunk = [&](int buf, int slot) {
#pragma unroll
        for (int u = 0; u < UPT; u++) {
            const int unit = tid + 256 * u;
            const int pix = unit >> 1;
            const int yy = ty0 - 1 + pix / PW, xx = tx0 - 1 + pix % PW;
            const bool in = unit < UNITS && yy >= 0 && yy < a.h && xx >= 0 && xx < a.w;
            // units up to the 11th block's end are written (zeros past the patch)
            if (unit < NB * 32 * 2)
                *reinterpret_cast<f16x8*>(&st.patch[buf][unit * 8]) = in ? reg[slot][u] : f16x8{};
        }
    };
    static_assert(UPT * 256 >= NB * 32 * 2, "the zero units past the patch are stored");
    // D[m][q] = sum over channels of A[m] . patch[q] on v_mfma_f32_32x32x16_f16:
    // wave w takes blocks w, w + 4, w + 8 of 32 patch pixels; lane l holds A
    // row l % 32 and B column (pixel) l % 32, k = 8 (l / 32) .. + 7
    constexpr int kBpw = (NB + 3) / 4;
    f32x16 acc[kBpw];
#pragma unroll
    for (int i = 0; i < kBpw; i++) acc[i] = f32x16{};
    const int l32 = lane & 31, khalf = lane >> 5;
    load_chunk(0, 0);
    load_chunk(1, 1);
    store_chunk(0, 0);
    __syncthreads();  // A and the first patch
    auto step = [&](int ch, int slot) {
        load_chunk(min(ch + 2, 7), slot == 0 ? 2 : slot - 1);
        const int buf = ch & 1;
        const f16x8 av = *reinterpret_cast<const f16x8*>(&st.A[ch][l32 * 16 + khalf * 8]);
#pragma unroll
        for (int i = 0; i < kBpw; i++) {
            const int blk = wave + 4 * i;
            if (blk < NB) {  // uniform
                const f16x8 bv = *reinterpret_cast<const f16x8*>(
                    &st.patch[buf][(blk * 32 + l32) * 16 + khalf * 8]);
                acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bv, acc[i], 0, 0, 0);
            }
        }
        if (ch + 1 < 8) store_chunk(buf ^ 1, slot == 2 ? 0 : slot + 1);
        __syncthreads();
    };
#pragma unroll
    for (int ch = 0; ch < 8; ch++) step(ch, ch % 3);
    // D to LDS (over the patch buffers, every wave past the last barrier):
    // register v of a block holds row 8 (v / 4) + 4 khalf + v % 4, column l32
#pragma unroll
    for (int i = 0; i < kBpw; i++) {
        const int blk = wave + 4 * i;
        if (blk >= NB) continue;
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int m = 8 * (v >> 2) + 4 * khalf + (v & 3);
            if (m < NM) D[m * (NB * 32) + blk * 32 + l32] = acc[i][v];
        }
    }
    __syncthreads();
    // one thread per output pixel: out[o] = sum over taps of D[t * 3 + o] at
    // the tap's patch pixel
    const int r = tid >> 5, c = tid & 31;
    const int y = ty0 + r, x = tx0 + c;
    if (y >= a.h || x >= a.w) return;
    const int p = y * a.w + x;
    const int mode = a.mode[head];
    float* out = a.out[head] + (long)n * a.out_nstride;
#pragma unroll
    for (int o = 0; o < 3; o++) {
        if (o >= Co) break;
        float sum = 0.0f;
#pragma unroll
        for (int t = 0; t < 9; t++) {
            const int q = (r + t / 3) * PW + c + t % 3;
            sum += D[(t * 3 + o) * (NB * 32) + q];
        }
        const float v = sum + a.b[head * 3 + o];
        float res;
        if (mode == 0) res = r16(v);
        else if (mode == 1) res = r16(sigm(v));
        else res = 0.01f * logf(1.0f + expf(r16(v)));
        out[(long)o * hw + p] = res;
    }
}

// ---------------------------------------------------------------- host side
constexpr int kNumLayers = 18;
struct LayerShape {
    const char* name;
    int co, ci, k;
};
constexpr LayerShape kLayers[kNumLayers] = {
    {"update_corr_encoder_0", 128, 196, 1}, {"update_corr_encoder_2", 128, 128, 3},
    {"update_flow_encoder_0", 128, 4, 7},   {"update_flow_encoder_2", 64, 128, 3},
    {"update_gru_convz", 128, 448, 3},      {"update_gru_convr", 128, 448, 3},
    {"update_gru_convq", 128, 448, 3},      {"update_gru_convz_glo", 128, 128, 1},
    {"update_gru_convr_glo", 128, 128, 1},  {"update_gru_convq_glo", 128, 128, 1},
    {"update_gru_w", 128, 128, 1},          {"update_weight_0", 128, 128, 3},
    {"update_weight_2", 3, 128, 3},         {"update_delta_0", 128, 128, 3},
    {"update_delta_2", 3, 128, 3},          {"update_agg_conv1", 128, 128, 3},
    {"update_agg_conv2", 128, 128, 3},      {"update_agg_eta_0", 1, 128, 3},
};
enum {
    L_CE0, L_CE2, L_FE0, L_FE2, L_Z, L_R, L_Q, L_ZG, L_RG, L_QG, L_W, L_WT0, L_WT2, L_DL0,
    L_DL2, L_AG1, L_AG2, L_ETA
};

// A packed GEMM operand: [taps][nchunk][co_tot][16] fp16 + bias [co_tot].
struct PackedConv {
    int k = 1, nchunk = 0, co_tot = 0, Co = 0;
    DevBuf wt, bias;
};

float round_half_host(float x) {
    // round to nearest even fp16 and back, on the host
    _Float16 h = (_Float16)x;
    return (float)h;
}

}  // namespace

struct UpdateState {
    int max_batch = 0, h = 0, w = 0;
    std::vector<float> hw_[kNumLayers], hb_[kNumLayers];  // host copies, reference layout
    bool have[kNumLayers] = {};
    bool packed = false;
    PackedConv ce0, ce2, fe0, fe2, gw, zr, q, heads, ag2;
    DevBuf glo_w, glo_b, small_w[3], small_b[3];  // [0]: delta_2 | weight_2, [2]: eta_0
    // activations (CK fp16) and small vectors
    DevBuf corr16, mot16, cat, tmp, zr_buf, glo, gterm, agg16, agg_t;
    DevBuf tmp_f, tmp_g;  // the flow encoder's and the gate's first-layer outputs
    DevBuf zero16;  // 256 zero bytes (staged units outside the image)
    // forward runs the flow encoder on side[0] and the gate on side[1]
    // (non-blocking, default priority) beside the correlation encoder on the
    // caller's stream: forked by ev_fork, joined by ev_join before convz|convr
    hipStream_t side[2] = {nullptr, nullptr};
    hipEvent_t ev_fork = nullptr, ev_join[2] = {nullptr, nullptr};
    // motion filter (batch 1): grid coords, lookup, motion, state copies, heads
    DevBuf mf_coords, mf_corr, mf_motion, mf_net, mf_inp, mf_delta, mf_weight, mf_agg;
    std::vector<float> mf_host;
    int tiles_x = 0, tiles_y = 0;
};

namespace {

int pack(PackedConv& pc, const UpdateState* s, std::initializer_list<int> layers) {
    // all listed layers share k and ci; their output rows are stacked
    int co = 0, ci = 0, k = 0;
    for (int L : layers) {
        co += kLayers[L].co;
        ci = kLayers[L].ci;
        k = kLayers[L].k;
    }
    pc.k = k;
    pc.Co = co;
    pc.nchunk = (ci + 15) / 16;
    pc.co_tot = (co + kCoT - 1) / kCoT * kCoT;
    const int taps = k * k;
    std::vector<_Float16> w((size_t)taps * pc.nchunk * pc.co_tot * 16, (_Float16)0.0f);
    std::vector<float> b(pc.co_tot, 0.0f);
    int row = 0;
    for (int L : layers) {
        const LayerShape& ls = kLayers[L];
        const std::vector<float>& src = s->hw_[L];
        for (int o = 0; o < ls.co; o++) {
            b[row + o] = s->hb_[L][o];
            for (int c = 0; c < ls.ci; c++)
                for (int t = 0; t < taps; t++) {
                    const float v = src[((size_t)o * ls.ci + c) * taps + t];
                    w[(((size_t)t * pc.nchunk + c / 16) * pc.co_tot + row + o) * 16 + c % 16] =
                        (_Float16)v;
                }
        }
        row += ls.co;
    }
    SLK_TRY(pc.wt.ensure(w.size() * sizeof(_Float16)));
    SLK_TRY(pc.bias.ensure(b.size() * sizeof(float)));
    SLK_HIP(hipMemcpy(pc.wt.ptr, w.data(), w.size() * sizeof(_Float16), hipMemcpyHostToDevice));
    SLK_HIP(hipMemcpy(pc.bias.ptr, b.data(), b.size() * sizeof(float), hipMemcpyHostToDevice));
    return SLK_OK;
}

// The 7x7 stem of 4 input channels with its taps packed into K (k_conv7p):
// [13][co_tot][16] fp16, k = 4 (t - 4 ks) + c; taps 49..51 zero.
int pack_taps4(PackedConv& pc, const UpdateState* s, int L) {
    const LayerShape& ls = kLayers[L];
    constexpr int kSteps = 13;
    if (ls.k != 7 || ls.ci != 4) return fail(SLK_E_STATE, "update: tap-packed layer shape");
    pc.k = 7;
    pc.Co = ls.co;
    pc.nchunk = kSteps;
    pc.co_tot = (ls.co + kCoT - 1) / kCoT * kCoT;
    std::vector<_Float16> w((size_t)kSteps * pc.co_tot * 16, (_Float16)0.0f);
    std::vector<float> b(pc.co_tot, 0.0f);
    const std::vector<float>& src = s->hw_[L];
    for (int o = 0; o < ls.co; o++) {
        b[o] = s->hb_[L][o];
        for (int c = 0; c < 4; c++)
            for (int t = 0; t < 49; t++)
                w[((size_t)(t / 4) * pc.co_tot + o) * 16 + 4 * (t % 4) + c] =
                    (_Float16)src[((size_t)o * 4 + c) * 49 + t];
    }
    SLK_TRY(pc.wt.ensure(w.size() * sizeof(_Float16)));
    SLK_TRY(pc.bias.ensure(b.size() * sizeof(float)));
    SLK_HIP(hipMemcpy(pc.wt.ptr, w.data(), w.size() * sizeof(_Float16), hipMemcpyHostToDevice));
    SLK_HIP(hipMemcpy(pc.bias.ptr, b.data(), b.size() * sizeof(float), hipMemcpyHostToDevice));
    return SLK_OK;
}

int upload_rounded(DevBuf& d, const std::vector<float>& v) {
    std::vector<float> r(v.size());
    for (size_t i = 0; i < v.size(); i++) r[i] = round_half_host(v[i]);
    SLK_TRY(d.ensure(std::max<size_t>(1, r.size()) * sizeof(float)));
    SLK_HIP(hipMemcpy(d.ptr, r.data(), r.size() * sizeof(float), hipMemcpyHostToDevice));
    return SLK_OK;
}

int upload(DevBuf& d, const std::vector<float>& v) {
    SLK_TRY(d.ensure(std::max<size_t>(1, v.size()) * sizeof(float)));
    SLK_HIP(hipMemcpy(d.ptr, v.data(), v.size() * sizeof(float), hipMemcpyHostToDevice));
    return SLK_OK;
}

// small 3x3 heads: weights fp16-rounded as float in the k_conv_small order
// [o][chunk][tap][16] (from the reference's [o][ci][3][3]); biases padded to 3
void small_layout(const UpdateState* s, int L, std::vector<float>& w, std::vector<float>& b) {
    const int co = kLayers[L].co;
    for (int o = 0; o < co; o++)
        for (int ch = 0; ch < 8; ch++)
            for (int t = 0; t < 9; t++)
                for (int i = 0; i < 16; i++)
                    w.push_back(round_half_host(s->hw_[L][((size_t)o * 128 + ch * 16 + i) * 9 + t]));
    for (int o = 0; o < 3; o++) b.push_back(o < co ? s->hb_[L][o] : 0.0f);
}

int pack_all(UpdateState* s) {
    for (int L = 0; L < kNumLayers; L++)
        if (!s->have[L])
            return fail(SLK_E_STATE, std::string("update: weights of ") + kLayers[L].name +
                                         " not set");
    SLK_TRY(pack(s->ce0, s, {L_CE0}));
    SLK_TRY(pack(s->ce2, s, {L_CE2}));
    SLK_TRY(pack_taps4(s->fe0, s, L_FE0));
    SLK_TRY(pack(s->fe2, s, {L_FE2}));
    SLK_TRY(pack(s->gw, s, {L_W}));
    SLK_TRY(pack(s->zr, s, {L_Z, L_R}));
    SLK_TRY(pack(s->q, s, {L_Q}));
    SLK_TRY(pack(s->heads, s, {L_DL0, L_WT0, L_AG1}));
    SLK_TRY(pack(s->ag2, s, {L_AG2}));
    // global convs: [384][128] rounded, stacked z | r | q
    std::vector<float> gw, gb;
    for (int L : {L_ZG, L_RG, L_QG}) {
        gw.insert(gw.end(), s->hw_[L].begin(), s->hw_[L].end());
        gb.insert(gb.end(), s->hb_[L].begin(), s->hb_[L].end());
    }
    SLK_TRY(upload_rounded(s->glo_w, gw));
    SLK_TRY(upload(s->glo_b, gb));
    {
        std::vector<float> w, b;  // delta_2 then weight_2: one launch, two heads
        small_layout(s, L_DL2, w, b);
        small_layout(s, L_WT2, w, b);
        SLK_TRY(upload(s->small_w[0], w));
        SLK_TRY(upload(s->small_b[0], b));
        std::vector<float> we, be;
        small_layout(s, L_ETA, we, be);
        SLK_TRY(upload(s->small_w[2], we));
        SLK_TRY(upload(s->small_b[2], be));
    }
    SLK_HIP(hipDeviceSynchronize());
    s->packed = true;
    return SLK_OK;
}

template <int KS, int EPI>
int launch_conv(const UpdateState* s, const PackedConv& pc, ConvArgs a, int N,
                hipStream_t stream) {
    a.nchunk = pc.nchunk;
    a.wt = pc.wt.as<_Float16>();
    a.bias = pc.bias.as<float>();
    a.co_tot = pc.co_tot;
    a.Co = pc.Co;
    a.h = s->h;
    a.w = s->w;
    a.tiles_x = s->tiles_x;
    if (a.s0.nchunk > a.nchunk) a.s0.nchunk = a.nchunk;
    if constexpr (KS == 1) {
        const int hw = s->h * s->w;
        hipLaunchKernelGGL((k_conv1x1<EPI>), dim3(pc.co_tot / kCoT, (hw + 255) / 256, N),
                           dim3(256), 0, stream, a);
    } else if constexpr (KS == 3) {
        a.zero16 = s->zero16.as<_Float16>();
        const int ty = (s->h + kTH3 - 1) / kTH3;
        hipLaunchKernelGGL((k_conv3<EPI, kTH3>), dim3(pc.co_tot / kCoT, s->tiles_x * ty, N),
                           dim3(256), 0, stream, a);
    } else {
        static_assert(KS == 7, "the 7x7 stem is the only other convolution");
        hipLaunchKernelGGL((k_conv7p<EPI>), dim3(pc.co_tot / kCoT, s->tiles_x * s->tiles_y, N),
                           dim3(256), 0, stream, a);
    }
    SLK_HIP(hipGetLastError());
    return SLK_OK;
}

CkSrc src(const DevBuf& b, int chunk0, int nchunk, long nstride, int hw) {
    CkSrc c;
    c.p = b.as<_Float16>() + (long)chunk0 * hw * 16;
    c.nchunk = nchunk;
    c.nstride = nstride;
    return c;
}

// chunks of the activation buffers (per image)
constexpr int kCorrCh = 13;  // 196 channels -> 13 chunks (208, zero-padded)
constexpr int kCatCh = 28;   // net 0..7 | inp 8..15 | corr features 16..23 | flow 24..27
constexpr int kTmpCh = 8;    // c1 / f1 / gate
constexpr int kZrCh = 16;    // z 0..7 | r*net 8..15; later the heads' 256 channels

}  // namespace
}  // namespace slk

using namespace slk;

struct slk_update {
    UpdateState s;
};

extern "C" int slk_update_create(slk_update** out, int max_batch, int h, int w) {
    if (!out) return fail(SLK_E_ARG, "update_create: null output");
    *out = nullptr;
    if (max_batch < 1 || h < 1 || w < 1 || (long)h * w > (1L << 22))
        return fail(SLK_E_ARG, "update_create: need max_batch >= 1, 1 <= h*w <= 2^22");
    slk_update* u = new slk_update();
    UpdateState& s = u->s;
    s.max_batch = max_batch;
    s.h = h;
    s.w = w;
    s.tiles_x = (w + kTW - 1) / kTW;
    s.tiles_y = (h + kTH - 1) / kTH;
    const size_t hw = (size_t)h * w, chunk = hw * 16 * sizeof(_Float16);
    const size_t N = (size_t)max_batch;
    int st = SLK_OK;
    if (st == SLK_OK) st = s.corr16.ensure(N * kCorrCh * chunk);
    if (st == SLK_OK) st = s.mot16.ensure(N * chunk);
    if (st == SLK_OK) st = s.cat.ensure(N * kCatCh * chunk);
    if (st == SLK_OK) st = s.tmp.ensure(N * kTmpCh * chunk);
    if (st == SLK_OK) st = s.tmp_f.ensure(N * kTmpCh * chunk);
    if (st == SLK_OK) st = s.tmp_g.ensure(N * kTmpCh * chunk);
    if (st == SLK_OK) st = s.zr_buf.ensure(N * kZrCh * chunk);
    if (st == SLK_OK) st = s.glo.ensure(N * 128 * sizeof(float));
    if (st == SLK_OK) st = s.gterm.ensure(N * 384 * sizeof(float));
    if (st == SLK_OK) st = s.zero16.ensure(256);
    if (st == SLK_OK && hipMemset(s.zero16.ptr, 0, 256) != hipSuccess)
        st = fail(SLK_E_HIP, "update_create: hipMemset failed");
    for (int i = 0; i < 2 && st == SLK_OK; i++)
        if (hipStreamCreateWithFlags(&s.side[i], hipStreamNonBlocking) != hipSuccess ||
            hipEventCreateWithFlags(&s.ev_join[i], hipEventDisableTiming) != hipSuccess)
            st = fail(SLK_E_HIP, "update_create: stream or event creation failed");
    if (st == SLK_OK && hipEventCreateWithFlags(&s.ev_fork, hipEventDisableTiming) != hipSuccess)
        st = fail(SLK_E_HIP, "update_create: event creation failed");
    if (st != SLK_OK) {
        slk_update_destroy(u);
        return st;
    }
    *out = u;
    return SLK_OK;
}

extern "C" int slk_update_destroy(slk_update* u) {
    if (!u) return SLK_OK;
    UpdateState& s = u->s;
    for (int i = 0; i < 2; i++) {
        if (s.side[i]) {
            // the side streams' work is finished before its buffers go
            (void)hipStreamSynchronize(s.side[i]);
            (void)hipStreamDestroy(s.side[i]);
        }
        if (s.ev_join[i]) (void)hipEventDestroy(s.ev_join[i]);
    }
    if (s.ev_fork) (void)hipEventDestroy(s.ev_fork);
    for (PackedConv* pc : {&s.ce0, &s.ce2, &s.fe0, &s.fe2, &s.gw, &s.zr, &s.q, &s.heads, &s.ag2}) {
        pc->wt.release();
        pc->bias.release();
    }
    for (DevBuf* b : {&s.glo_w, &s.glo_b, &s.small_w[0], &s.small_w[1], &s.small_w[2],
                      &s.small_b[0], &s.small_b[1], &s.small_b[2], &s.corr16, &s.mot16, &s.cat,
                      &s.tmp, &s.tmp_f, &s.tmp_g, &s.zr_buf, &s.glo, &s.gterm, &s.agg16, &s.agg_t,
                      &s.zero16, &s.mf_coords,
                      &s.mf_corr, &s.mf_motion, &s.mf_net, &s.mf_inp, &s.mf_delta, &s.mf_weight,
                      &s.mf_agg})
        b->release();
    delete u;
    return SLK_OK;
}

extern "C" int slk_update_num_layers(void) { return kNumLayers; }

extern "C" const char* slk_update_layer_name(int layer) {
    return layer >= 0 && layer < kNumLayers ? kLayers[layer].name : nullptr;
}

extern "C" int slk_update_layer_shape(int layer, int* co, int* ci, int* k) {
    if (layer < 0 || layer >= kNumLayers) return fail(SLK_E_ARG, "update_layer_shape: bad layer");
    if (co) *co = kLayers[layer].co;
    if (ci) *ci = kLayers[layer].ci;
    if (k) *k = kLayers[layer].k;
    return SLK_OK;
}

extern "C" int slk_update_set_conv(slk_update* u, int layer, const float* weight_host,
                                   const float* bias_host) {
    if (!u || layer < 0 || layer >= kNumLayers || !weight_host || !bias_host)
        return fail(SLK_E_ARG, "update_set_conv: bad argument");
    UpdateState& s = u->s;
    const LayerShape& ls = kLayers[layer];
    const size_t nw = (size_t)ls.co * ls.ci * ls.k * ls.k;
    s.hw_[layer].assign(weight_host, weight_host + nw);
    s.hb_[layer].assign(bias_host, bias_host + ls.co);
    s.have[layer] = true;
    s.packed = false;
    return SLK_OK;
}

extern "C" int slk_update_load_dir(slk_update* u, const char* dir) {
    if (!u || !dir) return fail(SLK_E_ARG, "update_load_dir: bad argument");
    for (int L = 0; L < kNumLayers; L++) {
        const LayerShape& ls = kLayers[L];
        std::vector<float> wb[2];
        for (int part = 0; part < 2; part++) {
            const std::string path = std::string(dir) + "/" + ls.name +
                                     (part ? "_bias.bin" : "_weight.bin");
            FILE* f = std::fopen(path.c_str(), "rb");
            if (!f) return fail(SLK_E_ARG, "update_load_dir: cannot open " + path);
            int nd = 0;
            bool ok = std::fread(&nd, sizeof(int), 1, f) == 1 && nd >= 1 && nd <= 4;
            size_t total = 1;
            int dims[4] = {0, 0, 0, 0};
            for (int d = 0; ok && d < nd; d++) {
                ok = std::fread(&dims[d], sizeof(int), 1, f) == 1 && dims[d] > 0;
                total *= ok ? (size_t)dims[d] : 0;
            }
            const size_t want = part ? (size_t)ls.co : (size_t)ls.co * ls.ci * ls.k * ls.k;
            ok = ok && total == want;
            if (ok) {
                wb[part].resize(total);
                ok = std::fread(wb[part].data(), sizeof(float), total, f) == total;
            }
            std::fclose(f);
            if (!ok) return fail(SLK_E_ARG, "update_load_dir: bad tensor file " + path);
        }
        SLK_TRY(slk_update_set_conv(u, L, wb[0].data(), wb[1].data()));
    }
    return SLK_OK;
}

extern "C" int slk_update_forward(slk_update* u, const float* corr, const float* motion,
                                  float* net, const float* inp, float* delta_out,
                                  float* weight_out, float* agg_conv1_out, int batch,
                                  hipStream_t stream) {
    if (!u) return fail(SLK_E_ARG, "update_forward: null module");
    UpdateState& s = u->s;
    if (batch < 0 || batch > s.max_batch)
        return fail(SLK_E_ARG, "update_forward: batch outside [0, max_batch]");
    if (batch == 0) return SLK_OK;
    if (!corr || !motion || !net || !inp || !delta_out || !weight_out || !agg_conv1_out)
        return fail(SLK_E_ARG, "update_forward: null argument");
    if (!s.packed) SLK_TRY(pack_all(&s));
    const int hw = s.h * s.w, N = batch;
    const long ck = (long)hw * 16;  // elements of one chunk
    // inputs to CK fp16: corr (196 ch), motion (4 ch), net and inp (128 ch)
    auto to_ck = [&](const float* in, int C, DevBuf& out, int out_ch, int c0, float* wb,
                     hipStream_t on) {
        dim3 g((hw + 255) / 256, (C + 15) / 16, N);
        hipLaunchKernelGGL(k_to_ck<false>, g, dim3(256), 0, on, in, (long)C * hw, C,
                           out.as<_Float16>(), out_ch * ck, c0, hw, wb);
    };
    const long catS = kCatCh * ck, tmpS = kTmpCh * ck, zrS = kZrCh * ck;
    // The three encoders of convz|convr's input are independent: the flow
    // encoder runs on side[0], the gate on side[1], the correlation encoder on
    // the caller's stream; each writes its own chunks of cat through its own
    // scratch, and the caller's stream waits for both sides before convz|convr.
    // The fork follows everything the caller queued before this call (the
    // inputs, and the previous call's readers of cat and the scratch).
    hipStream_t sf = s.side[0], sg = s.side[1];
    SLK_HIP(hipEventRecord(s.ev_fork, stream));
    SLK_HIP(hipStreamWaitEvent(sf, s.ev_fork, 0));
    SLK_HIP(hipStreamWaitEvent(sg, s.ev_fork, 0));
    // corr encoder: 1x1 196 -> 128, 3x3 128 -> 128 into cat chunks 16..23
    {
        to_ck(corr, 196, s.corr16, kCorrCh, 0, nullptr, stream);
        ConvArgs a{};
        a.s0 = src(s.corr16, 0, kCorrCh, kCorrCh * ck, hw);
        a.out16 = s.tmp.as<_Float16>();
        a.out16_nstride = tmpS;
        SLK_TRY((launch_conv<1, kEpiRelu>(&s, s.ce0, a, N, stream)));
        ConvArgs b{};
        b.s0 = src(s.tmp, 0, 8, tmpS, hw);
        b.out16 = s.cat.as<_Float16>() + 16 * ck;
        b.out16_nstride = catS;
        SLK_TRY((launch_conv<3, kEpiRelu>(&s, s.ce2, b, N, stream)));
    }
    // flow encoder: 7x7 4 -> 128, 3x3 128 -> 64 into cat chunks 24..27
    {
        to_ck(motion, 4, s.mot16, 1, 0, nullptr, sf);
        ConvArgs a{};
        a.s0 = src(s.mot16, 0, 1, ck, hw);
        a.out16 = s.tmp_f.as<_Float16>();
        a.out16_nstride = tmpS;
        SLK_TRY((launch_conv<7, kEpiRelu>(&s, s.fe0, a, N, sf)));
        ConvArgs b{};
        b.s0 = src(s.tmp_f, 0, 8, tmpS, hw);
        b.out16 = s.cat.as<_Float16>() + 24 * ck;
        b.out16_nstride = catS;
        SLK_TRY((launch_conv<3, kEpiRelu>(&s, s.fe2, b, N, sf)));
        SLK_HIP(hipEventRecord(s.ev_join[0], sf));
    }
    // net and inp into cat chunks 0..15; GRU gate = round16(sigmoid(w(net)))
    // * net, pooled; global terms
    {
        to_ck(net, 128, s.cat, kCatCh, 0, nullptr, sg);
        to_ck(inp, 128, s.cat, kCatCh, 8, nullptr, sg);
        ConvArgs a{};
        a.s0 = src(s.cat, 0, 8, catS, hw);
        a.out16 = s.tmp_g.as<_Float16>();
        a.out16_nstride = tmpS;
        a.net16 = s.cat.as<_Float16>();
        a.net_nstride = catS;
        SLK_TRY((launch_conv<1, kEpiGate>(&s, s.gw, a, N, sg)));
        hipLaunchKernelGGL(k_gate_pool, dim3(8, N), dim3(256), 0, sg, s.tmp_g.as<_Float16>(),
                           tmpS, hw, s.glo.as<float>());
        hipLaunchKernelGGL(k_glo_fc, dim3(N), dim3(384), 0, sg, s.glo.as<float>(),
                           s.glo_w.as<float>(), s.glo_b.as<float>(), s.gterm.as<float>());
        SLK_HIP(hipGetLastError());
        SLK_HIP(hipEventRecord(s.ev_join[1], sg));
    }
    SLK_HIP(hipStreamWaitEvent(stream, s.ev_join[0], 0));
    SLK_HIP(hipStreamWaitEvent(stream, s.ev_join[1], 0));
    // z | r (one 256-row GEMM over the 448-channel concatenation), then q and
    // the state update
    {
        ConvArgs a{};
        a.s0 = src(s.cat, 0, kCatCh, catS, hw);
        a.zbuf = s.zr_buf.as<_Float16>();
        a.rnet = s.zr_buf.as<_Float16>() + 8 * ck;
        a.zr_nstride = zrS;
        a.net16 = s.cat.as<_Float16>();
        a.net_nstride = catS;
        a.gterm = s.gterm.as<float>();
        SLK_TRY((launch_conv<3, kEpiZR>(&s, s.zr, a, N, stream)));
        ConvArgs b{};
        b.s0 = src(s.zr_buf, 8, 8, zrS, hw);   // r * net
        b.s1 = src(s.cat, 8, 20, catS, hw);    // inp | corr features | flow
        b.zbuf = s.zr_buf.as<_Float16>();
        b.zr_nstride = zrS;
        b.net16 = s.cat.as<_Float16>();
        b.net_nstride = catS;
        b.gterm = s.gterm.as<float>();
        b.out32 = net;
        b.out32_nstride = 128L * hw;
        SLK_TRY((launch_conv<3, kEpiQ>(&s, s.q, b, N, stream)));
    }
    // heads of the new state: delta_0 | weight_0 | agg_conv1
    {
        ConvArgs a{};
        a.s0 = src(s.cat, 0, 8, catS, hw);
        a.out16 = s.zr_buf.as<_Float16>();  // 16 chunks: delta_0 | weight_0
        a.out16_nstride = zrS;
        a.out32 = agg_conv1_out;
        a.out32_nstride = 128L * hw;
        SLK_TRY((launch_conv<3, kEpiHeads>(&s, s.heads, a, N, stream)));
        SmallArgs m{};
        m.in = s.zr_buf.as<_Float16>();  // delta_0 chunks 0..7, weight_0 chunks 8..15
        m.in_nstride = zrS;
        m.W = s.small_w[0].as<float>();
        m.b = s.small_b[0].as<float>();
        m.wstride = 3L * 8 * 9 * 16;
        m.Co = 3;
        m.h = s.h;
        m.w = s.w;
        m.tiles_x = s.tiles_x;
        m.nheads = 2;
        m.mode[0] = 0;
        m.mode[1] = 1;
        m.out[0] = delta_out;
        m.out[1] = weight_out;
        m.out_nstride = 3L * hw;
        hipLaunchKernelGGL(k_conv_small, dim3(s.tiles_x * s.tiles_y, 2, N), dim3(256), 0, stream,
                           m);
        SLK_HIP(hipGetLastError());
    }
    return SLK_OK;
}

extern "C" int slk_update_compute_eta(slk_update* u, float* agg_features, float* eta_out,
                                      int num_kf, hipStream_t stream) {
    if (!u) return fail(SLK_E_ARG, "update_compute_eta: null module");
    UpdateState& s = u->s;
    if (num_kf < 0) return fail(SLK_E_ARG, "update_compute_eta: num_kf < 0");
    if (num_kf == 0) return SLK_OK;
    if (!agg_features || !eta_out) return fail(SLK_E_ARG, "update_compute_eta: null argument");
    if (!s.packed) SLK_TRY(pack_all(&s));
    const int hw = s.h * s.w, K = num_kf;
    const long ck = (long)hw * 16;
    const size_t chunk = (size_t)ck * sizeof(_Float16);
    if (s.agg16.bytes < (size_t)K * 8 * chunk) {
        SLK_HIP(hipStreamSynchronize(stream));  // earlier calls may still read them
        SLK_TRY(s.agg16.ensure((size_t)K * 8 * chunk));
        SLK_TRY(s.agg_t.ensure((size_t)K * 8 * chunk));
    }
    // round16 of the features in place (main.cu:659), to CK fp16
    hipLaunchKernelGGL(k_to_ck<true>, dim3((hw + 255) / 256, 8, K), dim3(256), 0, stream,
                       agg_features, 128L * hw, 128, s.agg16.as<_Float16>(), 8 * ck, 0, hw,
                       agg_features);
    SLK_HIP(hipGetLastError());
    ConvArgs a{};
    a.s0 = src(s.agg16, 0, 8, 8 * ck, hw);
    a.out16 = s.agg_t.as<_Float16>();
    a.out16_nstride = 8 * ck;
    SLK_TRY((launch_conv<3, kEpiRelu>(&s, s.ag2, a, K, stream)));
    SmallArgs m{};
    m.in = s.agg_t.as<_Float16>();
    m.in_nstride = 8 * ck;
    m.W = s.small_w[2].as<float>();
    m.b = s.small_b[2].as<float>();
    m.Co = 1;
    m.h = s.h;
    m.w = s.w;
    m.tiles_x = s.tiles_x;
    m.nheads = 1;
    m.mode[0] = 2;
    m.out[0] = eta_out;
    m.out_nstride = hw;
    hipLaunchKernelGGL(k_conv_small, dim3(s.tiles_x * s.tiles_y, 1, K), dim3(256), 0, stream, m);
    SLK_HIP(hipGetLastError());
    return SLK_OK;
}

extern "C" int slk_motion_filter(slk_ctx* ctx, slk_update* u, const void* f_last,
                                 const void* f_cur, int dtype, const float* net_kf,
                                 const float* inp_kf, float* mean_flow, hipStream_t stream) {
    if (!ctx || !u || !f_last || !f_cur || !net_kf || !inp_kf || !mean_flow)
        return fail(SLK_E_ARG, "motion_filter: null argument");
    UpdateState& s = u->s;
    if (ctx->h != s.h || ctx->w != s.w)
        return fail(SLK_E_ARG, "motion_filter: context and update module map sizes differ");
    if (ctx->levels != 4) return fail(SLK_E_ARG, "motion_filter: needs a 4-level context");
    const int hw = s.h * s.w;
    const size_t f4 = sizeof(float);
    if (!s.mf_coords.ptr) {
        SLK_TRY(s.mf_coords.ensure(2 * hw * f4));
        SLK_TRY(s.mf_corr.ensure(196 * hw * f4));
        SLK_TRY(s.mf_motion.ensure(4 * hw * f4));
        SLK_TRY(s.mf_net.ensure(128 * hw * f4));
        SLK_TRY(s.mf_inp.ensure(128 * hw * f4));
        SLK_TRY(s.mf_delta.ensure(3 * hw * f4));
        SLK_TRY(s.mf_weight.ensure(3 * hw * f4));
        SLK_TRY(s.mf_agg.ensure(128 * hw * f4));
        s.mf_host.resize(2 * (size_t)hw);
    }
    // build_correlation(last_kf, temp slot) and the lookup at the identity
    // grid (main.cu:1939-1951)
    SLK_TRY(slk_corr_build(ctx, f_last, f_cur, dtype, stream));
    SLK_TRY(slk_fill_coords0(s.mf_coords.as<float>(), 1, s.h, s.w, stream));
    SLK_TRY(slk_corr_sample(ctx, s.mf_coords.as<float>(), s.mf_corr.as<float>(), stream));
    // the keyframe's hidden state and context, zero motion (main.cu:1954-1961)
    SLK_HIP(hipMemcpyAsync(s.mf_net.ptr, net_kf, 128 * hw * f4, hipMemcpyDeviceToDevice, stream));
    SLK_HIP(hipMemcpyAsync(s.mf_inp.ptr, inp_kf, 128 * hw * f4, hipMemcpyDeviceToDevice, stream));
    SLK_HIP(hipMemsetAsync(s.mf_motion.ptr, 0, 4 * hw * f4, stream));
    SLK_TRY(slk_update_forward(u, s.mf_corr.as<float>(), s.mf_motion.as<float>(),
                               s.mf_net.as<float>(), s.mf_inp.as<float>(), s.mf_delta.as<float>(),
                               s.mf_weight.as<float>(), s.mf_agg.as<float>(), 1, stream));
    // mean flow magnitude of delta's first two channels, summed on the host in
    // pixel order as the reference does (main.cu:1970-1981)
    SLK_HIP(hipMemcpyAsync(s.mf_host.data(), s.mf_delta.ptr, 2 * hw * f4, hipMemcpyDeviceToHost,
                           stream));
    SLK_HIP(hipStreamSynchronize(stream));
    float sum = 0.0f;
    for (int k = 0; k < hw; k++) {
        const float dx = s.mf_host[k], dy = s.mf_host[hw + k];
        sum += std::sqrt(dx * dx + dy * dy);
    }
    *mean_flow = sum / (float)hw;
    return SLK_OK;
}
