// Device helpers shared by the correlation kernels (corr.hip, corr_split.hip).
#pragma once

#include <hip/hip_runtime.h>

#include "slk_internal.hpp"

namespace slk {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef unsigned short u16x8_t __attribute__((ext_vector_type(8)));

constexpr int kMaxEdgesPerLaunch = 64;

// word 3 of a raw buffer resource on gfx9-family parts (32-bit data format,
// no swizzle; range checking against num_records)
constexpr int kBufWord3 = 0x00020000;
// an offset past any buffer the correlation kernels build a resource for: a
// store there is discarded and a load returns zeros, without a memory access
constexpr int kBufDiscard = 0x7FFFFFF0;
constexpr int kWinCells = 64;  // 8x8 window cells per level

// Lookup windows of a launch are stored row-major per window row,
// [slot][level][row][HW][8] (cell = 8*row + column of the 8x8 window): a
// window row of 8 consecutive sources is 256 contiguous bytes, so the
// correlation kernel's stores and the lookup's per-pixel reads are coalesced.
__host__ __device__ __forceinline__ size_t win_index(int slot, int l, int cell, int HW, int p) {
    return ((((size_t)slot * kMaxLevels + l) * 8 + (cell >> 3)) * HW + p) * 8 + (cell & 7);
}

// Workgroups are dispatched round-robin over the 8 XCDs; remap the linear id so
// each XCD walks a contiguous range of (edge, tile) ids and its L2 holds the
// few feature maps of the edges it is working on.
__device__ __forceinline__ int xcd_remap(int bid, int total) {
    constexpr int X = 8;
    const int q = total / X, rem = total % X;
    const int xcd = bid % X, local = bid / X;
    return (xcd < rem) ? xcd * (q + 1) + local : rem * (q + 1) + (xcd - rem) * q + local;
}

// First window cell of a lookup at level l: floor(c * 2^-l) - 3, with the
// coordinate scaled in fp32 as main.cu:1189-1190 does. Clamped so that far or
// non-finite coordinates give an origin no cell can match.
__device__ __forceinline__ int win_origin(float c, int l) {
    const float s = c * (1.0f / (float)(1 << l));
    return (int)fminf(fmaxf(floorf(s), -1048576.0f), 1048576.0f) - 3;
}

// floor(c) clamped to +-2^20 (NaN -> -2^20). Since c * 2^-l is exact and
// floor(floor(c) / 2^l) == floor(c / 2^l), (floor_clamped(c) >> l) - 3 equals
// win_origin(c, l) for |c| < 2^20; beyond that both are outside every level's
// grid (image sides are limited to 2^16).
__device__ __forceinline__ int floor_clamped(float c) {
    return (int)fminf(fmaxf(floorf(c), -1048576.0f), 1048576.0f);
}

// hi = rne_bf16(x), lo = rne_bf16(x - hi), packed as lo << 16 | hi
__device__ __forceinline__ unsigned split_bf16(float x) {
    const __bf16 h = (__bf16)x;
    const __bf16 l = (__bf16)(x - (float)h);
    return (unsigned)__builtin_bit_cast(unsigned short, h) |
           ((unsigned)__builtin_bit_cast(unsigned short, l) << 16);
}

}  // namespace slk
