// Deterministic wave64 / workgroup reductions (fixed butterfly order, so a
// result does not depend on scheduling; no atomics).
#pragma once

#include <hip/hip_runtime.h>

namespace slk {

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
    return v;
}

__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
    return v;
}

// Sums N values per thread over the workgroup (blockDim.x a multiple of 64,
// at most 1024). `scratch` holds N * (blockDim.x / 64) elements. On return
// every thread of the workgroup sees the totals in v[]. Contains barriers:
// call from all threads.
template <typename T, int N>
__device__ __forceinline__ void block_sum(T (&v)[N], T* scratch) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int nw = blockDim.x >> 6;
#pragma unroll
    for (int k = 0; k < N; k++) v[k] = wave_sum(v[k]);
    __syncthreads();
    if (lane == 0) {
#pragma unroll
        for (int k = 0; k < N; k++) scratch[k * nw + wave] = v[k];
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < N; k++) {
        T s = scratch[k * nw];
        for (int w = 1; w < nw; w++) s += scratch[k * nw + w];
        v[k] = s;
    }
    __syncthreads();
}

// Partner exchange for the butterfly: the value of a lane whose index differs
// in bit log2(M). Bits 0..3 use DPP inside rows of 16 lanes (quad permutes for
// M = 1, 2; the half-row mirror i <-> 7-i for M = 4 and the row mirror
// i <-> 15-i for M = 8: involutions that flip that bit), which are plain VALU
// moves; M = 16, 32 go through ds_bpermute.
template <int M>
__device__ __forceinline__ int xchg_i32(int v) {
    if constexpr (M == 1)
        return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
    else if constexpr (M == 2)
        return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
    else if constexpr (M == 4)
        return __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);  // row_half_mirror
    else if constexpr (M == 8)
        return __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false);  // row_mirror
    else
        return __shfl_xor(v, M);
}

template <int M>
__device__ __forceinline__ float xchg(float v) {
    return __builtin_bit_cast(float, xchg_i32<M>(__builtin_bit_cast(int, v)));
}

template <int M>
__device__ __forceinline__ double xchg(double v) {
    const int lo = xchg_i32<M>(__double2loint(v));
    const int hi = xchg_i32<M>(__double2hiint(v));
    return __hiloint2double(hi, lo);
}

// Butterfly reduce-scatter of N values over the 64 lanes of a wave. At each
// of the 6 levels (lane bits 3, 2, 1, 0, 4, 5: the many-value levels on DPP)
// a lane keeps
// one half of its values and trades the other half with its partner, so the
// whole reduction costs about N exchanges instead of the 6N of N independent
// wave_sum()s. On return lane l holds the wave totals of `valid` consecutive
// value indices starting at `base` in v[0..valid).
template <typename T, int C, int M>
__device__ __forceinline__ void rs_level(T* v, int lane, int& base, int& valid) {
    constexpr int H = (C + 1) / 2;
    const bool up = (lane & M) != 0;
#pragma unroll
    for (int k = 0; k < H; k++) {
        const T lo = v[k];
        const T hi = (k + H < C) ? v[k + H] : T(0);
        const T send = up ? lo : hi;
        const T keep = up ? hi : lo;
        v[k] = keep + xchg<M>(send);
    }
    if (up) {
        base += H;
        valid = valid > H ? valid - H : 0;
    } else {
        valid = valid < H ? valid : H;
    }
}

template <int N>
struct RsCounts {
    static constexpr int c0 = N, c1 = (c0 + 1) / 2, c2 = (c1 + 1) / 2, c3 = (c2 + 1) / 2,
                         c4 = (c3 + 1) / 2, c5 = (c4 + 1) / 2, c6 = (c5 + 1) / 2;
};

template <typename T, int N>
__device__ __forceinline__ void wave_reduce_scatter(T (&v)[N], int lane, int& base, int& valid) {
    using R = RsCounts<N>;
    base = 0;
    valid = N;
    // The partners of a level must agree in every bit already processed: the
    // mirrors flip all lower bits, so they come first (bit 3, then bit 2),
    // then the exact bit flips.
    rs_level<T, R::c0, 8>(v, lane, base, valid);
    rs_level<T, R::c1, 4>(v, lane, base, valid);
    rs_level<T, R::c2, 2>(v, lane, base, valid);
    rs_level<T, R::c3, 1>(v, lane, base, valid);
    rs_level<T, R::c4, 16>(v, lane, base, valid);
    rs_level<T, R::c5, 32>(v, lane, base, valid);
}

// Workgroup totals of N values per thread into tot[0..N) (LDS or global),
// deterministic: reduce-scatter inside each wave, then a fixed-order sum over
// the waves. `scratch` holds N * (blockDim.x / 64) elements of LDS. Contains
// barriers: call from all threads. v[] is clobbered.
template <typename T, int N>
__device__ __forceinline__ void block_sum_to(T (&v)[N], T* scratch, T* tot) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int nw = blockDim.x >> 6;
    int base, valid;
    wave_reduce_scatter(v, lane, base, valid);
    __syncthreads();
#pragma unroll
    for (int k = 0; k < RsCounts<N>::c6; k++)
        if (k < valid) scratch[(base + k) * nw + wave] = v[k];
    __syncthreads();
    for (int t = threadIdx.x; t < N; t += blockDim.x) {
        T s = scratch[t * nw];
        for (int w = 1; w < nw; w++) s += scratch[t * nw + w];
        tot[t] = s;
    }
    __syncthreads();
}

}  // namespace slk
