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

}  // namespace slk
