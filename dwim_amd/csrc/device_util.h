// Device helpers for gfx950: wave64 reductions and small math.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define DEV __device__ __forceinline__

// Sum over groups of `width` consecutive lanes (width a power of two <= 64),
// every lane of a group getting the group's total.
template <int WIDTH>
DEV float group_sum(float v) {
#pragma unroll
    for (int m = WIDTH / 2; m > 0; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

template <int WIDTH>
DEV float group_max(float v) {
#pragma unroll
    for (int m = WIDTH / 2; m > 0; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
    return v;
}

// Block-wide sum for blocks of NT threads (a multiple of 64); `red` holds
// NT/64 floats of LDS.  Every thread gets the total.
template <int NT>
DEV float block_sum(float v, float *red) {
    v = group_sum<64>(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (NT > 64) {
        __syncthreads();
        if (lane == 0) red[wave] = v;
        __syncthreads();
        float t = 0.0f;
#pragma unroll
        for (int i = 0; i < NT / 64; i++) t += red[i];
        v = t;
    }
    return v;
}

DEV float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }
DEV float softplusf_(float x) { return x > 20.0f ? x : logf(1.0f + expf(x)); }
