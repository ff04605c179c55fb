// Reduction helpers shared by the PPO and optimizer kernels.
#pragma once

#include "common.hpp"

namespace rl {

// f(x[i]) summed over i = first, first + stride, ... < n, in that order.  Eight loads are issued before
// their adds: a plain loop waits for each load before issuing the next, one memory round trip per term.
template <typename F>
__device__ __forceinline__ float strided_sum(const float* x, long long first, long long n, long long stride, F f) {
    float v = 0.0f;
    long long i = first;
    for (; i + 7 * stride < n; i += 8 * stride) {
        float w[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) w[u] = x[i + u * stride];
#pragma unroll
        for (int u = 0; u < 8; ++u) v += f(w[u]);
    }
    for (; i < n; i += stride) v += f(x[i]);
    return v;
}

// Sum of squares of x[start .. end) by a 256-thread workgroup: strided per-thread sums, then a halving
// tree through scratch (256 floats).  The gradient-clipping partials of every caller use this one order.
__device__ __forceinline__ float block_sum_squares(const float* x, long long start, long long end, float* scratch) {
    scratch[threadIdx.x] = strided_sum(x, start + threadIdx.x, end, 256, [](float y) { return y * y; });
    __syncthreads();
    for (int stride = 128; stride > 0; stride >>= 1) {
        if (static_cast<int>(threadIdx.x) < stride) scratch[threadIdx.x] += scratch[threadIdx.x + stride];
        __syncthreads();
    }
    return scratch[0];
}

}  // namespace rl
