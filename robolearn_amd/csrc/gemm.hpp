// Shared GEMM parameter block and launch entry points.
#pragma once

#include "common.hpp"

namespace rl {
namespace gemm {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef unsigned short u16x8_t __attribute__((ext_vector_type(8)));

constexpr int kThreads = 256;
constexpr int kTile = 128;

enum Epilogue : int { kNone = 0, kRelu = 1, kElu = 2 };

struct Params {
    const void* a;
    const void* b;
    float* d;            // output (or split-K workspace)
    const float* c;      // beta operand (same layout as d), may alias d
    const float* bias;   // length n, may be null
    long long lda, ldb, ldd;
    long long stride_a, stride_b, stride_d, stride_bias;
    int m, n, k;
    int batch;           // ensemble count
    int splits;          // K splits; >1 writes partial tiles into d = workspace
    int k_per_split;     // multiple of the K tile
    float beta;          // D = act(AB + bias) + beta * C (direct mode only)
    int epilogue;        // Epilogue (direct mode only)
    int a_vec, b_vec;    // 16-byte vector loads allowed
    unsigned short* d_bf16;  // optional bf16 copy of the output (direct mode only)
};

__device__ __forceinline__ float apply_epilogue(float v, int epilogue) {
    if (epilogue == 1) return v > 0.0f ? v : 0.0f;
    if (epilogue == 2) return v > 0.0f ? v : expm1f(v);
    return v;
}

// bf16 MFMA kernel family with 256x128 tiles (gemm_bf16.hip).
void launch_bf16(const Params& p, int a_bf16, int b_bf16, bool ak, bool bk, hipStream_t stream);

// 256x256-tile bf16 kernel for exactly tiling bf16 operands (gemm_bf16_big.hip).
bool big_eligible(const Params& p, int a_bf16, int b_bf16);
void launch_big(const Params& p, bool ak, bool bk, hipStream_t stream);

}  // namespace gemm
}  // namespace rl
