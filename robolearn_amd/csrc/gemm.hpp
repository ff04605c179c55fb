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

// kEluGrad (fp32 mode only): D = (A B) * elu'(C), where C holds the ELU
// outputs y and elu'(z) = 1 for y > 0, y + 1 otherwise (the input-gradient
// product of an ELU layer with the activation backward fused in).
enum Epilogue : int { kNone = 0, kRelu = 1, kElu = 2, kEluGrad = 3 };

__device__ __forceinline__ float elu_grad_from_output(float y) { return y > 0.0f ? 1.0f : y + 1.0f; }

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
    unsigned short* d_bf16;  // optional bf16 copy of the output (direct mode only; the only output when d is null)
    float* moments;      // optional per-256-row-chunk (mean, M2) of D: [batch][m / 256][2][n]
    int out_vec;         // 16-byte output stores allowed (n, ldd, strides multiple of 4; aligned outputs)
    float* a_sums;       // optional sum over this split's K of each row of op(A): [splits][batch][m] (fp32 family)
    long long sums_stride;  // direct mode: elements between batch members of a_sums
};

// Wave-local LDS fence: this wave's LDS operations are complete and the
// compiler may not move memory accesses across it.  Enough for LDS regions
// that only this wave touches (LDS executes a wave's operations in order).
__device__ __forceinline__ void lds_fence() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt unconstrained
    asm volatile("" ::: "memory");
}

__device__ __forceinline__ float apply_epilogue(float v, int epilogue) {
    if (epilogue == 1) return v > 0.0f ? v : 0.0f;
    if (epilogue == 2) return v > 0.0f ? v : expm1f(v);
    return v;
}

// bf16 MFMA kernel family with 256x128 tiles (gemm_bf16.hip).
void launch_bf16(const Params& p, int a_bf16, int b_bf16, bool ak, bool bk, hipStream_t stream);
// The same tiles on IEEE fp16 operands (a_f16 / b_f16: 16-bit fp16 storage,
// else fp32 rounded to fp16 on load).
void launch_f16(const Params& p, int a_f16, int b_f16, bool ak, bool bk, hipStream_t stream);

// 256x256-tile bf16 kernel for exactly tiling bf16 operands (gemm_bf16_big.hip).
bool big_eligible(const Params& p, int a_bf16, int b_bf16);
void launch_big(const Params& p, bool ak, bool bk, hipStream_t stream);

}  // namespace gemm

// Row-major batched GEMM with optional split-K, bf16 copy and output column
// moments (gemm.hip); the argument contract is rl_gemm's.
int run_gemm(int mode, int a_bf16, int b_bf16, int a_kcontig, int b_kcontig, int m, int n, int k, int batch,
             const void* a, long long lda, long long stride_a, const void* b, long long ldb, long long stride_b,
             const float* c, float* d, long long ldd, long long stride_d, const float* bias, long long stride_bias,
             float beta, int epilogue, int splits, float* workspace, std::size_t workspace_bytes, hipStream_t stream,
             unsigned short* d_bf16, float* moments, float* a_sums);

// Per-256-row-chunk column moments of a row-major [ensemble][rows][channels]
// fp32 (or, x_bf16, bf16) tensor into partial[e][chunk][2][channels] (norm.hip).
void bn_chunk_moments(int ensemble, const void* x, int x_bf16, long long x_stride, float* partial, int rows,
                      int channels, hipStream_t stream);

}  // namespace rl
