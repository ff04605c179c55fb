// Shared host/device helpers for the MI355X learner library.
//
// Error convention (mirrors robolearn/cuda/kernels.cu:70-79, 408): every
// extern "C" entry point returns 0 on success and -1 on a synchronous error,
// and leaves a message in a thread-local 512-byte buffer read through
// rl_last_error().  Run/step calls only enqueue work on the caller's HIP
// stream: they never allocate, free or synchronize, so they are legal inside
// hipStreamBeginCapture.  Plan create/destroy calls may allocate and must run
// outside capture.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>

#include <cstdarg>
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <limits>

#define RL_API extern "C" __attribute__((visibility("default")))

namespace rl {

extern thread_local char last_error[512];

struct Failure {};

inline void set_error(const char* format, ...) noexcept {
    va_list args;
    va_start(args, format);
    std::vsnprintf(last_error, sizeof(last_error), format, args);
    va_end(args);
}

inline void clear_error() noexcept { last_error[0] = '\0'; }

inline void require(bool condition, const char* message) {
    if (!condition) {
        set_error("%s", message);
        throw Failure{};
    }
}

inline void check_hip(hipError_t status, const char* operation) {
    if (status != hipSuccess) {
        set_error("%s: %s", operation, hipGetErrorString(status));
        throw Failure{};
    }
}

// Reports a launch error without clearing HIP's sticky state.
inline void check_launch(const char* operation) {
    const hipError_t status = hipPeekAtLastError();
    if (status != hipSuccess) {
        set_error("%s: %s", operation, hipGetErrorString(status));
        throw Failure{};
    }
}

inline bool aligned(const void* pointer, std::size_t bytes) noexcept {
    return reinterpret_cast<std::uintptr_t>(pointer) % bytes == 0;
}

inline hipStream_t as_stream(void* stream) noexcept { return reinterpret_cast<hipStream_t>(stream); }

// Runs body() and maps exceptions to the -1 status convention.
template <class Body>
int guarded(const char* what, Body&& body) noexcept {
    clear_error();
    try {
        body();
        return 0;
    } catch (const Failure&) {
        return -1;
    } catch (...) {
        set_error("Unexpected host error in %s.", what);
        return -1;
    }
}

template <class Body>
void* guarded_ptr(const char* what, Body&& body) noexcept {
    clear_error();
    try {
        return body();
    } catch (const Failure&) {
        return nullptr;
    } catch (...) {
        set_error("Unexpected host error in %s.", what);
        return nullptr;
    }
}

inline unsigned ceil_div(long long a, long long b) { return static_cast<unsigned>((a + b - 1) / b); }

// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------

constexpr int kWave = 64;

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// fp32 -> bf16 with round-to-nearest-even; on gfx950 this is the hardware
// conversion (v_cvt_pk_bf16_f32), two values per instruction.
__device__ __forceinline__ unsigned short f32_to_bf16_bits(float value) {
    return __builtin_bit_cast(unsigned short, static_cast<__bf16>(value));
}

// Packs (lo, hi) as two bf16 in one 32-bit word, lo in the low half.
__device__ __forceinline__ unsigned int f32x2_to_bf16x2(float lo, float hi) {
    return __builtin_bit_cast(unsigned int, __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
}

__device__ __forceinline__ float bf16_bits_to_f32(unsigned short bits) {
    return __uint_as_float(static_cast<unsigned int>(bits) << 16);
}

// fp32 -> IEEE binary16 with round-to-nearest-even (v_cvt_f16_f32 under the
// default rounding mode): subnormal results are kept, magnitudes past the
// largest finite half become infinities and NaN stays NaN.
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ unsigned short f32_to_f16_bits(float value) {
    return __builtin_bit_cast(unsigned short, static_cast<_Float16>(value));
}
__device__ __forceinline__ unsigned int f32x2_to_f16x2(float lo, float hi) {
    return __builtin_bit_cast(unsigned int, __builtin_convertvector((f32x2_t){lo, hi}, f16x2_t));
}

// DPP lane permutations within a row of 16 lanes (GCN/CDNA DPP16 controls).
constexpr int kDppXor1 = 0xB1;        // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7 - i within each 8
constexpr int kDppMirror = 0x140;     // lane i <-> 15 - i within each 16

template <int Control>
__device__ __forceinline__ float dpp(float value) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(value), Control, 0xF, 0xF, true));
}

__device__ __forceinline__ float lane_value(float value, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(value), lane));
}

// Wave-wide sum, returned to every lane.  Four DPP butterfly steps (VALU, no
// LDS round trips) leave each 16-lane row's sum in all of its lanes with
// identical bits (every step adds the same two operands in either order); the
// four row sums are then added in a fixed order.  Requires all 64 lanes active.
__device__ __forceinline__ float wave_sum(float value) {
    value += dpp<kDppXor1>(value);
    value += dpp<kDppXor2>(value);
    value += dpp<kDppHalfMirror>(value);
    value += dpp<kDppMirror>(value);
    return (lane_value(value, 0) + lane_value(value, 16)) + (lane_value(value, 32) + lane_value(value, 48));
}

__device__ __forceinline__ double wave_sum(double value) {
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) value += __shfl_xor(value, offset, kWave);
    return value;
}

__device__ __forceinline__ float wave_max(float value) {
    value = fmaxf(value, dpp<kDppXor1>(value));
    value = fmaxf(value, dpp<kDppXor2>(value));
    value = fmaxf(value, dpp<kDppHalfMirror>(value));
    value = fmaxf(value, dpp<kDppMirror>(value));
    return fmaxf(fmaxf(lane_value(value, 0), lane_value(value, 16)), fmaxf(lane_value(value, 32), lane_value(value, 48)));
}

// Fixed-order block sum for blockDim.x == Threads; the result is broadcast.
template <int Threads>
__device__ __forceinline__ float block_sum(float value, float* scratch) {
    value = wave_sum(value);
    const int wave = threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    __syncthreads();
    if (lane == 0) scratch[wave] = value;
    __syncthreads();
    float total = 0.0f;
#pragma unroll
    for (int w = 0; w < Threads / kWave; ++w) total += scratch[w];
    return total;
}

template <int Threads>
__device__ __forceinline__ double block_sum(double value, double* scratch) {
    value = wave_sum(value);
    const int wave = threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    __syncthreads();
    if (lane == 0) scratch[wave] = value;
    __syncthreads();
    double total = 0.0;
#pragma unroll
    for (int w = 0; w < Threads / kWave; ++w) total += scratch[w];
    return total;
}

}  // namespace rl
