// Categorical value head, two-hot TD target projection and cross-entropy.
//
// Reference semantics:
//   head      EnsembleCategoricalValue, robolearn/flashsac/layers.py:275-303:
//             lp = log_softmax(x W^T + b), Q = sum_j exp(lp_j) z_j with
//             z = linspace(min_v, max_v, K).
//   min-Q     _select_min_q_log_probs, robolearn/flashsac/updates.py:19-31
//             (argmin over critics, first critic on a tie).
//   target    _compute_categorical_td_target, updates.py:34-80:
//             v_j = r + (gamma * (z_j - alpha logpi')) * (1 - done), clamp,
//             b = (v - min_v) / width, two-hot split with scatter_add_ over
//             j in order (all lower-bin adds, then all upper-bin adds).
//   CE        updates.py:254-257: loss = mean over (critic, row) of
//             -sum_j t_j lp_j on the current-observation half.
//   Native    robolearn/cuda/categorical_kernels.cuh:35-176.
//
// One wavefront owns one row (K <= 512, at most 8 bins per lane).  The
// projection is deterministic and reproduces the reference's per-bin summation
// order: every lane owns its target bins and walks the source bins in order,
// so no atomics are involved.
#include "common.hpp"

#include <cmath>

namespace rl {
namespace cat {

constexpr int kMaxBins = 512;
constexpr int kPerLane = kMaxBins / kWave;
constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;

struct RowSoftmax {
    float lp[kPerLane];
    float q;
};

// log_softmax of one row held as kPerLane values per lane, plus expectation.
__device__ __forceinline__ void log_softmax_row(const float* logits, const float* bias, const float* support, int bins,
                                                float* lp, float& q) {
    const int lane = threadIdx.x % kWave;
    float x[kPerLane];
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < kPerLane; ++i) {
        const int j = lane + i * kWave;
        x[i] = j < bins ? logits[j] + (bias ? bias[j] : 0.0f) : -INFINITY;
        m = fmaxf(m, x[i]);
    }
    m = wave_max(m);
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < kPerLane; ++i) {
        const int j = lane + i * kWave;
        if (j < bins) s += expf(x[i] - m);
    }
    const float lse = logf(wave_sum(s));
    float e = 0.0f;
#pragma unroll
    for (int i = 0; i < kPerLane; ++i) {
        const int j = lane + i * kWave;
        lp[i] = x[i] - m - lse;
        if (j < bins) e += expf(lp[i]) * support[j];
    }
    q = wave_sum(e);
}

// Head forward over ensemble x rows: lp (optional) and Q.
__global__ __launch_bounds__(kThreads) void head_forward(const float* logits, const float* bias, long long bias_stride,
                                                         const float* support, float* log_probs, float* values,
                                                         long long rows, int bins, int ensemble) {
    const long long row = blockIdx.x * static_cast<long long>(kWaves) + threadIdx.x / kWave;
    if (row >= rows * ensemble) return;
    const int e = static_cast<int>(row / rows);
    const int lane = threadIdx.x % kWave;
    float lp[kPerLane];
    float q;
    log_softmax_row(logits + row * bins, bias ? bias + e * bias_stride : nullptr, support, bins, lp, q);
    if (log_probs) {
#pragma unroll
        for (int i = 0; i < kPerLane; ++i) {
            const int j = lane + i * kWave;
            if (j < bins) log_probs[row * bins + j] = lp[i];
        }
    }
    if (lane == 0) values[row] = q;
}

// dlogits_j (+)= dlp_j + p_j (dq z_j - sum_k (dlp_k + dq p_k z_k)), from log-probs.
__global__ __launch_bounds__(kThreads) void head_backward(const float* log_probs, const float* support,
                                                          const float* dlog_probs, const float* dvalues, float* draw,
                                                          float* scratch, long long rows, int bins, int accumulate) {
    const long long row = blockIdx.x * static_cast<long long>(kWaves) + threadIdx.x / kWave;
    if (row >= rows) return;
    const int lane = threadIdx.x % kWave;
    const float dq = dvalues ? dvalues[row] : 0.0f;
    const float* lp = log_probs + row * bins;
    float total = 0.0f;
    for (int j = lane; j < bins; j += kWave)
        total += (dlog_probs ? dlog_probs[row * bins + j] : 0.0f) + dq * expf(lp[j]) * support[j];
    total = wave_sum(total);
    for (int j = lane; j < bins; j += kWave) {
        const float p = expf(lp[j]);
        const float g = (dlog_probs ? dlog_probs[row * bins + j] : 0.0f) + p * (dq * support[j] - total);
        if (draw) draw[row * bins + j] = (accumulate ? draw[row * bins + j] : 0.0f) + g;
        if (scratch) scratch[row * bins + j] = g;
    }
}

// Q-gradient through a head given raw logits (actor phase): dlogits = dq p (z - Q).
__global__ __launch_bounds__(kThreads) void head_backward_q(const float* logits, const float* bias,
                                                            long long bias_stride, const float* support,
                                                            const float* dvalues, float* dlogits,
                                                            unsigned short* dlogits_bf16, long long rows, int bins,
                                                            int ensemble) {
    const long long row = blockIdx.x * static_cast<long long>(kWaves) + threadIdx.x / kWave;
    if (row >= rows * ensemble) return;
    const int e = static_cast<int>(row / rows);
    const int lane = threadIdx.x % kWave;
    float lp[kPerLane];
    float q;
    log_softmax_row(logits + row * bins, bias ? bias + e * bias_stride : nullptr, support, bins, lp, q);
    const float dq = dvalues[row];
#pragma unroll
    for (int i = 0; i < kPerLane; ++i) {
        const int j = lane + i * kWave;
        if (j < bins) {
            const float g = dq * expf(lp[i]) * (support[j] - q);
            if (dlogits) dlogits[row * bins + j] = g;
            if (dlogits_bf16) dlogits_bf16[row * bins + j] = f32_to_bf16_bits(g);
        }
    }
}

struct TargetArgs {
    const float* support;
    const float* reward;
    const float* terminated;
    const float* discount;
    const float* next_log_probs;
    const float* alpha;
    float min_v, max_v, width;
    int bins;
};

// Two-hot projection of one row's selected probabilities, in the reference's
// scatter order.  probs[i] holds p_j for j = lane + i * 64.  Returns t in the
// same layout.  lds must hold 4 * bins floats for this wave.
__device__ __forceinline__ void project_row(const TargetArgs& a, long long row, const float* probs, float* t,
                                            float* lds) {
    const int lane = threadIdx.x % kWave;
    const int bins = a.bins;
    float* lower_idx = lds;
    float* upper_idx = lds + bins;
    float* lower_mass = lds + 2 * bins;
    float* upper_mass = lds + 3 * bins;
    const float entropy = a.alpha[0] * a.next_log_probs[row];
    const float r = a.reward[row];
    const float g = a.discount[row];
    const float not_done = 1.0f - a.terminated[row];
#pragma unroll
    for (int i = 0; i < kPerLane; ++i) {
        const int j = lane + i * kWave;
        if (j < bins) {
            const float z = a.support ? a.support[j] : a.min_v + static_cast<float>(j) * a.width;
            float v = r + (g * (z - entropy)) * not_done;
            v = fminf(fmaxf(v, a.min_v), a.max_v);
            const float b = (v - a.min_v) / a.width;
            int lower = static_cast<int>(floorf(b));
            lower = min(max(lower, 0), bins - 1);
            const int upper = min(lower + 1, bins - 1);
            const float frac = b - static_cast<float>(lower);
            lower_idx[j] = static_cast<float>(lower);
            upper_idx[j] = static_cast<float>(upper);
            lower_mass[j] = probs[i] * (1.0f - frac);
            upper_mass[j] = probs[i] * frac;
        }
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int i = 0; i < kPerLane; ++i) t[i] = 0.0f;
    for (int j = 0; j < bins; ++j) {
        const int lj = static_cast<int>(lower_idx[j]);
        const float mj = lower_mass[j];
#pragma unroll
        for (int i = 0; i < kPerLane; ++i)
            if (lj == lane + i * kWave) t[i] += mj;
    }
    for (int j = 0; j < bins; ++j) {
        const int uj = static_cast<int>(upper_idx[j]);
        const float mj = upper_mass[j];
#pragma unroll
        for (int i = 0; i < kPerLane; ++i)
            if (uj == lane + i * kWave) t[i] += mj;
    }
}

// Fused target + cross-entropy for one row i < B:
//   target critic (ensemble 2) logits of the next-observation rows -> min-Q
//   selection -> two-hot target; online critic logits of the current rows ->
//   loss rows and dlogits = scale * (p * sum(t) - t) for both members.
__global__ __launch_bounds__(kThreads) void td_cross_entropy(TargetArgs a, const float* target_logits,
                                                             const float* target_bias, long long target_rows,
                                                             const float* online_logits, const float* online_bias,
                                                             long long online_rows, long long batch, float scale,
                                                             float* target_out, float* dlogits,
                                                             unsigned short* dlogits_bf16, float* loss_rows,
                                                             float* entropy_rows, float* q_next) {
    __shared__ float lds[kWaves][4 * kMaxBins];
    const int wave = threadIdx.x / kWave;
    const long long row = blockIdx.x * static_cast<long long>(kWaves) + wave;
    if (row >= batch) return;
    const int lane = threadIdx.x % kWave;
    const int bins = a.bins;
    float lp0[kPerLane], lp1[kPerLane];
    float q0, q1;
    log_softmax_row(target_logits + row * bins, target_bias, a.support, bins, lp0, q0);
    log_softmax_row(target_logits + (target_rows + row) * bins, target_bias ? target_bias + bins : nullptr, a.support,
                    bins, lp1, q1);
    const bool second = q1 < q0;
    float probs[kPerLane];
#pragma unroll
    for (int i = 0; i < kPerLane; ++i) probs[i] = expf(second ? lp1[i] : lp0[i]);
    float t[kPerLane];
    project_row(a, row, probs, t, lds[wave]);
    float tsum = 0.0f;
#pragma unroll
    for (int i = 0; i < kPerLane; ++i)
        if (lane + i * kWave < bins) tsum += t[i];
    tsum = wave_sum(tsum);
    if (target_out) {
#pragma unroll
        for (int i = 0; i < kPerLane; ++i) {
            const int j = lane + i * kWave;
            if (j < bins) target_out[row * bins + j] = t[i];
        }
    }
    for (int member = 0; member < 2; ++member) {
        const long long orow = member * online_rows + row;
        float lp[kPerLane];
        float q;
        log_softmax_row(online_logits + orow * bins, online_bias ? online_bias + member * bins : nullptr, a.support,
                        bins, lp, q);
        float ce = 0.0f;
#pragma unroll
        for (int i = 0; i < kPerLane; ++i) {
            const int j = lane + i * kWave;
            if (j < bins) {
                ce -= t[i] * lp[i];
                const float g = scale * (expf(lp[i]) * tsum - t[i]);
                if (dlogits) dlogits[orow * bins + j] = g;
                if (dlogits_bf16) dlogits_bf16[orow * bins + j] = f32_to_bf16_bits(g);
            }
        }
        ce = wave_sum(ce);
        if (lane == 0) loss_rows[member * batch + row] = ce;
    }
    if (lane == 0) {
        entropy_rows[row] = a.alpha[0] * a.next_log_probs[row];
        if (q_next) {
            q_next[row] = q0;
            q_next[batch + row] = q1;
        }
    }
}

// Reference-compatible target kernel (categorical_kernels.cuh:87-114): q is
// [2, 2B], log_probs [2, 2B, K]; the next-observation half is used.  The
// maximum entropy bonus is an order-independent atomic float maximum, so the
// result stays deterministic.
__device__ __forceinline__ void atomic_max_float(float* address, float value) {
    unsigned int* bits = reinterpret_cast<unsigned int*>(address);
    unsigned int old = __hip_atomic_load(bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    while (__uint_as_float(old) < value) {
        const unsigned int expected = old;
        old = atomicCAS(bits, expected, __float_as_uint(value));
        if (old == expected) break;
    }
}

__global__ __launch_bounds__(kThreads) void project_target(TargetArgs a, const float* q, const float* log_probs,
                                                           long long batch, float* target, float* maximum_entropy) {
    __shared__ float lds[kWaves][4 * kMaxBins];
    const int wave = threadIdx.x / kWave;
    const long long row = blockIdx.x * static_cast<long long>(kWaves) + wave;
    if (row >= batch) return;
    const int lane = threadIdx.x % kWave;
    const int bins = a.bins;
    const int selected = q[3 * batch + row] < q[batch + row] ? 1 : 0;
    const float* src = log_probs + (static_cast<long long>(selected) * (2 * batch) + batch + row) * bins;
    float probs[kPerLane];
#pragma unroll
    for (int i = 0; i < kPerLane; ++i) {
        const int j = lane + i * kWave;
        probs[i] = j < bins ? expf(src[j]) : 0.0f;
    }
    float t[kPerLane];
    project_row(a, row, probs, t, lds[wave]);
#pragma unroll
    for (int i = 0; i < kPerLane; ++i) {
        const int j = lane + i * kWave;
        if (j < bins) target[row * bins + j] = t[i];
    }
    if (lane == 0) atomic_max_float(maximum_entropy, a.alpha[0] * a.next_log_probs[row]);
}

// Fixed-order single-workgroup reductions of a vector: op 0 sum * scale,
// op 1 max.  Writes out[0].
__global__ __launch_bounds__(1024) void reduce_vector(const float* x, long long n, float scale, int op, float* out) {
    __shared__ float part[1024];
    float v = op == 1 ? -INFINITY : 0.0f;
    for (long long i = threadIdx.x; i < n; i += blockDim.x) v = op == 1 ? fmaxf(v, x[i]) : v + x[i];
    part[threadIdx.x] = v;
    __syncthreads();
    for (int s = blockDim.x / 2; s > 0; s >>= 1) {
        if (static_cast<int>(threadIdx.x) < s)
            part[threadIdx.x] = op == 1 ? fmaxf(part[threadIdx.x], part[threadIdx.x + s]) : part[threadIdx.x] + part[threadIdx.x + s];
        __syncthreads();
    }
    if (threadIdx.x == 0) out[0] = op == 1 ? part[0] : part[0] * scale;
}

}  // namespace cat

void reduce_vector(const float* x, long long n, float scale, int op, float* out, hipStream_t stream) {
    require(x && out && n > 0, "Reduction needs a nonempty vector and an output.");
    require(op == 0 || op == 1, "Reduction op must be 0 (scaled sum) or 1 (max).");
    hipLaunchKernelGGL(cat::reduce_vector, dim3(1), dim3(1024), 0, stream, x, n, scale, op, out);
    check_launch("Launch vector reduction");
}

}  // namespace rl

using rl::cat::kMaxBins;

RL_API int rl_reduce(const float* x, long long n, float scale, int op, float* out, void* stream) noexcept {
    return rl::guarded("rl_reduce", [&] { rl::reduce_vector(x, n, scale, op, out, rl::as_stream(stream)); });
}

RL_API int rl_categorical_head_forward(const float* logits, const float* bias, long long bias_stride,
                                       const float* support, float* log_probs, float* values, long long rows,
                                       int bins, int ensemble, void* stream) noexcept {
    return rl::guarded("rl_categorical_head_forward", [&] {
        rl::require(logits && support && values && rows > 0 && bins >= 2 && bins <= kMaxBins && ensemble > 0,
                    "Categorical head needs logits, support, values and 2..512 bins.");
        hipLaunchKernelGGL(rl::cat::head_forward, dim3(rl::ceil_div(rows * ensemble, rl::cat::kWaves)),
                           dim3(rl::cat::kThreads), 0, rl::as_stream(stream), logits, bias, bias_stride, support,
                           log_probs, values, rows, bins, ensemble);
        rl::check_launch("Launch categorical head forward");
    });
}

RL_API int rl_categorical_head_backward_q(const float* logits, const float* bias, long long bias_stride,
                                          const float* support, const float* dvalues, float* dlogits,
                                          void* dlogits_bf16, long long rows, int bins, int ensemble,
                                          void* stream) noexcept {
    return rl::guarded("rl_categorical_head_backward_q", [&] {
        rl::require(logits && support && dvalues && (dlogits || dlogits_bf16) && rows > 0 && bins >= 2 &&
                        bins <= kMaxBins,
                    "Categorical Q backward needs logits, support, dvalues, an output and 2..512 bins.");
        hipLaunchKernelGGL(rl::cat::head_backward_q, dim3(rl::ceil_div(rows * ensemble, rl::cat::kWaves)),
                           dim3(rl::cat::kThreads), 0, rl::as_stream(stream), logits, bias, bias_stride, support,
                           dvalues, dlogits, static_cast<unsigned short*>(dlogits_bf16), rows, bins, ensemble);
        rl::check_launch("Launch categorical Q backward");
    });
}

RL_API int rl_categorical_td_cross_entropy(const float* target_logits, const float* target_bias,
                                           long long target_rows, const float* online_logits,
                                           const float* online_bias, long long online_rows, const float* support,
                                           const float* reward, const float* terminated, const float* discount,
                                           const float* next_log_probs, const float* alpha, float min_v, float max_v,
                                           long long batch, int bins, float scale, float* target_out, float* dlogits,
                                           void* dlogits_bf16, float* loss_rows, float* entropy_rows, float* q_next,
                                           void* stream) noexcept {
    return rl::guarded("rl_categorical_td_cross_entropy", [&] {
        rl::require(target_logits && online_logits && support && reward && terminated && discount && next_log_probs &&
                        alpha && (dlogits || dlogits_bf16) && loss_rows && entropy_rows,
                    "TD cross-entropy needs every input and output buffer.");
        rl::require(batch > 0 && bins >= 2 && bins <= kMaxBins && min_v < max_v, "TD cross-entropy needs 2..512 bins.");
        rl::require(target_rows >= batch && online_rows >= batch, "Member row strides must cover the batch.");
        rl::cat::TargetArgs a{support, reward, terminated, discount, next_log_probs, alpha, min_v, max_v,
                              static_cast<float>((static_cast<double>(max_v) - min_v) / (bins - 1)), bins};
        hipLaunchKernelGGL(rl::cat::td_cross_entropy, dim3(rl::ceil_div(batch, rl::cat::kWaves)),
                           dim3(rl::cat::kThreads), 0, rl::as_stream(stream), a, target_logits, target_bias,
                           target_rows, online_logits, online_bias, online_rows, batch, scale, target_out, dlogits,
                           static_cast<unsigned short*>(dlogits_bf16), loss_rows, entropy_rows, q_next);
        rl::check_launch("Launch TD cross-entropy");
    });
}

// ---------------------------------------------------------------------------
// Reference-compatible entry points (categorical_kernels.cuh:126-176).
// ---------------------------------------------------------------------------
RL_API int rl_flash_categorical_forward(const void* raw, const void* bias, const void* support, void* log_probs,
                                        void* values, int batch, int bins, void* stream) noexcept {
    return rl::guarded("rl_flash_categorical_forward", [&] {
        rl::require(raw && bias && support && log_probs && values && batch >= 1 && bins >= 2 && bins <= kMaxBins,
                    "Categorical forward requires nonempty FP32 buffers and 2..512 bins.");
        hipLaunchKernelGGL(rl::cat::head_forward, dim3(rl::ceil_div(batch, rl::cat::kWaves)), dim3(rl::cat::kThreads),
                           0, rl::as_stream(stream), static_cast<const float*>(raw), static_cast<const float*>(bias),
                           0LL, static_cast<const float*>(support), static_cast<float*>(log_probs),
                           static_cast<float*>(values), static_cast<long long>(batch), bins, 1);
        rl::check_launch("Launch categorical forward");
    });
}

// Scratch receives the per-row logit gradients (batch x bins) whenever dbias
// is requested; the bias gradient is accumulated from it in fixed row order.
RL_API int rl_flash_categorical_backward(const void* log_probs, const void* support, const void* dlog_probs,
                                         const void* dvalues, void* scratch, void* draw, void* dbias, int batch,
                                         int bins, void* stream) noexcept {
    return rl::guarded("rl_flash_categorical_backward", [&] {
        rl::require(log_probs && support && (draw || dbias) && (!dbias || scratch) && batch >= 1 && bins >= 2,
                    "Categorical backward requires FP32 buffers, gradients and valid dimensions.");
        const hipStream_t st = rl::as_stream(stream);
        hipLaunchKernelGGL(rl::cat::head_backward, dim3(rl::ceil_div(batch, rl::cat::kWaves)), dim3(rl::cat::kThreads),
                           0, st, static_cast<const float*>(log_probs), static_cast<const float*>(support),
                           static_cast<const float*>(dlog_probs), static_cast<const float*>(dvalues),
                           static_cast<float*>(draw), dbias ? static_cast<float*>(scratch) : nullptr,
                           static_cast<long long>(batch), bins, 1);
        rl::check_launch("Launch categorical backward");
    });
    // dbias accumulation is issued by rl_bias_grad on the scratch rows.
}

RL_API int rl_flash_categorical_target(const void* q, const void* log_probs, const void* reward,
                                       const void* terminated, const void* discount, const void* next_log_probs,
                                       const void* alpha, void* target, void* maximum_entropy, int batch, int bins,
                                       float min_v, float max_v, void* stream) noexcept {
    return rl::guarded("rl_flash_categorical_target", [&] {
        rl::require(q && log_probs && reward && terminated && discount && next_log_probs && alpha && target &&
                        maximum_entropy && batch >= 1 && bins >= 2 && bins <= kMaxBins && min_v < max_v,
                    "Categorical target requires FP32 buffers, valid support and 2..512 bins.");
        // Support min_v + j * width, as the reference kernel builds it.
        rl::cat::TargetArgs a{nullptr, static_cast<const float*>(reward), static_cast<const float*>(terminated),
                              static_cast<const float*>(discount), static_cast<const float*>(next_log_probs),
                              static_cast<const float*>(alpha), min_v, max_v, (max_v - min_v) / static_cast<float>(bins - 1),
                              bins};
        hipLaunchKernelGGL(rl::cat::project_target, dim3(rl::ceil_div(batch, rl::cat::kWaves)),
                           dim3(rl::cat::kThreads), 0, rl::as_stream(stream), a, static_cast<const float*>(q),
                           static_cast<const float*>(log_probs), static_cast<long long>(batch),
                           static_cast<float*>(target), static_cast<float*>(maximum_entropy));
        rl::check_launch("Launch categorical target");
    });
}
