// One coalesced pass that fuses Adam, the unit-norm weight projection, the
// target EMA and 16-bit operand shadows over every tensor of a network (bf16
// for the fused learner plans, IEEE fp16 for the reference projection and EMA
// plans).
//
// Reference semantics:
//   Adam          torch.optim.Adam single-tensor path, as called from
//                 robolearn/flashsac/agent.py:64-65 (form 0), or the native
//                 bias-corrected form of robolearn/cuda/kernels.cu:310-337 (form 1).
//   LR schedule   warmup + cosine, robolearn/flashsac/_utils/scheduler.py:43-65,
//                 stepped after each optimizer step (agent.py:66-69, updates.py:151-153).
//   Projection    unit Linear rows (layers.py:24-29, 185-186), BN affine pairs
//                 (layers.py:57-64, 216-222), RMS scales (layers.py:76-81, 235-240),
//                 robolearn/cuda/flash_kernels.cuh:112-131.
//   EMA           target <- target + tau * (online - target), network.py:66-80.
//
// Work decomposition: one wavefront owns one projection unit (a weight row, one
// BN (weight, bias) pair, one RMS vector) or one 1024-element chunk of a plain
// tensor, so the row norm needed by the projection is a wave reduction and no
// inter-workgroup communication is needed.  Pass 1 reads p, g, m1, m2, writes
// the moments and the unprojected parameter and accumulates the row's squared
// norm; pass 2 rereads the row (resident in L2), scales it, writes it, its 16-bit
// shadow and the EMA target.  All scalar step state lives on the device, so a
// step is graph-capturable.
#include "common.hpp"
#include "reduce.hpp"

#include <algorithm>
#include <cmath>
#include <memory>
#include <vector>

namespace rl {
namespace opt {

enum Kind : int { kUnitRow = 0, kBatchNormPair = 1, kRmsScale = 2, kPlain = 3 };
constexpr int kChunk = 1024;
constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;

struct Part {
    float* p;
    const float* g;
    float* m1;
    float* m2;
    float* target;
    unsigned short* shadow;
    unsigned short* target_shadow;
};

struct Tensor {
    Part part[2];        // part[1] is the BN bias of a kBatchNormPair
    long long rows;      // projection units (rows of a unit Linear, ensemble members of BN/RMS)
    long long cols;      // elements per unit (plain: total elements, rows == 1)
    int kind;
    int vec4;
};

struct Work {
    int tensor;
    int unit;            // row, or chunk index for kPlain
};

struct Schedule {
    int enabled;
    double init, peak, end;
    double warmup, decay;
};

struct Scalars {
    float a;             // form 0: -lr / bc1          form 1: lr
    float b;             // form 0: sqrt(bc2)          form 1: 1 / bc1
    float c;             // form 1: 1 / bc2
    float pad;
};

__device__ double schedule_value(const Schedule& s, double step) {
    double value = s.end;
    if (step < s.warmup) value = s.init + (s.peak - s.init) * (step / s.warmup);
    else if (step < s.decay) {
        const double progress = (step - s.warmup) / (s.decay - s.warmup);
        value = s.end + (s.peak - s.end) * 0.5 * (1.0 + cos(M_PI * progress));
    }
    // LambdaLR scales the base (peak) rate by schedule / peak.
    return s.peak * (value / s.peak);
}

__device__ __forceinline__ void prepare_body(float* timestep, float* lr, Schedule schedule, double beta1, double beta2,
                                             int form, Scalars* out) {
    const float t = timestep[0] + 1.0f;
    timestep[0] = t;
    double lr_used = lr[0];
    if (schedule.enabled) {
        lr_used = schedule_value(schedule, static_cast<double>(t) - 1.0);
        lr[0] = static_cast<float>(schedule_value(schedule, static_cast<double>(t)));
    }
    Scalars s{};
    if (form == 0) {
        const double bc1 = 1.0 - pow(beta1, static_cast<double>(t));
        const double bc2 = 1.0 - pow(beta2, static_cast<double>(t));
        s.a = static_cast<float>(-(lr_used / bc1));
        s.b = static_cast<float>(sqrt(bc2));
    } else {
        s.a = static_cast<float>(lr_used);
        s.b = 1.0f / (1.0f - powf(static_cast<float>(beta1), t));
        s.c = 1.0f / (1.0f - powf(static_cast<float>(beta2), t));
    }
    out[0] = s;
}

__global__ void prepare(float* timestep, float* lr, Schedule schedule, double beta1, double beta2, int form,
                        const int* skip, Scalars* out) {
    if (skip && skip[0]) return;
    prepare_body(timestep, lr, schedule, beta1, beta2, form, out);
}

// The gradient sum-of-squares partials of clipping (one per 4096-element block, the order of
// rl_clip_grad_norm's partials), with the step's scalars prepared by workgroup 0 in the same launch.
__global__ __launch_bounds__(256) void sumsq_prepare(const float* g, long long n, float* partial, float* timestep,
                                                     float* lr, Schedule schedule, double beta1, double beta2,
                                                     int form, Scalars* out) {
    __shared__ float scratch[256];
    const long long start = static_cast<long long>(blockIdx.x) * 4096;
    const float total = block_sum_squares(g, start, min(n, start + 4096), scratch);
    if (threadIdx.x == 0) {
        partial[blockIdx.x] = total;
        if (blockIdx.x == 0) prepare_body(timestep, lr, schedule, beta1, beta2, form, out);
    }
}

// Dynamic loss scaling around an Adam step (robolearn/cuda/kernels.cu:356-405):
// a step whose unscaled gradients held a non-finite value is skipped and the
// scale backs off (floored at 2^-126); otherwise the step runs and the scale
// grows by growth_factor every growth_interval successful steps.
__global__ void scaled_prepare(float* timestep, float* lr, Schedule schedule, double beta1, double beta2, int form,
                               float* loss_scale, int* growth_tracker, const int* found_inf, int* step_skipped,
                               long long* attempted, long long* skipped, float growth_factor, float backoff_factor,
                               int growth_interval, Scalars* out) {
    attempted[0] += 1;
    step_skipped[0] = found_inf[0] != 0;
    if (step_skipped[0]) {
        skipped[0] += 1;
        growth_tracker[0] = 0;
        loss_scale[0] = fmaxf(loss_scale[0] * backoff_factor, 0x1p-126f);
        return;
    }
    prepare_body(timestep, lr, schedule, beta1, beta2, form, out);
    const int growth = growth_tracker[0] + 1;
    if (growth >= growth_interval) {
        const float increased = loss_scale[0] * growth_factor;
        if (isfinite(increased)) loss_scale[0] = increased;
        growth_tracker[0] = 0;
    } else {
        growth_tracker[0] = growth;
    }
}

__global__ void reset_flag(int* flag) { flag[0] = 0; }

struct StepArgs {
    const Tensor* tensors;
    const Work* work;
    int work_count;
    const Scalars* scalars;
    float beta1, beta2, one_minus_beta1, one_minus_beta2, eps, tau;
    int form, do_adam, do_project, do_ema;
    int shadow_f16;      // shadows hold IEEE fp16 (the reference projection/EMA plans) instead of bf16
    const int* skip;
    // gradient-norm clipping folded into the step (null: none): the sum-of-squares partials of the
    // gradients (one per 4096-element block), the norm bound, and where the sum of squares goes
    const float* clip_partial;
    long long clip_blocks;
    float clip_max_norm;
    float* clip_sum_squares;
};

__device__ __forceinline__ float adam_element(const StepArgs& a, const Scalars& s, float p, float g, float& m1, float& m2) {
    if (a.form == 0) {
        // exp_avg.lerp_(grad, 1 - beta1); exp_avg_sq.mul_(beta2).addcmul_(grad, grad, 1 - beta2)
        m1 = m1 + a.one_minus_beta1 * (g - m1);
        m2 = m2 * a.beta2 + a.one_minus_beta2 * g * g;
        const float denom = sqrtf(m2) / s.b + a.eps;
        return p + s.a * (m1 / denom);
    }
    m1 = a.beta1 * m1 + a.one_minus_beta1 * g;
    m2 = a.beta2 * m2 + a.one_minus_beta2 * (g * g);
    return p - s.a * ((m1 * s.b) / (sqrtf(m2 * s.c) + a.eps));
}

// The 16-bit shadow copy of one value (bf16, or IEEE fp16 for plans whose
// shadows are fp16; RNE either way), and of four as one 8-byte store (vec4
// spans start at multiples of 4 elements).
__device__ __forceinline__ unsigned short shadow_bits(const StepArgs& a, float v) {
    return a.shadow_f16 ? f32_to_f16_bits(v) : f32_to_bf16_bits(v);
}
__device__ __forceinline__ void store_shadow4(const StepArgs& a, unsigned short* dst, float4 v) {
    *reinterpret_cast<uint2*>(dst) = a.shadow_f16 ? make_uint2(f32x2_to_f16x2(v.x, v.y), f32x2_to_f16x2(v.z, v.w))
                                                  : make_uint2(f32x2_to_bf16x2(v.x, v.y), f32x2_to_bf16x2(v.z, v.w));
}

// Pass 1 over one contiguous span: optional Adam, returns the squared norm of
// the resulting parameters.
// coef scales the gradients (gradient-norm clipping); with clipping on, the scaled gradients are written
// back, as an in-place clip would leave them.
__device__ float update_span(const StepArgs& a, const Scalars& s, const Part& part, long long offset, long long length,
                             bool vec4, float coef) {
    const int lane = threadIdx.x % kWave;
    float sumsq = 0.0f;
    float* p = part.p + offset;
    if (vec4) {
        const long long n4 = length / 4;
        for (long long i = lane; i < n4; i += kWave) {
            float4 pv = reinterpret_cast<float4*>(p)[i];
            if (a.do_adam) {
                float4 gv = reinterpret_cast<const float4*>(part.g + offset)[i];
                float4 m1v = reinterpret_cast<float4*>(part.m1 + offset)[i];
                float4 m2v = reinterpret_cast<float4*>(part.m2 + offset)[i];
                if (a.clip_partial) {  // the clipped entry's grad range holds these gradients, writable
                    gv = make_float4(gv.x * coef, gv.y * coef, gv.z * coef, gv.w * coef);
                    reinterpret_cast<float4*>(const_cast<float*>(part.g) + offset)[i] = gv;
                }
                pv.x = adam_element(a, s, pv.x, gv.x, m1v.x, m2v.x);
                pv.y = adam_element(a, s, pv.y, gv.y, m1v.y, m2v.y);
                pv.z = adam_element(a, s, pv.z, gv.z, m1v.z, m2v.z);
                pv.w = adam_element(a, s, pv.w, gv.w, m1v.w, m2v.w);
                reinterpret_cast<float4*>(part.m1 + offset)[i] = m1v;
                reinterpret_cast<float4*>(part.m2 + offset)[i] = m2v;
                reinterpret_cast<float4*>(p)[i] = pv;
            }
            sumsq += pv.x * pv.x + pv.y * pv.y + pv.z * pv.z + pv.w * pv.w;
        }
    } else {
        for (long long i = lane; i < length; i += kWave) {
            float pv = p[i];
            if (a.do_adam) {
                float m1 = part.m1[offset + i];
                float m2 = part.m2[offset + i];
                float g = part.g[offset + i];
                if (a.clip_partial) {  // the clipped entry's grad range holds these gradients, writable
                    g *= coef;
                    const_cast<float*>(part.g)[offset + i] = g;
                }
                pv = adam_element(a, s, pv, g, m1, m2);
                part.m1[offset + i] = m1;
                part.m2[offset + i] = m2;
                p[i] = pv;
            }
            sumsq += pv * pv;
        }
    }
    return sumsq;
}

// Pass 2: scale (projection), shadows and EMA.  mode 0 divides by factor
// (unit rows, F.normalize), mode 1 multiplies (BN/RMS norm factors), mode 2
// leaves values unchanged.
__device__ void finish_span(const StepArgs& a, const Part& part, long long offset, long long length, bool vec4,
                            int mode, float factor) {
    const int lane = threadIdx.x % kWave;
    const bool write_p = mode != 2;
    if (!write_p && !part.shadow && !(a.do_ema && part.target)) return;
    float* p = part.p + offset;
    auto scale = [&](float v) { return mode == 0 ? v / factor : (mode == 1 ? v * factor : v); };
    auto tail = [&](long long i, float v) {
        if (part.shadow) part.shadow[offset + i] = shadow_bits(a, v);
        if (a.do_ema && part.target) {
            float t = part.target[offset + i];
            t = t + a.tau * (v - t);
            part.target[offset + i] = t;
            if (part.target_shadow) part.target_shadow[offset + i] = shadow_bits(a, t);
        }
    };
    if (vec4) {
        const long long n4 = length / 4;
        for (long long i = lane; i < n4; i += kWave) {
            float4 v = reinterpret_cast<float4*>(p)[i];
            if (write_p) {
                v.x = scale(v.x);
                v.y = scale(v.y);
                v.z = scale(v.z);
                v.w = scale(v.w);
                reinterpret_cast<float4*>(p)[i] = v;
            }
            if (a.do_ema && part.target) {
                float4 t = reinterpret_cast<float4*>(part.target + offset)[i];
                t.x = t.x + a.tau * (v.x - t.x);
                t.y = t.y + a.tau * (v.y - t.y);
                t.z = t.z + a.tau * (v.z - t.z);
                t.w = t.w + a.tau * (v.w - t.w);
                reinterpret_cast<float4*>(part.target + offset)[i] = t;
                if (part.target_shadow) store_shadow4(a, part.target_shadow + offset + 4 * i, t);
            }
            if (part.shadow) store_shadow4(a, part.shadow + offset + 4 * i, v);
        }
    } else {
        for (long long i = lane; i < length; i += kWave) {
            float v = p[i];
            if (write_p) {
                v = scale(v);
                p[i] = v;
            }
            tail(i, v);
        }
    }
}

// A unit row of up to 4 * kWave * R elements keeps its updated values in registers
// between the Adam pass and the projection pass: each parameter is read and written
// once.  The arithmetic is that of update_span and finish_span (mode 0).  R is 16
// (rows up to 4096: the 4h -> h block weights) when the plan has such rows, else 4
// (rows up to 1024), since the buffer's registers cost occupancy for short rows.
// The Adam pass of a register-resident unit row: the updated row into v, its sum of squares returned.
// The four arrays are distinct (restrict), so the compiler may issue a later element's loads ahead of
// an earlier element's moment stores instead of waiting for them.  g is written only by a clipped step
// (the clipped entry's grad range, writable); m1 and m2 are null in a plan without Adam.
template <int R>
__device__ __forceinline__ float adam_row(const StepArgs& a, const Scalars& s, const float4* __restrict__ p,
                                          float4* __restrict__ g, float4* __restrict__ m1, float4* __restrict__ m2,
                                          long long n4, float coef, float4 (&v)[R]) {
    const int lane = threadIdx.x % kWave;
    float sumsq = 0.0f;
#pragma unroll
    for (int j = 0; j < R; ++j) {
        const long long i = lane + static_cast<long long>(j) * kWave;
        if (i < n4) {
            float4 pv = p[i];
            if (a.do_adam) {
                float4 gv = g[i];
                float4 m1v = m1[i];
                float4 m2v = m2[i];
                if (a.clip_partial) {
                    gv = make_float4(gv.x * coef, gv.y * coef, gv.z * coef, gv.w * coef);
                    g[i] = gv;
                }
                pv.x = adam_element(a, s, pv.x, gv.x, m1v.x, m2v.x);
                pv.y = adam_element(a, s, pv.y, gv.y, m1v.y, m2v.y);
                pv.z = adam_element(a, s, pv.z, gv.z, m1v.z, m2v.z);
                pv.w = adam_element(a, s, pv.w, gv.w, m1v.w, m2v.w);
                m1[i] = m1v;
                m2[i] = m2v;
            }
            v[j] = pv;
            sumsq += pv.x * pv.x + pv.y * pv.y + pv.z * pv.z + pv.w * pv.w;
        }
    }
    return sumsq;
}

template <int R>
__device__ void unit_row_in_registers(const StepArgs& a, const Scalars& s, const Part& part, long long offset,
                                      long long cols, float coef) {
    constexpr int kRegRow = R;
    const int lane = threadIdx.x % kWave;
    const long long n4 = cols / 4;
    float4* p = reinterpret_cast<float4*>(part.p + offset);
    float4 v[kRegRow];
    float sumsq = adam_row<kRegRow>(a, s, p, reinterpret_cast<float4*>(const_cast<float*>(part.g) + offset),
                                    reinterpret_cast<float4*>(part.m1 + offset),
                                    reinterpret_cast<float4*>(part.m2 + offset), n4, coef, v);
    sumsq = wave_sum(sumsq);
    const float factor = fmaxf(sqrtf(sumsq), 1.0e-8f);
#pragma unroll
    for (int j = 0; j < kRegRow; ++j) {
        const long long i = lane + static_cast<long long>(j) * kWave;
        if (i < n4) {
            float4 x = v[j];
            x.x = x.x / factor;
            x.y = x.y / factor;
            x.z = x.z / factor;
            x.w = x.w / factor;
            p[i] = x;
            if (part.shadow) store_shadow4(a, part.shadow + offset + 4 * i, x);
            if (a.do_ema && part.target) {
                float4 t = reinterpret_cast<float4*>(part.target + offset)[i];
                t.x = t.x + a.tau * (x.x - t.x);
                t.y = t.y + a.tau * (x.y - t.y);
                t.z = t.z + a.tau * (x.z - t.z);
                t.w = t.w + a.tau * (x.w - t.w);
                reinterpret_cast<float4*>(part.target + offset)[i] = t;
                if (part.target_shadow) store_shadow4(a, part.target_shadow + offset + 4 * i, t);
            }
        }
    }
}

template <int R>
__global__ __launch_bounds__(kThreads) void step_kernel(StepArgs a) {
    if (a.skip && a.skip[0]) return;
    // clipping: every workgroup sums the partials in one fixed order (strided per-thread sums, then a
    // halving tree; for up to 256 partials the same sum rl_clip_grad_norm forms) and derives the same
    // coefficient; workgroup 0 publishes the sum of squares
    float coef = 1.0f;
    if (a.clip_partial) {
        __shared__ float scratch[kThreads];
        float v = 0.0f;
        for (long long i = threadIdx.x; i < a.clip_blocks; i += kThreads) v += a.clip_partial[i];
        scratch[threadIdx.x] = v;
        __syncthreads();
        for (int stride = kThreads / 2; stride > 0; stride >>= 1) {
            if (static_cast<int>(threadIdx.x) < stride) scratch[threadIdx.x] += scratch[threadIdx.x + stride];
            __syncthreads();
        }
        const float total = scratch[0];
        if (blockIdx.x == 0 && threadIdx.x == 0) a.clip_sum_squares[0] = total;
        coef = fminf(1.0f, a.clip_max_norm / (sqrtf(total) + 1.0e-6f));
    }
    const int item = static_cast<int>(blockIdx.x) * kWaves + static_cast<int>(threadIdx.x) / kWave;
    if (item >= a.work_count) return;
    const Work w = a.work[item];
    const Tensor t = a.tensors[w.tensor];
    const Scalars s = a.do_adam ? a.scalars[0] : Scalars{};
    const bool vec4 = t.vec4 != 0;
    if (t.kind == kPlain) {
        const long long offset = static_cast<long long>(w.unit) * kChunk;
        const long long length = min(static_cast<long long>(kChunk), t.cols - offset);
        update_span(a, s, t.part[0], offset, length, vec4, coef);
        finish_span(a, t.part[0], offset, length, vec4, 2, 1.0f);
        return;
    }
    const long long offset = static_cast<long long>(w.unit) * t.cols;
    if (t.kind == kUnitRow && vec4 && a.do_project && t.cols <= 4LL * kWave * R) {
        unit_row_in_registers<R>(a, s, t.part[0], offset, t.cols, coef);
        return;
    }
    float sumsq = update_span(a, s, t.part[0], offset, t.cols, vec4, coef);
    if (t.kind == kBatchNormPair) sumsq += update_span(a, s, t.part[1], offset, t.cols, vec4, coef);
    sumsq = wave_sum(sumsq);
    if (!a.do_project) {
        finish_span(a, t.part[0], offset, t.cols, vec4, 2, 1.0f);
        if (t.kind == kBatchNormPair) finish_span(a, t.part[1], offset, t.cols, vec4, 2, 1.0f);
        return;
    }
    if (t.kind == kUnitRow) {
        finish_span(a, t.part[0], offset, t.cols, vec4, 0, fmaxf(sqrtf(sumsq), 1.0e-8f));
    } else {
        const float factor = sqrtf(static_cast<float>(t.cols)) * (1.0f / sqrtf(sumsq + 1.0e-8f));
        finish_span(a, t.part[0], offset, t.cols, vec4, 1, factor);
        if (t.kind == kBatchNormPair) finish_span(a, t.part[1], offset, t.cols, vec4, 1, factor);
    }
}

// Gradient unscale and overflow check (robolearn/cuda/kernels.cu:358-376):
// g <- g * (1 / scale); found_inf is raised when a gradient, its unscaled
// value or the scale is non-finite, or the scale is not positive.  Every
// writer stores the same value 1, so the flag needs no atomic and the result
// does not depend on wave order.  Same work decomposition as step_kernel.
__device__ bool unscale_span(float* g, long long length, float inverse, bool bad_scale) {
    const int lane = threadIdx.x % kWave;
    bool bad = false;
    for (long long i = lane; i < length; i += kWave) {
        const float gradient = g[i];
        const float unscaled = gradient * inverse;
        bad = bad || !isfinite(gradient) || !isfinite(unscaled) || bad_scale;
        g[i] = unscaled;
    }
    return bad;
}

__global__ __launch_bounds__(kThreads) void unscale_kernel(const Tensor* tensors, const Work* work, int work_count,
                                                           const float* loss_scale, int* found_inf) {
    const int item = static_cast<int>(blockIdx.x) * kWaves + static_cast<int>(threadIdx.x) / kWave;
    if (item >= work_count) return;
    const Work w = work[item];
    const Tensor t = tensors[w.tensor];
    const float scale = loss_scale[0];
    const float inverse = 1.0f / scale;
    const bool bad_scale = !isfinite(scale) || !(scale > 0.0f);
    long long offset, length;
    if (t.kind == kPlain) {
        offset = static_cast<long long>(w.unit) * kChunk;
        length = min(static_cast<long long>(kChunk), t.cols - offset);
    } else {
        offset = static_cast<long long>(w.unit) * t.cols;
        length = t.cols;
    }
    bool bad = unscale_span(const_cast<float*>(t.part[0].g) + offset, length, inverse, bad_scale);
    if (t.kind == kBatchNormPair) bad = unscale_span(const_cast<float*>(t.part[1].g) + offset, length, inverse, bad_scale) || bad;
    if (bad) found_inf[0] = 1;
}

// Grouped zero of fp32 spans (robolearn/cuda/zero_kernels.cuh:38-48): one
// 256-thread workgroup per span chunk of up to kZeroChunk floats, 16-byte
// stores where the chunk start allows.
constexpr unsigned kZeroChunk = 4096;

struct ZeroBlock {
    float* pointer;
    unsigned length;
};

__global__ __launch_bounds__(kThreads) void zero_kernel(const ZeroBlock* blocks) {
    const ZeroBlock block = blocks[blockIdx.x];
    unsigned head = 0;
    if (reinterpret_cast<std::uintptr_t>(block.pointer) % 16 == 0) {
        typedef float f32x4 __attribute__((ext_vector_type(4)));
        f32x4* vectors = reinterpret_cast<f32x4*>(block.pointer);
        const unsigned count = block.length / 4;
        for (unsigned i = threadIdx.x; i < count; i += kThreads) vectors[i] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
        head = count * 4;
    }
    for (unsigned i = head + threadIdx.x; i < block.length; i += kThreads) block.pointer[i] = 0.0f;
}

struct ZeroPlan {
    ZeroBlock* blocks = nullptr;
    unsigned count = 0;
    ~ZeroPlan() {
        if (blocks) (void)hipFree(blocks);
    }
};

struct Plan {
    Tensor* tensors = nullptr;
    Work* work = nullptr;
    Scalars* scalars = nullptr;
    int work_count = 0;
    float* timestep = nullptr;
    float* lr = nullptr;
    Schedule schedule{};
    double beta1 = 0.9, beta2 = 0.999, eps = 1e-8;
    float tau = 0.0f;
    int form = 0;
    int has_adam = 0;
    int has_projection = 0;
    int has_ema = 0;
    int long_rows = 0;  // a vector unit row longer than 1024 elements: step_kernel<16>
    int shadow_f16 = 0; // shadows are IEEE fp16 (reference projection/EMA plans), else bf16
    // the lowest and one past the highest gradient element of the plan's tensors (host-side bounds, for
    // the check that a clipped step's gradient range covers them); null without gradients
    const float* grad_begin = nullptr;
    const float* grad_end = nullptr;
    // dynamic loss scaling (reference-compatible rl_adam_set_scaler); null when unused
    float* loss_scale = nullptr;
    int* growth_tracker = nullptr;
    int* found_inf = nullptr;
    int* step_skipped = nullptr;
    long long* attempted_steps = nullptr;
    long long* skipped_steps = nullptr;
    float growth_factor = 2.0f, backoff_factor = 0.5f;
    int growth_interval = 2000;

    ~Plan() {
        if (tensors) (void)hipFree(tensors);
        if (work) (void)hipFree(work);
        if (scalars) (void)hipFree(scalars);
    }
};

bool all_aligned16(const Part& part) {
    auto ok = [](const void* q) { return q == nullptr || aligned(q, 16); };
    // 16-bit copies take 8-byte stores of four elements
    auto ok8 = [](const void* q) { return q == nullptr || aligned(q, 8); };
    return ok(part.p) && ok(part.g) && ok(part.m1) && ok(part.m2) && ok(part.target) && ok8(part.shadow) &&
           ok8(part.target_shadow);
}

std::unique_ptr<Plan> build(std::vector<Tensor> tensors) {
    require(!tensors.empty(), "Optimizer plan needs at least one tensor.");
    std::vector<Work> work;
    for (std::size_t i = 0; i < tensors.size(); ++i) {
        Tensor& t = tensors[i];
        require(t.rows > 0 && t.cols > 0, "Optimizer tensors must be nonempty.");
        require(t.kind >= 0 && t.kind <= 3, "Unknown optimizer tensor kind.");
        require(t.part[0].p != nullptr, "Optimizer tensor parameters must be nonnull.");
        if (t.kind == kBatchNormPair) require(t.part[1].p != nullptr, "BN projection needs both weight and bias.");
        bool vec = t.cols % 4 == 0 && all_aligned16(t.part[0]) && (t.kind != kBatchNormPair || all_aligned16(t.part[1]));
        t.vec4 = vec ? 1 : 0;
        if (t.kind == kPlain) {
            const long long total = t.rows * t.cols;
            t.cols = total;
            t.rows = 1;
            t.vec4 = (total % 4 == 0 && all_aligned16(t.part[0])) ? 1 : 0;
            const long long chunks = (total + kChunk - 1) / kChunk;
            for (long long c = 0; c < chunks; ++c) work.push_back({static_cast<int>(i), static_cast<int>(c)});
        } else {
            for (long long r = 0; r < t.rows; ++r) work.push_back({static_cast<int>(i), static_cast<int>(r)});
        }
        require(work.size() < static_cast<std::size_t>(std::numeric_limits<int>::max() / 2), "Too many optimizer work items.");
    }
    auto plan = std::make_unique<Plan>();
    check_hip(hipMalloc(&plan->tensors, tensors.size() * sizeof(Tensor)), "Allocate optimizer tensor table");
    check_hip(hipMalloc(&plan->work, work.size() * sizeof(Work)), "Allocate optimizer work table");
    check_hip(hipMalloc(&plan->scalars, sizeof(Scalars)), "Allocate optimizer scalars");
    check_hip(hipMemcpy(plan->tensors, tensors.data(), tensors.size() * sizeof(Tensor), hipMemcpyHostToDevice),
              "Copy optimizer tensor table");
    check_hip(hipMemcpy(plan->work, work.data(), work.size() * sizeof(Work), hipMemcpyHostToDevice),
              "Copy optimizer work table");
    check_hip(hipMemset(plan->scalars, 0, sizeof(Scalars)), "Clear optimizer scalars");
    plan->work_count = static_cast<int>(work.size());
    for (const Tensor& t : tensors) {
        if (t.kind == kUnitRow && t.vec4 && t.cols > 1024) plan->long_rows = 1;
        for (int q = 0; q < (t.kind == kBatchNormPair ? 2 : 1); ++q) {
            const float* g = t.part[q].g;
            if (!g) continue;
            const float* end = g + t.rows * t.cols;
            if (!plan->grad_begin || g < plan->grad_begin) plan->grad_begin = g;
            if (!plan->grad_end || end > plan->grad_end) plan->grad_end = end;
        }
    }
    return plan;
}

// clip (optional): the gradient buffer of clipping and its partial sums, prepared by the caller's
// sumsq_prepare launch, which also ran the prepare step
struct Clip {
    const float* partial;
    long long blocks;
    float max_norm;
    float* sum_squares;
};

void step(Plan* plan, int do_adam, int do_project, int do_ema, const int* skip, hipStream_t stream,
          const Clip* clip = nullptr) {
    require(plan != nullptr, "Optimizer plan is null.");
    require(!do_adam || plan->has_adam, "This plan has no Adam state.");
    if (clip) {
        // the scalars were prepared with the clipping partials
    } else if (do_adam && plan->loss_scale) {
        require(skip == nullptr, "A plan with dynamic loss scaling takes its skip flag from the scaler.");
        hipLaunchKernelGGL(scaled_prepare, dim3(1), dim3(1), 0, stream, plan->timestep, plan->lr, plan->schedule,
                           plan->beta1, plan->beta2, plan->form, plan->loss_scale, plan->growth_tracker,
                           static_cast<const int*>(plan->found_inf), plan->step_skipped, plan->attempted_steps,
                           plan->skipped_steps, plan->growth_factor, plan->backoff_factor, plan->growth_interval,
                           plan->scalars);
        check_launch("Launch optimizer scaled prepare");
        skip = plan->step_skipped;
    } else if (do_adam) {
        hipLaunchKernelGGL(prepare, dim3(1), dim3(1), 0, stream, plan->timestep, plan->lr, plan->schedule, plan->beta1,
                           plan->beta2, plan->form, skip, plan->scalars);
        check_launch("Launch optimizer prepare");
    }
    StepArgs a{};
    a.tensors = plan->tensors;
    a.work = plan->work;
    a.work_count = plan->work_count;
    a.scalars = plan->scalars;
    a.beta1 = static_cast<float>(plan->beta1);
    a.beta2 = static_cast<float>(plan->beta2);
    a.one_minus_beta1 = static_cast<float>(1.0 - plan->beta1);
    a.one_minus_beta2 = static_cast<float>(1.0 - plan->beta2);
    a.eps = static_cast<float>(plan->eps);
    a.tau = plan->tau;
    a.form = plan->form;
    a.do_adam = do_adam;
    a.do_project = do_project;
    a.do_ema = do_ema;
    a.shadow_f16 = plan->shadow_f16;
    a.skip = skip;
    if (clip) {
        a.clip_partial = clip->partial;
        a.clip_blocks = clip->blocks;
        a.clip_max_norm = clip->max_norm;
        a.clip_sum_squares = clip->sum_squares;
    }
    if (plan->long_rows)
        hipLaunchKernelGGL(step_kernel<16>, dim3(ceil_div(plan->work_count, kWaves)), dim3(kThreads), 0, stream, a);
    else
        hipLaunchKernelGGL(step_kernel<4>, dim3(ceil_div(plan->work_count, kWaves)), dim3(kThreads), 0, stream, a);
    check_launch("Launch fused optimizer step");
}

// Gradient-norm clipping of grad[0 .. n) folded into an Adam step: one launch for the sum-of-squares
// partials and the step's scalars, one for the step with the clipped gradients.
void step_clipped(Plan* plan, int do_project, int do_ema, float* grad, long long n, float* partial,
                  float* sum_squares, float max_norm, hipStream_t stream) {
    require(plan != nullptr, "Optimizer plan is null.");
    require(plan->has_adam && !plan->loss_scale, "Clipped steps need an Adam plan without dynamic loss scaling.");
    require(grad && partial && sum_squares && n > 0 && max_norm > 0.0f,
            "Gradient-norm clipping needs buffers and a positive norm.");
    require(plan->grad_begin && plan->grad_begin >= grad && plan->grad_end <= grad + n,
            "The clipped gradient range must hold every gradient of the optimizer plan.");
    const long long blocks = (n + 4095) / 4096;
    require(blocks <= (1LL << 31) - 1, "Clipped gradient range is too large.");
    hipLaunchKernelGGL(sumsq_prepare, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, grad, n, partial,
                       plan->timestep, plan->lr, plan->schedule, plan->beta1, plan->beta2, plan->form, plan->scalars);
    check_launch("Launch clipping partials and optimizer prepare");
    const Clip clip{partial, blocks, max_norm, sum_squares};
    step(plan, 1, do_project, do_ema, nullptr, stream, &clip);
}

void unscale(Plan* plan, hipStream_t stream) {
    require(plan != nullptr && plan->loss_scale != nullptr, "Unscale requires an Adam plan with dynamic loss scaling.");
    hipLaunchKernelGGL(reset_flag, dim3(1), dim3(1), 0, stream, plan->found_inf);
    check_launch("Launch loss-scale flag reset");
    hipLaunchKernelGGL(unscale_kernel, dim3(ceil_div(plan->work_count, kWaves)), dim3(kThreads), 0, stream,
                       static_cast<const Tensor*>(plan->tensors), static_cast<const Work*>(plan->work), plan->work_count,
                       static_cast<const float*>(plan->loss_scale), plan->found_inf);
    check_launch("Launch gradient unscale");
}

}  // namespace opt
}  // namespace rl

using rl::opt::Part;
using rl::opt::Plan;
using rl::opt::Tensor;

// ---------------------------------------------------------------------------
// Fused plan (no reference counterpart; replaces the sequence CudaAdam.step ->
// CudaProjection.step -> CudaEMA.step of robolearn/warp/flashsac.py:645-649,
// 788-789, 874-876, 927-929 with one pass).
// ---------------------------------------------------------------------------
RL_API void* rl_fused_optimizer_create(std::size_t count, const int* kinds, const long long* rows,
                                       const long long* cols, void* const* params, const void* const* grads,
                                       void* const* m1, void* const* m2, void* const* targets, void* const* shadows,
                                       void* const* target_shadows, const int* partner, void* timestep,
                                       void* learning_rate, double beta1, double beta2, double eps, double tau,
                                       int form, int schedule_enabled, double lr_init, double lr_peak, double lr_end,
                                       long long warmup_steps, long long decay_steps) noexcept {
    return rl::guarded_ptr("rl_fused_optimizer_create", [&]() -> void* {
        rl::require(count && kinds && rows && cols && params, "Fused optimizer requires nonempty tensor tables.");
        rl::require(form == 0 || form == 1, "Optimizer form must be 0 (torch) or 1 (native).");
        const bool adam = grads != nullptr;
        if (adam) {
            rl::require(m1 && m2 && timestep && learning_rate, "Adam needs moments, timestep and learning rate.");
            rl::require(std::isfinite(beta1) && std::isfinite(beta2) && beta1 >= 0 && beta1 < 1 && beta2 >= 0 &&
                            beta2 < 1 && eps > 0,
                        "Adam betas must lie in [0,1) and epsilon must be positive.");
        }
        rl::require(std::isfinite(tau) && tau >= 0 && tau <= 1, "EMA tau must lie in [0, 1].");
        if (schedule_enabled)
            rl::require(lr_peak > 0 && decay_steps > 0 && warmup_steps >= 0 && warmup_steps < decay_steps,
                        "Learning-rate schedule needs positive peak and warmup < decay.");
        std::vector<Tensor> tensors;
        std::vector<bool> is_partner(count, false);
        if (partner)
            for (std::size_t i = 0; i < count; ++i)
                if (partner[i] >= 0) {
                    rl::require(static_cast<std::size_t>(partner[i]) < count, "Partner index out of range.");
                    is_partner[partner[i]] = true;
                }
        auto part_of = [&](std::size_t i) {
            Part part{};
            part.p = static_cast<float*>(params[i]);
            part.g = adam ? static_cast<const float*>(grads[i]) : nullptr;
            part.m1 = adam ? static_cast<float*>(m1[i]) : nullptr;
            part.m2 = adam ? static_cast<float*>(m2[i]) : nullptr;
            part.target = targets ? static_cast<float*>(targets[i]) : nullptr;
            part.shadow = shadows ? static_cast<unsigned short*>(shadows[i]) : nullptr;
            part.target_shadow = target_shadows ? static_cast<unsigned short*>(target_shadows[i]) : nullptr;
            if (adam) rl::require(part.g && part.m1 && part.m2, "Adam tensors must be nonnull.");
            return part;
        };
        bool has_projection = false, has_ema = false;
        for (std::size_t i = 0; i < count; ++i) {
            if (is_partner[i]) continue;
            Tensor t{};
            t.kind = kinds[i];
            t.rows = rows[i];
            t.cols = cols[i];
            t.part[0] = part_of(i);
            if (t.kind == rl::opt::kBatchNormPair) {
                rl::require(partner && partner[i] >= 0, "BN pair needs a partner bias tensor.");
                const std::size_t j = static_cast<std::size_t>(partner[i]);
                rl::require(rows[j] == rows[i] && cols[j] == cols[i], "BN weight and bias shapes differ.");
                t.part[1] = part_of(j);
            }
            has_projection = has_projection || t.kind != rl::opt::kPlain;
            has_ema = has_ema || t.part[0].target != nullptr;
            tensors.push_back(t);
        }
        auto plan = rl::opt::build(std::move(tensors));
        plan->timestep = static_cast<float*>(timestep);
        plan->lr = static_cast<float*>(learning_rate);
        plan->beta1 = beta1;
        plan->beta2 = beta2;
        plan->eps = eps;
        plan->tau = static_cast<float>(tau);
        plan->form = form;
        plan->has_adam = adam;
        plan->has_projection = has_projection;
        plan->has_ema = has_ema;
        plan->schedule.enabled = schedule_enabled;
        plan->schedule.init = lr_init;
        plan->schedule.peak = lr_peak;
        plan->schedule.end = lr_end;
        plan->schedule.warmup = static_cast<double>(warmup_steps);
        plan->schedule.decay = static_cast<double>(decay_steps);
        return plan.release();
    });
}

RL_API int rl_fused_optimizer_step(void* plan, int do_adam, int do_project, int do_ema, const void* skip,
                                   void* stream) noexcept {
    return rl::guarded("rl_fused_optimizer_step", [&] {
        rl::opt::step(static_cast<Plan*>(plan), do_adam, do_project, do_ema, static_cast<const int*>(skip),
                      rl::as_stream(stream));
    });
}

RL_API int rl_fused_optimizer_step_clipped(void* plan, int do_project, int do_ema, float* grad, long long count,
                                           float* partial, float* sum_squares, float max_norm, void* stream) noexcept {
    return rl::guarded("rl_fused_optimizer_step_clipped", [&] {
        rl::opt::step_clipped(static_cast<Plan*>(plan), do_project, do_ema, grad, count, partial, sum_squares,
                              max_norm, rl::as_stream(stream));
    });
}

RL_API int rl_fused_optimizer_destroy(void* plan) noexcept {
    rl::clear_error();
    delete static_cast<Plan*>(plan);
    return 0;
}

// ---------------------------------------------------------------------------
// Reference-compatible plans.
// ---------------------------------------------------------------------------

// robolearn/cuda/kernels.cu:760-820, 878-916: native-form Adam over a pointer
// table, device float timestep and learning rate.
RL_API void* rl_adam_create(std::size_t count, const void* const* parameters, const void* const* gradients,
                            const void* const* m1, const void* const* m2, const std::size_t* sizes, void* timestep,
                            void* learning_rate, double beta1, double beta2, double eps) noexcept {
    return rl::guarded_ptr("rl_adam_create", [&]() -> void* {
        rl::require(count && parameters && gradients && m1 && m2 && sizes && timestep && learning_rate,
                    "Adam requires nonempty host pointer tables and device step/lr buffers.");
        rl::require(std::isfinite(beta1) && std::isfinite(beta2) && std::isfinite(eps) && beta1 >= 0.0 &&
                        beta1 < 1.0 && beta2 >= 0.0 && beta2 < 1.0 && eps > 0.0,
                    "Adam betas must lie in [0,1) and epsilon must be positive.");
        std::vector<Tensor> tensors;
        for (std::size_t i = 0; i < count; ++i) {
            rl::require(parameters[i] && gradients[i] && m1[i] && m2[i] && sizes[i] > 0,
                        "Adam tensors must be nonnull and nonempty.");
            Tensor t{};
            t.kind = rl::opt::kPlain;
            t.rows = 1;
            t.cols = static_cast<long long>(sizes[i]);
            t.part[0].p = static_cast<float*>(const_cast<void*>(parameters[i]));
            t.part[0].g = static_cast<const float*>(gradients[i]);
            t.part[0].m1 = static_cast<float*>(const_cast<void*>(m1[i]));
            t.part[0].m2 = static_cast<float*>(const_cast<void*>(m2[i]));
            tensors.push_back(t);
        }
        auto plan = rl::opt::build(std::move(tensors));
        plan->timestep = static_cast<float*>(timestep);
        plan->lr = static_cast<float*>(learning_rate);
        plan->beta1 = beta1;
        plan->beta2 = beta2;
        plan->eps = eps;
        plan->form = 1;
        plan->has_adam = 1;
        return plan.release();
    });
}

RL_API int rl_adam_step(void* plan, void* stream) noexcept {
    return rl::guarded("rl_adam_step", [&] { rl::opt::step(static_cast<Plan*>(plan), 1, 0, 0, nullptr, rl::as_stream(stream)); });
}

RL_API int rl_adam_destroy(void* plan) noexcept {
    rl::clear_error();
    delete static_cast<Plan*>(plan);
    return 0;
}

// robolearn/cuda/kernels.cu:822-854: attach persistent device state for
// dynamic loss scaling.  Works on any plan with Adam state (the fused plan too).
RL_API int rl_adam_set_scaler(void* plan, void* loss_scale, void* growth_tracker, void* found_inf, void* step_skipped,
                              void* attempted_steps, void* skipped_steps, double growth_factor, double backoff_factor,
                              int growth_interval) noexcept {
    return rl::guarded("rl_adam_set_scaler", [&] {
        rl::require(plan && loss_scale && growth_tracker && found_inf && step_skipped && attempted_steps && skipped_steps,
                    "Dynamic loss scaling requires persistent device state.");
        rl::require(rl::aligned(loss_scale, alignof(float)) && rl::aligned(growth_tracker, alignof(int)) &&
                        rl::aligned(found_inf, alignof(int)) && rl::aligned(step_skipped, alignof(int)) &&
                        rl::aligned(attempted_steps, alignof(long long)) && rl::aligned(skipped_steps, alignof(long long)),
                    "Dynamic loss scaling state has invalid alignment.");
        rl::require(std::isfinite(growth_factor) && growth_factor > 1.0 && std::isfinite(backoff_factor) &&
                        backoff_factor > 0.0 && backoff_factor < 1.0 && growth_interval > 0,
                    "Dynamic scale growth/backoff/interval are invalid.");
        auto* p = static_cast<Plan*>(plan);
        rl::require(p->has_adam, "Dynamic loss scaling needs a plan with Adam state.");
        p->loss_scale = static_cast<float*>(loss_scale);
        p->growth_tracker = static_cast<int*>(growth_tracker);
        p->found_inf = static_cast<int*>(found_inf);
        p->step_skipped = static_cast<int*>(step_skipped);
        p->attempted_steps = static_cast<long long*>(attempted_steps);
        p->skipped_steps = static_cast<long long*>(skipped_steps);
        p->growth_factor = static_cast<float>(growth_factor);
        p->backoff_factor = static_cast<float>(backoff_factor);
        p->growth_interval = growth_interval;
    });
}

// robolearn/cuda/kernels.cu:856-876: clear found_inf, then unscale and check
// every gradient of the plan.  Call once after backward, before clipping/step.
RL_API int rl_adam_unscale(void* plan, void* stream) noexcept {
    return rl::guarded("rl_adam_unscale", [&] { rl::opt::unscale(static_cast<Plan*>(plan), rl::as_stream(stream)); });
}

// robolearn/cuda/zero_kernels.cuh:53-116: sorted, disjoint fp32 spans
// (lengths in floats) cleared by one launch.  The descriptor table is copied
// at creation; step only enqueues the kernel, so it is graph-capturable.
RL_API void* rl_zero_create(std::size_t count, const void* const* pointers, const std::size_t* lengths) noexcept {
    return rl::guarded_ptr("rl_zero_create", [&]() -> void* {
        using rl::opt::ZeroBlock;
        rl::require(count && pointers && lengths, "Zero plan requires nonempty host pointer/length tables.");
        std::vector<ZeroBlock> blocks;
        std::uintptr_t previous_end = 0;
        for (std::size_t i = 0; i < count; ++i) {
            const auto start = reinterpret_cast<std::uintptr_t>(pointers[i]);
            rl::require(start && rl::aligned(pointers[i], alignof(float)) && lengths[i],
                        "Zero plan requires aligned, nonempty fp32 spans.");
            rl::require(lengths[i] <= (std::numeric_limits<std::uintptr_t>::max() - start) / sizeof(float),
                        "Zero span pointer arithmetic overflows.");
            rl::require(start >= previous_end, "Zero spans must be sorted and nonoverlapping.");
            previous_end = start + lengths[i] * sizeof(float);
            const std::size_t chunks = (lengths[i] - 1) / rl::opt::kZeroChunk + 1;
            rl::require(chunks <= static_cast<std::size_t>(std::numeric_limits<int>::max()) - blocks.size(),
                        "Zero plan block count exceeds the grid limit.");
            float* base = static_cast<float*>(const_cast<void*>(pointers[i]));
            for (std::size_t offset = 0; offset < lengths[i]; offset += rl::opt::kZeroChunk) {
                const std::size_t remaining = lengths[i] - offset;
                blocks.push_back({base + offset, static_cast<unsigned>(std::min<std::size_t>(remaining, rl::opt::kZeroChunk))});
            }
        }
        auto plan = std::make_unique<rl::opt::ZeroPlan>();
        rl::check_hip(hipMalloc(&plan->blocks, blocks.size() * sizeof(ZeroBlock)), "Allocate grouped-zero descriptors");
        rl::check_hip(hipMemcpy(plan->blocks, blocks.data(), blocks.size() * sizeof(ZeroBlock), hipMemcpyHostToDevice),
                      "Copy grouped-zero descriptors");
        plan->count = static_cast<unsigned>(blocks.size());
        return plan.release();
    });
}

RL_API int rl_zero_step(void* plan, void* stream) noexcept {
    return rl::guarded("rl_zero_step", [&] {
        rl::require(plan != nullptr, "Zero plan is null.");
        const auto* p = static_cast<const rl::opt::ZeroPlan*>(plan);
        hipLaunchKernelGGL(rl::opt::zero_kernel, dim3(p->count), dim3(rl::opt::kThreads), 0, rl::as_stream(stream),
                           static_cast<const rl::opt::ZeroBlock*>(p->blocks));
        rl::check_launch("Launch grouped zero");
    });
}

RL_API int rl_zero_destroy(void* plan) noexcept {
    rl::clear_error();
    delete static_cast<rl::opt::ZeroPlan*>(plan);
    return 0;
}

// robolearn/cuda/flash_kernels.cuh:398-445: one descriptor per unit row
// (kind 0), BN (weight, bias) pair (kind 1) or RMS scale (kind 2); optional
// shadows receive the IEEE fp16 (RNE) copy of the projected first vector, as
// the reference's __half shadows (flash_kernels.cuh:128).
static void* create_projection(std::size_t count, const void* const* first, const void* const* second,
                               const std::size_t* lengths, const int* kinds, const void* const* shadows) {
    rl::require(count && first && lengths && kinds, "Projection requires nonempty host tables.");
    std::vector<Tensor> tensors;
    for (std::size_t i = 0; i < count; ++i) {
        rl::require(first[i] && lengths[i] > 0 && kinds[i] >= 0 && kinds[i] <= 2,
                    "Projection descriptors need nonnull rows, positive lengths and kinds 0..2.");
        rl::require(kinds[i] != 1 || (second && second[i]), "BN projection needs a bias vector.");
        Tensor t{};
        t.kind = kinds[i];
        t.rows = 1;
        t.cols = static_cast<long long>(lengths[i]);
        t.part[0].p = static_cast<float*>(const_cast<void*>(first[i]));
        t.part[0].shadow = shadows ? static_cast<unsigned short*>(const_cast<void*>(shadows[i])) : nullptr;
        if (kinds[i] == 1) t.part[1].p = static_cast<float*>(const_cast<void*>(second[i]));
        tensors.push_back(t);
    }
    auto plan = rl::opt::build(std::move(tensors));
    plan->has_projection = 1;
    plan->shadow_f16 = 1;
    return plan.release();
}

RL_API void* rl_flash_projection_create(std::size_t count, const void* const* first, const void* const* second,
                                        const std::size_t* lengths, const int* kinds) noexcept {
    return rl::guarded_ptr("rl_flash_projection_create",
                           [&]() -> void* { return create_projection(count, first, second, lengths, kinds, nullptr); });
}

RL_API void* rl_flash_projection_create_with_shadows(std::size_t count, const void* const* first,
                                                     const void* const* second, const std::size_t* lengths,
                                                     const int* kinds, const void* const* shadows) noexcept {
    return rl::guarded_ptr("rl_flash_projection_create_with_shadows",
                           [&]() -> void* { return create_projection(count, first, second, lengths, kinds, shadows); });
}

RL_API int rl_flash_projection_step(void* plan, void* stream) noexcept {
    return rl::guarded("rl_flash_projection_step",
                       [&] { rl::opt::step(static_cast<Plan*>(plan), 0, 1, 0, nullptr, rl::as_stream(stream)); });
}

RL_API int rl_flash_projection_destroy(void* plan) noexcept {
    rl::clear_error();
    delete static_cast<Plan*>(plan);
    return 0;
}

// robolearn/cuda/flash_kernels.cuh:447-498: target = (1 - tau) target + tau source;
// optional shadows receive the IEEE fp16 (RNE) copy of the new target
// (flash_kernels.cuh:138).
static void* create_ema(std::size_t count, const void* const* source, const void* const* target,
                        const std::size_t* lengths, float tau, const void* const* shadows) {
    rl::require(count && source && target && lengths, "EMA requires nonempty host tables.");
    rl::require(std::isfinite(tau) && tau >= 0.0f && tau <= 1.0f, "EMA tau must lie in [0, 1].");
    std::vector<Tensor> tensors;
    for (std::size_t i = 0; i < count; ++i) {
        rl::require(source[i] && target[i] && lengths[i] > 0, "EMA descriptors need nonnull buffers.");
        Tensor t{};
        t.kind = rl::opt::kPlain;
        t.rows = 1;
        t.cols = static_cast<long long>(lengths[i]);
        t.part[0].p = static_cast<float*>(const_cast<void*>(source[i]));
        t.part[0].target = static_cast<float*>(const_cast<void*>(target[i]));
        t.part[0].target_shadow = shadows ? static_cast<unsigned short*>(const_cast<void*>(shadows[i])) : nullptr;
        tensors.push_back(t);
    }
    auto plan = rl::opt::build(std::move(tensors));
    plan->tau = tau;
    plan->has_ema = 1;
    plan->shadow_f16 = 1;
    return plan.release();
}

RL_API void* rl_flash_ema_create(std::size_t count, const void* const* source, const void* const* target,
                                 const std::size_t* lengths, float tau) noexcept {
    return rl::guarded_ptr("rl_flash_ema_create",
                           [&]() -> void* { return create_ema(count, source, target, lengths, tau, nullptr); });
}

RL_API void* rl_flash_ema_create_with_shadows(std::size_t count, const void* const* source, const void* const* target,
                                              const std::size_t* lengths, float tau,
                                              const void* const* shadows) noexcept {
    return rl::guarded_ptr("rl_flash_ema_create_with_shadows",
                           [&]() -> void* { return create_ema(count, source, target, lengths, tau, shadows); });
}

RL_API int rl_flash_ema_step(void* plan, void* stream) noexcept {
    return rl::guarded("rl_flash_ema_step",
                       [&] { rl::opt::step(static_cast<Plan*>(plan), 0, 0, 1, nullptr, rl::as_stream(stream)); });
}

RL_API int rl_flash_ema_destroy(void* plan) noexcept {
    rl::clear_error();
    delete static_cast<Plan*>(plan);
    return 0;
}
