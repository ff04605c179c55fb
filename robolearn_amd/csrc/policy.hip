// Tanh-Gaussian policy head, actor/temperature objectives, replay sampling
// and gather, counter-based random numbers and small glue kernels.
//
// Reference semantics:
//   policy head  NormalTanhPolicy, robolearn/flashsac/layers.py:116-166:
//                log_std = -10 + 6 (1 + tanh(raw)), std = exp(log_std),
//                raw_a = mean + std eps, a = tanh(raw_a),
//                log pi = sum_j Normal(mean, std).log_prob(raw_a)
//                         - 2 (ln 2 - raw_a - softplus(-2 raw_a))
//                (robolearn/flashsac/_utils/distribution.py:12-19).
//   actor loss   robolearn/flashsac/updates.py:105-137 (torch.minimum splits
//                its derivative equally at ties, as robolearn/warp/flashsac.py:140-145).
//   temperature  updates.py:297-326.
//   replay       TorchUniformBuffer.sample, robolearn/flashsac/replay.py:179-194.
//
// Random numbers: Philox-4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random
// numbers: as easy as 1, 2, 3", SC 2011) keyed by a 64-bit seed, with the
// counter built from (element block, device draw counter, stream id).  Normal
// variates use the Box-Muller transform.  The draw counter lives in device
// memory and is advanced by a kernel, so captured graphs draw fresh numbers on
// every replay.
#include "common.hpp"

#include <algorithm>
#include <cmath>

namespace rl {
namespace policy {

__device__ __forceinline__ void mulhilo(unsigned int a, unsigned int b, unsigned int& hi, unsigned int& lo) {
    const unsigned long long p = static_cast<unsigned long long>(a) * b;
    hi = static_cast<unsigned int>(p >> 32);
    lo = static_cast<unsigned int>(p);
}

__device__ __forceinline__ uint4 philox4x32_10(uint4 c, uint2 k) {
#pragma unroll
    for (int round = 0; round < 10; ++round) {
        unsigned int hi0, lo0, hi1, lo1;
        mulhilo(0xD2511F53u, c.x, hi0, lo0);
        mulhilo(0xCD9E8D57u, c.z, hi1, lo1);
        c = make_uint4(hi1 ^ c.y ^ k.x, lo1, hi0 ^ c.w ^ k.y, lo0);
        k.x += 0x9E3779B9u;
        k.y += 0xBB67AE85u;
    }
    return c;
}

__device__ __forceinline__ float uniform_open0(unsigned int x) {  // (0, 1]
    return (static_cast<float>(x >> 8) + 1.0f) * (1.0f / 16777216.0f);
}
__device__ __forceinline__ float uniform01(unsigned int x) {  // [0, 1)
    return static_cast<float>(x >> 8) * (1.0f / 16777216.0f);
}

// out[i] ~ N(0, 1) for i < n.  Four variates per Philox block.
__global__ void normal_kernel(unsigned long long seed, const long long* counter, unsigned int stream_id, float* out,
                              long long n) {
    const long long block = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x;
    const long long first = block * 4;
    if (first >= n) return;
    const unsigned long long draw = static_cast<unsigned long long>(counter ? counter[0] : 0);
    const uint4 c = make_uint4(static_cast<unsigned int>(block), static_cast<unsigned int>(draw),
                               static_cast<unsigned int>(draw >> 32), stream_id);
    const uint4 r = philox4x32_10(c, make_uint2(static_cast<unsigned int>(seed), static_cast<unsigned int>(seed >> 32)));
    const float two_pi = 6.28318530717958647692f;
    const float r0 = sqrtf(-2.0f * logf(uniform_open0(r.x)));
    const float r1 = sqrtf(-2.0f * logf(uniform_open0(r.z)));
    float s0, c0, s1, c1;
    sincosf(two_pi * uniform01(r.y), &s0, &c0);
    sincosf(two_pi * uniform01(r.w), &s1, &c1);
    const float v[4] = {r0 * c0, r0 * s0, r1 * c1, r1 * s1};
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (first + i < n) out[first + i] = v[i];
}

// idx[i] uniform in [0, count) by 32x64-bit multiply-high of a Philox word.
__global__ void sample_indices(unsigned long long seed, const long long* counter, unsigned int stream_id,
                               const long long* count, long long fixed_count, long long* idx, long long n) {
    const long long i = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x;
    if (i >= n) return;
    const unsigned long long draw = static_cast<unsigned long long>(counter ? counter[0] : 0);
    const uint4 c = make_uint4(static_cast<unsigned int>(i), static_cast<unsigned int>(i >> 32),
                               static_cast<unsigned int>(draw), stream_id ^ (static_cast<unsigned int>(draw >> 32) << 16));
    const uint4 r = philox4x32_10(c, make_uint2(static_cast<unsigned int>(seed), static_cast<unsigned int>(seed >> 32)));
    const unsigned long long limit = static_cast<unsigned long long>(count ? count[0] : fixed_count);
    const unsigned long long word = (static_cast<unsigned long long>(r.x) << 32) | r.y;
    // 64-bit multiply-high maps the uniform word onto [0, limit).
    idx[i] = static_cast<long long>(__umul64hi(word, limit));
}

// batch_x[i, :] = store_x[idx[i], :] for the seven replay fields.
struct GatherArgs {
    const long long* idx;
    long long batch;
    const float* obs;
    const float* next_obs;
    const float* action;
    const float* reward;
    const float* terminated;
    const float* truncated;
    const float* discount;
    float* out_obs;
    float* out_next_obs;
    float* out_action;
    float* out_reward;
    float* out_terminated;
    float* out_truncated;
    float* out_discount;
    int obs_dim, action_dim;
    long long capacity;
    int* error;
};

// Replay gather of the concatenated row [obs | next_obs | action | reward, terminated, truncated,
// discount]: one wave per sampled row, grid-stride over the rows so the batch size has no launch-shape
// limit.  The row's index is read once, then every lane loads its (up to eight) values of the row before
// storing any, so a row costs two memory round trips (the index, then the values).  An index outside
// [0, capacity) raises *error and reads row 0 instead.
// Column j of the concatenated row of replay row k.
__device__ __forceinline__ float gather_value(const GatherArgs& a, long long k, int j) {
    if (j < a.obs_dim) return a.obs[k * a.obs_dim + j];
    if (j < 2 * a.obs_dim) return a.next_obs[k * a.obs_dim + (j - a.obs_dim)];
    if (j < 2 * a.obs_dim + a.action_dim) return a.action[k * a.action_dim + (j - 2 * a.obs_dim)];
    const int f = j - 2 * a.obs_dim - a.action_dim;
    if (f == 0) return a.reward[k];
    if (f == 1) return a.terminated[k];
    if (f == 2) return a.truncated ? a.truncated[k] : 0.0f;
    return a.discount[k];
}

// Column j of batch row i of the outputs.
__device__ __forceinline__ void gather_store(const GatherArgs& a, long long i, int j, float v) {
    if (j < a.obs_dim) a.out_obs[i * a.obs_dim + j] = v;
    else if (j < 2 * a.obs_dim) a.out_next_obs[i * a.obs_dim + (j - a.obs_dim)] = v;
    else if (j < 2 * a.obs_dim + a.action_dim) a.out_action[i * a.action_dim + (j - 2 * a.obs_dim)] = v;
    else {
        const int f = j - 2 * a.obs_dim - a.action_dim;
        if (f == 0) a.out_reward[i] = v;
        else if (f == 1) a.out_terminated[i] = v;
        else if (f == 2) {
            if (a.out_truncated) a.out_truncated[i] = v;
        } else a.out_discount[i] = v;
    }
}

__global__ void gather_kernel(GatherArgs a) {
    constexpr int kPer = 8;  // values per lane loaded before the first store
    const int width = 2 * a.obs_dim + a.action_dim + 4;
    const int lane = threadIdx.x % kWave;
    const long long waves = static_cast<long long>(gridDim.x) * (blockDim.x / kWave);
    for (long long i = static_cast<long long>(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave; i < a.batch;
         i += waves) {
        long long k = a.idx[i];
        if (k < 0 || k >= a.capacity) {
            if (lane == 0 && a.error) atomicExch(a.error, 1);
            k = 0;
        }
        for (int j0 = 0; j0 < width; j0 += kPer * kWave) {
            float v[kPer];
#pragma unroll
            for (int u = 0; u < kPer; ++u) {
                const int j = j0 + u * kWave + lane;
                v[u] = j < width ? gather_value(a, k, j) : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < kPer; ++u) {
                const int j = j0 + u * kWave + lane;
                if (j < width) gather_store(a, i, j, v[u]);
            }
        }
    }
}

// out[r, :] = [a[r, :ca], b[r, :cb]] for rows r; b may be null (cb == 0).
__global__ void concat_kernel(float* out, long long ld_out, long long rows, const float* a, long long lda, int ca,
                              const float* b, long long ldb, int cb) {
    const long long total = rows * (ca + cb);
    for (long long idx = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x; idx < total;
         idx += static_cast<long long>(gridDim.x) * blockDim.x) {
        const long long r = idx / (ca + cb);
        const int c = static_cast<int>(idx % (ca + cb));
        out[r * ld_out + c] = c < ca ? a[r * lda + c] : b[r * ldb + (c - ca)];
    }
}

__device__ __forceinline__ float softplus(float x) {
    // torch.nn.functional.softplus with beta 1 and threshold 20.
    return x > 20.0f ? x : log1pf(expf(x));
}

// head[r, :A] = mean, head[r, A:2A] = raw log-std (bias already added).
// Writes actions (ld_actions stride), log pi and optionally std.  One wave per
// row (kPolicyRows rows per workgroup): lane j handles actions j, j + 64, ...
// with coalesced loads, and log pi is a fixed-order wave sum.
constexpr int kPolicyRows = 4;

__global__ __launch_bounds__(kPolicyRows* kWave) void tanh_gaussian_forward(const float* head, const float* noise,
                                                                           float* actions, long long ld_actions,
                                                                           float* log_probs, long long rows,
                                                                           int action_dim, int deterministic) {
    const long long r = static_cast<long long>(blockIdx.x) * kPolicyRows + threadIdx.x / kWave;
    if (r >= rows) return;  // wave-uniform
    const int lane = threadIdx.x % kWave;
    const float* h = head + r * 2 * action_dim;
    const float half_log_two_pi = 0.91893853320467274178f;  // log(sqrt(2 pi))
    const float ln2 = 0.69314718055994530942f;
    float lp = 0.0f;
    for (int j = lane; j < action_dim; j += kWave) {
        const float mean = h[j];
        if (deterministic) {
            actions[r * ld_actions + j] = tanhf(mean);
            continue;
        }
        const float log_std = -10.0f + 6.0f * (1.0f + tanhf(h[action_dim + j]));
        const float std = expf(log_std);
        const float eps = noise[r * action_dim + j];
        const float raw = mean + eps * std;
        actions[r * ld_actions + j] = tanhf(raw);
        const float diff = raw - mean;
        const float log_normal = -(diff * diff) / (2.0f * (std * std)) - logf(std) - half_log_two_pi;
        const float correction = 2.0f * (ln2 - raw - softplus(-2.0f * raw));
        lp += log_normal - correction;
    }
    if (log_probs && !deterministic) {
        lp = wave_sum(lp);
        if (lane == 0) log_probs[r] = lp;
    }
}

// Backward of the head given dL/da (rows < grad_rows, else zero) and dL/dlogpi.
// dhead[r, :A] = dL/dmean, dhead[r, A:] = dL/draw_log_std.  One thread per
// (row, action) element.
__global__ void tanh_gaussian_backward(const float* head, const float* noise, const float* dactions,
                                       long long ld_dactions, long long grad_rows, const float* dlog_probs,
                                       float* dhead, unsigned short* dhead_bf16, long long rows, int action_dim) {
    const long long idx = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= rows * action_dim) return;
    const long long r = idx / action_dim;
    const int j = static_cast<int>(idx - r * action_dim);
    const float* h = head + r * 2 * action_dim;
    const float dlp = dlog_probs ? dlog_probs[r] : 0.0f;
    const float mean = h[j];
    const float t = tanhf(h[action_dim + j]);
    const float log_std = -10.0f + 6.0f * (1.0f + t);
    const float std = expf(log_std);
    const float eps = noise[idx];
    const float raw = mean + eps * std;
    const float a = tanhf(raw);
    const float da = (dactions && r < grad_rows) ? dactions[r * ld_dactions + j] : 0.0f;
    const float g_raw = da * (1.0f - a * a) + dlp * 2.0f * a;
    const float dstd = g_raw * eps - dlp / std;
    const float dlog_std = dstd * std;
    const float g_std = dlog_std * 6.0f * (1.0f - t * t);
    if (dhead) {
        dhead[r * 2 * action_dim + j] = g_raw;
        dhead[r * 2 * action_dim + action_dim + j] = g_std;
    }
    if (dhead_bf16) {
        dhead_bf16[r * 2 * action_dim + j] = f32_to_bf16_bits(g_raw);
        dhead_bf16[r * 2 * action_dim + action_dim + j] = f32_to_bf16_bits(g_std);
    }
}

// Actor objective over the first `batch` rows:
//   q = min(q0, q1); loss = mean(alpha logpi - q) [+ bc term];
//   entropy = -mean(logpi); mean_action = mean(a).
// Gradients: dlogpi (total_rows rows, zero past batch), dq [2, batch],
// daction_bc (optional, batch x A) for the behaviour-cloning term.
// objective_rows: one thread per row; each workgroup writes its kObjTerms
// partial sums to partial[block * kObjTerms + term].  objective_finish adds
// the partials in block order and writes the metrics and, for the bc term,
// mean |q| to partial[blocks * kObjTerms]; bc_gradient then scales the
// per-element differences by it.
constexpr int kObjThreads = 256;
constexpr int kObjTerms = 5;  // |q|, log pi, action, bc squared difference, alpha log pi - q

__global__ __launch_bounds__(kObjThreads) void objective_rows(const float* q0, const float* q1, const float* log_probs,
                                                              const float* actions, long long ld_actions,
                                                              const float* replay_actions, const float* alpha,
                                                              float bc_alpha, long long batch, long long total_rows,
                                                              int action_dim, float* dlog_probs, float* dq0,
                                                              float* dq1, float* partial) {
    __shared__ float scratch[kObjThreads / kWave];
    const float a = alpha[0];
    const float inv = 1.0f / static_cast<float>(batch);
    const long long row0 = static_cast<long long>(blockIdx.x) * kObjThreads;
    const long long i = row0 + threadIdx.x;
    float terms[kObjTerms] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    if (i < batch) {
        const float x0 = q0[i], x1 = q1[i];
        const float q = fminf(x0, x1);
        const float lp = log_probs[i];
        terms[0] = fabsf(q);
        terms[1] = lp;
        terms[4] = a * lp - q;
        dlog_probs[i] = a * inv;
        dq0[i] = -inv * (x0 < x1 ? 1.0f : (x0 == x1 ? 0.5f : 0.0f));
        dq1[i] = -inv * (x1 < x0 ? 1.0f : (x0 == x1 ? 0.5f : 0.0f));
    } else if (i < total_rows) {
        dlog_probs[i] = 0.0f;
    }
    // this workgroup's rows of the action matrix, walked as one flat range
    const long long rows_here = max(0LL, min(batch, row0 + kObjThreads) - row0);
    const long long elements = rows_here * action_dim;
    // eight elements per thread loaded before their adds (a plain loop waits for each load in turn); the
    // adds keep the element order
    long long e = threadIdx.x;
    for (; e + 7 * kObjThreads < elements; e += 8 * kObjThreads) {
        float v[8], w[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const long long r = row0 + (e + u * kObjThreads) / action_dim;
            const int j = static_cast<int>((e + u * kObjThreads) % action_dim);
            v[u] = actions[r * ld_actions + j];
            w[u] = bc_alpha > 0.0f ? replay_actions[r * action_dim + j] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            terms[2] += v[u];
            if (bc_alpha > 0.0f) {
                const float d = v[u] - w[u];
                terms[3] += d * d;
            }
        }
    }
    for (; e < elements; e += kObjThreads) {
        const long long r = row0 + e / action_dim;
        const int j = static_cast<int>(e % action_dim);
        const float v = actions[r * ld_actions + j];
        terms[2] += v;
        if (bc_alpha > 0.0f) {
            const float d = v - replay_actions[r * action_dim + j];
            terms[3] += d * d;
        }
    }
#pragma unroll
    for (int t = 0; t < kObjTerms; ++t) {
        const float total = block_sum<kObjThreads>(terms[t], scratch);
        if (threadIdx.x == 0) partial[static_cast<long long>(blockIdx.x) * kObjTerms + t] = total;
    }
}

__global__ __launch_bounds__(kObjThreads) void objective_finish(const float* partial_in, int blocks, float bc_alpha,
                                                                long long batch, int action_dim, float* metrics,
                                                                float* qabs_out) {
    __shared__ float scratch[kObjThreads / kWave];
    float totals[kObjTerms];
#pragma unroll
    for (int t = 0; t < kObjTerms; ++t) {
        float v = 0.0f;
        for (int b = threadIdx.x; b < blocks; b += kObjThreads) v += partial_in[static_cast<long long>(b) * kObjTerms + t];
        totals[t] = block_sum<kObjThreads>(v, scratch);
    }
    if (threadIdx.x != 0) return;
    const float inv = 1.0f / static_cast<float>(batch);
    const float qabs = totals[0] * inv;
    const float count = static_cast<float>(batch * action_dim);
    float loss = totals[4] * inv;
    if (bc_alpha > 0.0f) loss += bc_alpha * qabs * (totals[3] / count);
    metrics[0] = loss;
    metrics[1] = -totals[1] * inv;
    metrics[2] = totals[2] / count;
    qabs_out[0] = qabs;
}

__global__ void bc_gradient(const float* actions, long long ld_actions, const float* replay_actions, float bc_alpha,
                            const float* qabs, long long batch, int action_dim, float* dactions_bc) {
    const long long idx = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= batch * action_dim) return;
    if (!(bc_alpha > 0.0f)) {
        dactions_bc[idx] = 0.0f;
        return;
    }
    const long long r = idx / action_dim;
    const int j = static_cast<int>(idx - r * action_dim);
    const float d = actions[r * ld_actions + j] - replay_actions[idx];
    dactions_bc[idx] = bc_alpha * qabs[0] * 2.0f * d / static_cast<float>(batch * action_dim);
}

// Temperature objective: value = exp(log_temp); loss = value (entropy - H*);
// d loss / d log_temp = loss.  metrics[0] = loss, metrics[1] = value.
__global__ void temperature_objective(const float* log_temp, const float* entropy, float target_entropy,
                                      float* grad, float* metrics) {
    const float value = expf(log_temp[0]);
    const float loss = value * (entropy[0] - target_entropy);
    grad[0] = loss;
    metrics[0] = loss;
    metrics[1] = value;
}

__global__ void exp_scalar(const float* x, float* out) { out[0] = expf(x[0]); }

__global__ void fill_kernel(float* x, long long n, float value) {
    for (long long i = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<long long>(gridDim.x) * blockDim.x)
        x[i] = value;
}

__global__ void add_kernel(float* x, const float* y, long long n) {
    for (long long i = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<long long>(gridDim.x) * blockDim.x)
        x[i] += y[i];
}

// counters[0] += 1 (updates), counters[1..2] += actor (actor, temperature).
__global__ void advance_counters(long long* counters, int actor) {
    counters[0] += 1;
    counters[1] += actor;
    counters[2] += actor;
}

// Exploration-noise repeats (robolearn/flashsac/agent.py:159-214, Warp
// _exploration_repeat/_exploration_actions, robolearn/warp/flashsac.py:269-299).
// state = int32 [count, length, refresh].  A call whose count is 0 or has
// reached length draws a new repeat length n ~ truncated zeta (the first k with
// u < cdf[k], plus one; when no entry exceeds u the length is 1, which is what
// torch.argmax returns for an all-false mask) and asks for fresh noise; count
// then advances.  The draw counter `step` is advanced here; exploration_noise
// uses the value this kernel read.
constexpr unsigned int kRepeatStream = 41;
constexpr unsigned int kExplorationStream = 37;

__global__ void exploration_repeat(unsigned long long seed, long long* step, const float* cdf, int max_n, int* state,
                                   const float* uniform) {
    if (blockIdx.x != 0 || threadIdx.x != 0) return;
    const unsigned long long draw = static_cast<unsigned long long>(step[0]);
    float u;
    if (uniform) {
        u = uniform[0];
    } else {
        const uint4 c = make_uint4(0u, static_cast<unsigned int>(draw), static_cast<unsigned int>(draw >> 32),
                                   kRepeatStream);
        u = uniform01(philox4x32_10(c, make_uint2(static_cast<unsigned int>(seed),
                                                  static_cast<unsigned int>(seed >> 32))).x);
    }
    int length = 1;
    for (int k = 0; k < max_n; ++k) {
        if (u < cdf[k]) {
            length = k + 1;
            break;
        }
    }
    const int count = state[0];
    const bool reset = count == 0 || count >= state[1];
    if (reset) state[1] = length;
    state[0] = (reset ? 0 : count) + 1;
    state[2] = reset ? 1 : 0;
    step[0] = static_cast<long long>(draw + 1);
}

// cached[i] <- a fresh N(0, 1) draw (or fresh[i] when given) if this call refreshed
// the noise; otherwise the previous noise is kept.  Four variates per thread.
__global__ void exploration_noise(unsigned long long seed, const long long* step, const int* state, float* cached,
                                  long long n, const float* fresh) {
    const long long block = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x;
    const long long first = block * 4;
    if (first >= n || state[2] == 0) return;
    if (fresh) {
        for (long long i = first; i < min(first + 4, n); ++i) cached[i] = fresh[i];
        return;
    }
    const unsigned long long draw = static_cast<unsigned long long>(step[0] - 1);  // the repeat kernel's draw
    const uint4 c = make_uint4(static_cast<unsigned int>(block), static_cast<unsigned int>(draw),
                               static_cast<unsigned int>(draw >> 32), kExplorationStream);
    const uint4 r = philox4x32_10(c, make_uint2(static_cast<unsigned int>(seed), static_cast<unsigned int>(seed >> 32)));
    const float two_pi = 6.28318530717958647692f;
    const float r0 = sqrtf(-2.0f * logf(uniform_open0(r.x)));
    const float r1 = sqrtf(-2.0f * logf(uniform_open0(r.z)));
    float s0, c0, s1, c1;
    sincosf(two_pi * uniform01(r.y), &s0, &c0);
    sincosf(two_pi * uniform01(r.w), &s1, &c1);
    const float v[4] = {r0 * c0, r0 * s0, r1 * c1, r1 * s1};
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (first + i < n) cached[first + i] = v[i];
}

// rewards[i] *= 1 / max(sqrt(var + eps), G_r_max / G_max) (reward_normalization.py:28-38).
__global__ void scale_rewards(float* rewards, long long n, const float* var, const float* r_max, float g_max, float eps) {
    const long long i = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x;
    if (i >= n) return;
    const float denominator = fmaxf(sqrtf(var[0] + eps), r_max[0] / g_max);
    rewards[i] = rewards[i] / denominator;
}

inline unsigned blocks_for(long long n, int threads = 256) {
    return static_cast<unsigned>(std::max<long long>(1, std::min<long long>((n + threads - 1) / threads, 65536)));
}

}  // namespace policy
}  // namespace rl

namespace P = rl::policy;

RL_API int rl_philox_normal(unsigned long long seed, const long long* counter, unsigned int stream_id, float* out,
                            long long n, void* stream) noexcept {
    return rl::guarded("rl_philox_normal", [&] {
        rl::require(out && n > 0, "Normal sampling needs a nonempty output.");
        const long long blocks = (n + 3) / 4;
        hipLaunchKernelGGL(P::normal_kernel, dim3(rl::ceil_div(blocks, 256)), dim3(256), 0, rl::as_stream(stream),
                           seed, counter, stream_id, out, n);
        rl::check_launch("Launch normal sampling");
    });
}

RL_API int rl_replay_sample_indices(unsigned long long seed, const long long* counter, unsigned int stream_id,
                                    const long long* count, long long fixed_count, long long* idx, long long n,
                                    void* stream) noexcept {
    return rl::guarded("rl_replay_sample_indices", [&] {
        rl::require(idx && n > 0 && (count || fixed_count > 0), "Index sampling needs an output and a positive count.");
        hipLaunchKernelGGL(P::sample_indices, dim3(rl::ceil_div(n, 256)), dim3(256), 0, rl::as_stream(stream), seed,
                           counter, stream_id, count, fixed_count, idx, n);
        rl::check_launch("Launch index sampling");
    });
}

RL_API int rl_exploration_noise(unsigned long long seed, long long* step, const float* cdf, int max_n, int* state,
                                float* cached_noise, long long count, const float* uniform, const float* fresh_noise,
                                void* stream) noexcept {
    return rl::guarded("rl_exploration_noise", [&] {
        rl::require(step && cdf && state && cached_noise && max_n > 0 && count > 0,
                    "Exploration noise needs the draw counter, the zeta CDF, the repeat state and the noise buffer.");
        hipStream_t st = rl::as_stream(stream);
        hipLaunchKernelGGL(P::exploration_repeat, dim3(1), dim3(1), 0, st, seed, step, cdf, max_n, state, uniform);
        rl::check_launch("Launch exploration repeat");
        hipLaunchKernelGGL(P::exploration_noise, dim3(rl::ceil_div((count + 3) / 4, 256)), dim3(256), 0, st, seed,
                           step, state, cached_noise, count, fresh_noise);
        rl::check_launch("Launch exploration noise");
    });
}

RL_API int rl_replay_gather(const long long* idx, long long batch, long long capacity, int obs_dim, int action_dim,
                            const float* obs, const float* next_obs, const float* action, const float* reward,
                            const float* terminated, const float* truncated, const float* discount, float* out_obs,
                            float* out_next_obs, float* out_action, float* out_reward, float* out_terminated,
                            float* out_truncated, float* out_discount, int* error, void* stream) noexcept {
    return rl::guarded("rl_replay_gather", [&] {
        rl::require(idx && batch > 0 && capacity > 0 && obs_dim > 0 && action_dim > 0, "Gather needs indices and shapes.");
        rl::require(obs && next_obs && action && reward && terminated && discount && out_obs && out_next_obs &&
                        out_action && out_reward && out_terminated && out_discount,
                    "Gather needs every storage and output field.");
        P::GatherArgs a{idx, batch, obs, next_obs, action, reward, terminated, truncated, discount, out_obs,
                        out_next_obs, out_action, out_reward, out_terminated, out_truncated, out_discount, obs_dim,
                        action_dim, capacity, error};
        const long long blocks = std::min<long long>((batch + 3) / 4, 1LL << 20);  // a wave per row
        hipLaunchKernelGGL(P::gather_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, rl::as_stream(stream),
                           a);
        rl::check_launch("Launch replay gather");
    });
}

RL_API int rl_concat_columns(float* out, long long ld_out, long long rows, const float* a, long long lda, int ca,
                             const float* b, long long ldb, int cb, void* stream) noexcept {
    return rl::guarded("rl_concat_columns", [&] {
        rl::require(out && a && rows > 0 && ca > 0 && cb >= 0 && (cb == 0 || b) && ld_out >= ca + cb,
                    "Concatenation needs valid buffers and widths.");
        hipLaunchKernelGGL(P::concat_kernel, dim3(P::blocks_for(rows * (ca + cb))), dim3(256), 0,
                           rl::as_stream(stream), out, ld_out, rows, a, lda, ca, b, ldb, cb);
        rl::check_launch("Launch concatenation");
    });
}

RL_API int rl_tanh_gaussian_forward(const float* head, const float* noise, float* actions, long long ld_actions,
                                    float* log_probs, long long rows, int action_dim, int deterministic,
                                    void* stream) noexcept {
    return rl::guarded("rl_tanh_gaussian_forward", [&] {
        rl::require(head && actions && rows > 0 && action_dim > 0 && (deterministic || noise),
                    "Policy forward needs head, noise and actions.");
        hipLaunchKernelGGL(P::tanh_gaussian_forward, dim3(rl::ceil_div(rows, P::kPolicyRows)),
                           dim3(P::kPolicyRows * rl::kWave), 0,
                           rl::as_stream(stream), head, noise, actions, ld_actions, log_probs, rows, action_dim,
                           deterministic);
        rl::check_launch("Launch policy forward");
    });
}

RL_API int rl_tanh_gaussian_backward(const float* head, const float* noise, const float* dactions,
                                     long long ld_dactions, long long grad_rows, const float* dlog_probs, float* dhead,
                                     void* dhead_bf16, long long rows, int action_dim, void* stream) noexcept {
    return rl::guarded("rl_tanh_gaussian_backward", [&] {
        rl::require(head && noise && (dhead || dhead_bf16) && rows > 0 && action_dim > 0,
                    "Policy backward needs head, noise and an output.");
        hipLaunchKernelGGL(P::tanh_gaussian_backward, dim3(rl::ceil_div(rows * action_dim, 256)), dim3(256), 0,
                           rl::as_stream(stream), head, noise, dactions, ld_dactions, grad_rows, dlog_probs, dhead,
                           static_cast<unsigned short*>(dhead_bf16), rows, action_dim);
        rl::check_launch("Launch policy backward");
    });
}

RL_API int rl_actor_objective(const float* q0, const float* q1, const float* log_probs, const float* actions,
                              long long ld_actions, const float* replay_actions, const float* alpha, float bc_alpha,
                              long long batch, long long total_rows, int action_dim, float* metrics, float* dlog_probs,
                              float* dq0, float* dq1, float* dactions_bc, float* partial, void* stream) noexcept {
    return rl::guarded("rl_actor_objective", [&] {
        rl::require(q0 && q1 && log_probs && actions && alpha && metrics && dlog_probs && dq0 && dq1 && partial,
                    "Actor objective needs Q values, log-probs, actions, alpha, outputs and partial scratch.");
        rl::require(batch > 0 && total_rows >= batch && action_dim > 0, "Actor objective shapes are invalid.");
        rl::require(bc_alpha <= 0.0f || replay_actions, "Behaviour cloning needs replay actions.");
        const hipStream_t st = rl::as_stream(stream);
        const unsigned blocks = rl::ceil_div(total_rows, P::kObjThreads);
        hipLaunchKernelGGL(P::objective_rows, dim3(blocks), dim3(P::kObjThreads), 0, st, q0, q1, log_probs, actions,
                           ld_actions, replay_actions, alpha, bc_alpha, batch, total_rows, action_dim, dlog_probs, dq0,
                           dq1, partial);
        rl::check_launch("Launch actor objective rows");
        float* qabs = partial + static_cast<long long>(blocks) * P::kObjTerms;
        hipLaunchKernelGGL(P::objective_finish, dim3(1), dim3(P::kObjThreads), 0, st, static_cast<const float*>(partial),
                           static_cast<int>(blocks), bc_alpha, batch, action_dim, metrics, qabs);
        rl::check_launch("Launch actor objective finish");
        if (dactions_bc) {
            hipLaunchKernelGGL(P::bc_gradient, dim3(rl::ceil_div(batch * action_dim, 256)), dim3(256), 0, st, actions,
                               ld_actions, replay_actions, bc_alpha, static_cast<const float*>(qabs), batch,
                               action_dim, dactions_bc);
            rl::check_launch("Launch behaviour-cloning gradient");
        }
    });
}

RL_API int rl_temperature_objective(const float* log_temp, const float* entropy, float target_entropy, float* grad,
                                    float* metrics, void* stream) noexcept {
    return rl::guarded("rl_temperature_objective", [&] {
        rl::require(log_temp && entropy && grad && metrics, "Temperature objective needs all buffers.");
        hipLaunchKernelGGL(P::temperature_objective, dim3(1), dim3(1), 0, rl::as_stream(stream), log_temp, entropy,
                           target_entropy, grad, metrics);
        rl::check_launch("Launch temperature objective");
    });
}

RL_API int rl_exp_scalar(const float* x, float* out, void* stream) noexcept {
    return rl::guarded("rl_exp_scalar", [&] {
        rl::require(x && out, "exp needs buffers.");
        hipLaunchKernelGGL(P::exp_scalar, dim3(1), dim3(1), 0, rl::as_stream(stream), x, out);
        rl::check_launch("Launch exp");
    });
}

// Graph-safe fill (a kernel, never a memset node).
RL_API int rl_fill(float* x, long long n, float value, void* stream) noexcept {
    return rl::guarded("rl_fill", [&] {
        rl::require(x && n > 0, "Fill needs a nonempty buffer.");
        hipLaunchKernelGGL(P::fill_kernel, dim3(P::blocks_for(n)), dim3(256), 0, rl::as_stream(stream), x, n, value);
        rl::check_launch("Launch fill");
    });
}

RL_API int rl_add(float* x, const float* y, long long n, void* stream) noexcept {
    return rl::guarded("rl_add", [&] {
        rl::require(x && y && n > 0, "Add needs nonempty buffers.");
        hipLaunchKernelGGL(P::add_kernel, dim3(P::blocks_for(n)), dim3(256), 0, rl::as_stream(stream), x, y, n);
        rl::check_launch("Launch add");
    });
}

RL_API int rl_advance_counters(long long* counters, int actor, void* stream) noexcept {
    return rl::guarded("rl_advance_counters", [&] {
        rl::require(counters != nullptr, "Counters must be nonnull.");
        hipLaunchKernelGGL(P::advance_counters, dim3(1), dim3(1), 0, rl::as_stream(stream), counters, actor);
        rl::check_launch("Launch counter advance");
    });
}

RL_API int rl_scale_rewards(float* rewards, long long n, const float* var, const float* r_max, float g_max, float eps,
                            void* stream) noexcept {
    return rl::guarded("rl_scale_rewards", [&] {
        rl::require(rewards && var && r_max && n > 0 && g_max > 0, "Reward scaling needs buffers and G_max > 0.");
        hipLaunchKernelGGL(P::scale_rewards, dim3(rl::ceil_div(n, 256)), dim3(256), 0, rl::as_stream(stream), rewards,
                           n, var, r_max, g_max, eps);
        rl::check_launch("Launch reward scaling");
    });
}
