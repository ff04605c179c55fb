// PPO update kernels: GAE, advantage normalization, minibatch permutation
// and gather, the clipped surrogate / value / entropy loss with its
// gradients, KL-adaptive learning rate and gradient-norm statistics.
//
// Reference semantics (robolearn/warp/ppo.py):
//   _gae :101-133            reverse scan per environment, time-major k = t E + i
//   _advantage_* :136-159    two-pass mean / variance normalization
//   _gather_batch :172-204   minibatch gather
//   kl_kernel :207-230       KL(N_old || N_new) averaged over the minibatch
//   _adapt_learning_rate :233-238
//   _gradient_sum_squares / _clip_gradients :241-252
//   loss_kernel :255-310
// All reductions are fixed-order (no atomics), so captured replays are
// bitwise repeatable.
#include "common.hpp"
#include "reduce.hpp"

#include <cmath>

namespace rl {
namespace ppo {

constexpr int kThreads = 1024;

// One thread per environment.
__global__ void gae_kernel(int horizon, int num_envs, float gamma, float lambda, int current_timeout_bootstrap,
                           const float* rewards, const float* values, const float* next_values, const int* terminated,
                           const int* truncated, float* advantages, float* returns) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= num_envs) return;
    // the inputs of eight steps are loaded before the first of them is processed: the stores of a step
    // would otherwise hold back the next step's loads, one memory round trip per step
    constexpr int kSteps = 8;
    float advantage = 0.0f;
    for (int top = horizon - 1; top >= 0; top -= kSteps) {
        float reward[kSteps], value[kSteps], next[kSteps];
        int term[kSteps], trunc[kSteps];
#pragma unroll
        for (int u = 0; u < kSteps; ++u) {
            const int step = top - u;
            if (step >= 0) {
                const long long k = static_cast<long long>(step) * num_envs + i;
                reward[u] = rewards[k];
                value[u] = values[k];
                next[u] = next_values[k];
                term[u] = terminated[k];
                trunc[u] = truncated[k];
            }
        }
#pragma unroll
        for (int u = 0; u < kSteps; ++u) {
            const int step = top - u;
            if (step < 0) break;
            const long long k = static_cast<long long>(step) * num_envs + i;
            float bootstrap = term[u] != 0 ? 0.0f : 1.0f;
            const float continuation = (term[u] != 0 || trunc[u] != 0) ? 0.0f : 1.0f;
            float next_value = next[u];
            if (current_timeout_bootstrap && trunc[u] != 0) {
                next_value = value[u];
                bootstrap = 1.0f;
            }
            const float delta = reward[u] + gamma * bootstrap * next_value - value[u];
            advantage = delta + gamma * lambda * continuation * advantage;
            advantages[k] = advantage;
            returns[k] = advantage + value[u];
        }
    }
}

__device__ float block_sum(float v, float* s) {
    s[threadIdx.x] = v;
    __syncthreads();
    for (int stride = kThreads / 2; stride > 0; stride >>= 1) {
        if (static_cast<int>(threadIdx.x) < stride) s[threadIdx.x] += s[threadIdx.x + stride];
        __syncthreads();
    }
    const float total = s[0];
    __syncthreads();
    return total;
}

// Single workgroup: mean, then centered variance, then normalize in place.
// stats[0] = sum, stats[1] = sum of squared deviations.
__global__ __launch_bounds__(kThreads) void normalize_kernel(float* advantages, long long n, int sample_std,
                                                             float* stats) {
    __shared__ float s[kThreads];
    float sum = strided_sum(advantages, threadIdx.x, n, kThreads, [](float x) { return x; });
    sum = block_sum(sum, s);
    const float nf = static_cast<float>(n);
    const float mean = sum / nf;
    float sq = strided_sum(advantages, threadIdx.x, n, kThreads, [mean](float x) {
        const float c = x - mean;
        return c * c;
    });
    sq = block_sum(sq, s);
    if (threadIdx.x == 0 && stats) {
        stats[0] = sum;
        stats[1] = sq;
    }
    const float denom = sample_std ? sqrtf(sq / fmaxf(nf - 1.0f, 1.0f)) + 1.0e-8f : sqrtf(sq / nf + 1.0e-8f);
    // eight loads ahead of their stores (each element is read and written by the same thread only)
    long long i = threadIdx.x;
    for (; i + 7 * kThreads < n; i += 8 * kThreads) {
        float w[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) w[u] = advantages[i + u * kThreads];
#pragma unroll
        for (int u = 0; u < 8; ++u) advantages[i + u * kThreads] = (w[u] - mean) / denom;
    }
    for (; i < n; i += kThreads) advantages[i] = (advantages[i] - mean) / denom;
}

__device__ __forceinline__ unsigned int mix32(unsigned int x) {
    // Integer finalizer (murmur3 fmix32).
    x ^= x >> 16;
    x *= 0x85EBCA6Bu;
    x ^= x >> 13;
    x *= 0xC2B2AE35u;
    x ^= x >> 16;
    return x;
}

// Keyed 4-round balanced Feistel bijection on [0, 2^(2h)).
__device__ __forceinline__ unsigned long long feistel(unsigned long long x, int h, unsigned int key0, unsigned int key1) {
    const unsigned long long mask = (1ull << h) - 1ull;
    unsigned long long left = x >> h;
    unsigned long long right = x & mask;
#pragma unroll
    for (int round = 0; round < 4; ++round) {
        const unsigned int f = mix32(static_cast<unsigned int>(right) ^ mix32(key0 + 0x9E3779B9u * (round + 1)) ^ key1);
        const unsigned long long next = left ^ (f & mask);
        left = right;
        right = next;
    }
    return (left << h) | right;
}

// perm[i] for i < n: cycle-walk the Feistel permutation back into [0, n).
// The walk starting from i < n returns into [0, n) before it can complete the
// cycle through i, so at most 2^(2h) steps are taken.
__global__ void permutation_kernel(long long n, int h, unsigned long long seed, const int* seed_counter,
                                   long long* perm_out, int* perm32_out) {
    const long long i = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x;
    if (i >= n) return;
    const unsigned int c = seed_counter ? static_cast<unsigned int>(seed_counter[0]) : 0u;
    const unsigned int key0 = mix32(static_cast<unsigned int>(seed) ^ mix32(c));
    const unsigned int key1 = mix32(static_cast<unsigned int>(seed >> 32) + 0x632BE5ABu * (c + 1u));
    const unsigned long long domain = 1ull << (2 * h);
    unsigned long long x = static_cast<unsigned long long>(i);
    for (unsigned long long step = 0; step < domain; ++step) {
        x = feistel(x, h, key0, key1);
        if (x < static_cast<unsigned long long>(n)) break;
    }
    if (perm_out) perm_out[i] = static_cast<long long>(x);
    if (perm32_out) perm32_out[i] = static_cast<int>(x);
}

__global__ void advance_int(int* value) { value[0] += 1; }

struct GatherArgs {
    const int* indices;
    long long offset, rows;
    int obs_dim, action_dim, obs_ld;
    const float *obs, *actions, *log_probs, *values, *advantages, *returns, *means, *stds;
    float *b_obs, *b_actions, *b_log_probs, *b_values, *b_advantages, *b_returns, *b_means, *b_stds;
};

// kGatherRows sampled rows per wave, four waves per workgroup: the wave loads its
// rows' indices at once, then issues every row's observation, action, mean and
// std loads (coalesced within a row) before the first store, so one memory
// round trip covers all of its rows; lanes 0 .. kGatherRows - 1 copy the rows'
// scalars.
constexpr int kGatherRows = 4;
constexpr int kGatherWaves = 4;

__global__ __launch_bounds__(kGatherWaves* kWave) void gather_kernel(GatherArgs a) {
    const int lane = threadIdx.x % kWave;
    const long long r0 = (static_cast<long long>(blockIdx.x) * kGatherWaves + threadIdx.x / kWave) * kGatherRows;
    if (r0 >= a.rows) return;  // wave-uniform
    const long long mine = r0 + lane;
    const bool scalar_lane = lane < kGatherRows && mine < a.rows;
    const long long kl = scalar_lane ? a.indices[a.offset + mine] : 0;
    long long k[kGatherRows];
#pragma unroll
    for (int i = 0; i < kGatherRows; ++i) k[i] = __shfl(kl, i);
    // the per-row scalars are loaded with the rows, ahead of every store (a load after the stores would
    // wait for them: the compiler cannot tell the buffers apart)
    float lp = 0.0f, value = 0.0f, advantage = 0.0f, ret = 0.0f;
    if (scalar_lane) {
        lp = a.log_probs[kl];
        value = a.values[kl];
        advantage = a.advantages[kl];
        ret = a.returns[kl];
    }
    constexpr int kObsPer = 4;  // observation values per lane and row (obs_dim <= 256)
    float obs[kGatherRows][kObsPer], act[kGatherRows], mean[kGatherRows], std[kGatherRows];
#pragma unroll
    for (int i = 0; i < kGatherRows; ++i) {
        const bool live = r0 + i < a.rows;
#pragma unroll
        for (int q = 0; q < kObsPer; ++q) {
            const int j = lane + q * kWave;
            obs[i][q] = live && j < a.obs_dim ? a.obs[k[i] * a.obs_dim + j] : 0.0f;
        }
        const bool c = live && lane < a.action_dim;
        act[i] = c ? a.actions[k[i] * a.action_dim + lane] : 0.0f;
        mean[i] = c ? a.means[k[i] * a.action_dim + lane] : 0.0f;
        std[i] = c ? a.stds[k[i] * a.action_dim + lane] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < kGatherRows; ++i) {
        const long long r = r0 + i;
        if (r >= a.rows) break;
#pragma unroll
        for (int q = 0; q < kObsPer; ++q) {
            const int j = lane + q * kWave;
            if (j < a.obs_dim) a.b_obs[r * a.obs_ld + j] = obs[i][q];
        }
        if (lane < a.action_dim) {
            a.b_actions[r * a.action_dim + lane] = act[i];
            a.b_means[r * a.action_dim + lane] = mean[i];
            a.b_stds[r * a.action_dim + lane] = std[i];
        }
    }
    if (scalar_lane) {
        a.b_log_probs[mine] = lp;
        a.b_values[mine] = value;
        a.b_advantages[mine] = advantage;
        a.b_returns[mine] = ret;
    }
}

// Rows wider than the register-batched kernel holds (obs_dim > 256 or
// action_dim > 64): one wave per sampled row, lanes striding over the row.
__global__ __launch_bounds__(kGatherWaves* kWave) void gather_rows_kernel(GatherArgs a) {
    const int lane = threadIdx.x % kWave;
    const long long r = static_cast<long long>(blockIdx.x) * kGatherWaves + threadIdx.x / kWave;
    if (r >= a.rows) return;  // wave-uniform
    const long long k = a.indices[a.offset + r];
    for (int j = lane; j < a.obs_dim; j += kWave) a.b_obs[r * a.obs_ld + j] = a.obs[k * a.obs_dim + j];
    for (int j = lane; j < a.action_dim; j += kWave) {
        a.b_actions[r * a.action_dim + j] = a.actions[k * a.action_dim + j];
        a.b_means[r * a.action_dim + j] = a.means[k * a.action_dim + j];
        a.b_stds[r * a.action_dim + j] = a.stds[k * a.action_dim + j];
    }
    if (lane == 0) {
        a.b_log_probs[r] = a.log_probs[k];
        a.b_values[r] = a.values[k];
        a.b_advantages[r] = a.advantages[k];
        a.b_returns[r] = a.returns[k];
    }
}

// Row-parallel passes over the minibatch: one wave per row (lanes over the
// action dimensions), kRowsPerBlock rows per workgroup, per-workgroup sums in
// fixed order, then one finishing workgroup that adds the partials in fixed
// order.  No atomics, so captured replays are bitwise repeatable.
constexpr int kRowThreads = 256;
constexpr int kRowWaves = kRowThreads / kWave;
constexpr int kRowsPerBlock = 16;

__device__ __forceinline__ float std_of(float p, int std_type, float std_min, float std_max) {
    return std_type == 1 ? fminf(fmaxf(p, std_min), std_max) : expf(p);
}

// Sum over the block's rows of KL(N_old || N_new) = sum_j log(s/s0) + (s0^2 + (m0 - m)^2) / (2 s^2) - 1/2.
__global__ __launch_bounds__(kRowThreads) void kl_partials(const float* mean, long long ld_mean,
                                                           const float* std_param, const float* old_mean,
                                                           const float* old_std, long long rows, int action_dim,
                                                           int std_type, float std_min, float std_max,
                                                           float* partial) {
    __shared__ float waves[kRowWaves];
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    float v = 0.0f;
    for (int r = wave; r < kRowsPerBlock; r += kRowWaves) {
        const long long row = blockIdx.x * static_cast<long long>(kRowsPerBlock) + r;
        if (row >= rows) break;
        for (int j = lane; j < action_dim; j += kWave) {
            const float std = std_of(std_param[j], std_type, std_min, std_max);
            const float ratio = old_std[row * action_dim + j] / std;
            const float delta = (old_mean[row * action_dim + j] - mean[row * ld_mean + j]) / std;
            v += 0.5f * (ratio * ratio + delta * delta - 1.0f) - logf(ratio);
        }
    }
    v = wave_sum(v);
    if (lane == 0) waves[wave] = v;
    __syncthreads();
    if (threadIdx.x == 0) {
        float total = 0.0f;
        for (int w = 0; w < kRowWaves; ++w) total += waves[w];
        partial[blockIdx.x] = total;
    }
}

// Mean KL over the minibatch and the adaptive learning-rate rule
// (robolearn/warp/ppo.py:233-238): lr / 1.5 (>= 1e-5) above 2 x target,
// lr x 1.5 (<= 1e-2) for 0 < KL < target / 2.
__global__ __launch_bounds__(kThreads) void kl_finish(const float* partial, int blocks, long long rows,
                                                      float desired_kl, int adapt, float* kl_out, float* lr) {
    __shared__ float s[kThreads];
    float v = 0.0f;
    for (int i = threadIdx.x; i < blocks; i += kThreads) v += partial[i];
    v = block_sum(v, s);
    if (threadIdx.x == 0) {
        const float kl = v / static_cast<float>(rows);
        kl_out[0] = kl;
        if (adapt) {
            if (kl > desired_kl * 2.0f) lr[0] = fmaxf(1.0e-5f, lr[0] / 1.5f);
            else if (kl < desired_kl / 2.0f && kl > 0.0f) lr[0] = fminf(1.0e-2f, lr[0] * 1.5f);
        }
    }
}

struct LossArgs {
    const float* mean;
    long long ld_mean;
    const float* value;       // critic output, row pitch ld_value
    long long ld_value;
    const float* std_param;
    const float* actions;
    const float* old_log_probs;
    const float* old_values;
    const float* advantages;
    const float* returns;
    long long rows;
    int action_dim;
    int std_type;
    float std_min, std_max;
    float clip_ratio, value_coefficient, entropy_coefficient, value_loss_scale;
    int clip_value;
    float* dmean;             // [rows, A]
    float* dvalue;            // row pitch ld_dvalue
    long long ld_dvalue;
    float* dstd_rows;         // [rows, A] per-row std-parameter gradient (when std_partial is null)
    float* partial;           // [4, blocks]: total, policy, value, entropy sums (already scaled by 1/rows)
    // fused minibatch form: KL(N_old || N_new) sums in partial row 4 (old_mean, old_std given), and the
    // std-parameter gradient as per-workgroup column sums in partial rows 5 .. 5 + A instead of dstd_rows
    const float* old_mean;
    const float* old_std;
    bool fused;
};

// Clipped surrogate, clipped value and entropy terms of one row and their
// gradients with respect to the mean, the value and the std parameter.
// Terms of action dimension j that depend only on the std parameter (shared by every row): the log
// std, its inverse exponential, d log std / d parameter and the std itself.
struct DimTerms {
    float ls, inv_std, dls_dp, std;
};

__device__ __forceinline__ DimTerms dim_terms(const LossArgs& a, int j) {
    const float p = a.std_param[j];
    DimTerms d;
    if (a.std_type == 1) {
        const float c = fminf(fmaxf(p, a.std_min), a.std_max);
        d.ls = logf(c);
        d.dls_dp = (p >= a.std_min && p <= a.std_max) ? 1.0f / c : 0.0f;
    } else {
        d.ls = p;
        d.dls_dp = 1.0f;
    }
    d.inv_std = expf(-d.ls);
    d.std = std_of(p, a.std_type, a.std_min, a.std_max);
    return d;
}

__global__ __launch_bounds__(kRowThreads) void loss_kernel(LossArgs a) {
    __shared__ float waves[5][kRowWaves];
    __shared__ float std_cols[kRowWaves][kWave];
    const float ln_two_pi = 1.8378770664093453f;
    const float entropy_const = 1.4189385332046727f;
    const float scale = 1.0f / static_cast<float>(a.rows);
    const float lo = 1.0f - a.clip_ratio, hi = 1.0f + a.clip_ratio;
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    float sums[5] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    float std_col = 0.0f;  // fused form: this lane's std-gradient column (lane < A, A <= 64)
    // At most one action dimension per lane (A <= 64): its std terms and the row entropy, which does not
    // depend on the row, are computed once per wave instead of once per row (the same expressions, so the
    // same values); wider actions take the per-row loops.
    const bool one_dim = a.action_dim <= kWave;
    const bool mine = lane < a.action_dim;
    DimTerms own{0.0f, 0.0f, 0.0f, 1.0f};
    float row_entropy = 0.0f;
    if (one_dim) {
        if (mine) own = dim_terms(a, lane);
        row_entropy = wave_sum(mine ? own.ls + entropy_const : 0.0f);
    }
    // A row's inputs.  With one dimension per lane every wave loads all of its rows' inputs before it
    // processes the first, so the rows' memory round trips overlap instead of following one another;
    // the rows are then processed in the same order as the per-row form (the same sums).
    struct RowIn {
        float act, mu, old_mu, old_sd, old_lp, adv, v, ret, old_v;
    };
    const auto load_row = [&](long long i) {
        RowIn in{0.0f, 0.0f, 0.0f, 1.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
        if (i < a.rows) {
            if (one_dim && mine) {
                in.act = a.actions[i * a.action_dim + lane];
                in.mu = a.mean[i * a.ld_mean + lane];
                if (a.fused) {
                    in.old_mu = a.old_mean[i * a.action_dim + lane];
                    in.old_sd = a.old_std[i * a.action_dim + lane];
                }
            }
            in.old_lp = a.old_log_probs[i];
            in.adv = a.advantages[i];
            in.v = a.value[i * a.ld_value];
            in.ret = a.returns[i];
            if (a.clip_value) in.old_v = a.old_values[i];
        }
        return in;
    };
    const auto process = [&](long long i, const RowIn& in) {
        float log_prob = 0.0f, entropy = 0.0f;
        if (one_dim) {
            if (mine) {
                const float residual = (in.act - in.mu) * own.inv_std;
                log_prob -= 0.5f * (residual * residual + 2.0f * own.ls + ln_two_pi);
            }
            log_prob = wave_sum(log_prob);
            entropy = row_entropy;
        } else {
            for (int j = lane; j < a.action_dim; j += kWave) {
                const DimTerms d = dim_terms(a, j);
                const float residual = (a.actions[i * a.action_dim + j] - a.mean[i * a.ld_mean + j]) * d.inv_std;
                log_prob -= 0.5f * (residual * residual + 2.0f * d.ls + ln_two_pi);
                entropy += d.ls + entropy_const;
            }
            log_prob = wave_sum(log_prob);
            entropy = wave_sum(entropy);
        }
        const float ratio = expf(log_prob - in.old_lp);
        const float adv = in.adv;
        const float clipped_ratio = fminf(fmaxf(ratio, lo), hi);
        const float unclipped = ratio * adv;
        const float clipped = clipped_ratio * adv;
        const float policy_loss = -fminf(unclipped, clipped);
        // d policy / d ratio: the smaller branch carries the gradient; on a tie
        // inside the clip range both branches have derivative -adv.
        float dratio;
        if (unclipped <= clipped) dratio = -adv;
        else dratio = (ratio > lo && ratio < hi) ? -adv : 0.0f;
        const float v = in.v;
        const float error = v - in.ret;
        float value_loss = error * error;
        float dv = 2.0f * error;
        if (a.clip_value) {
            const float d = v - in.old_v;
            const float cv = in.old_v + fminf(fmaxf(d, -a.clip_ratio), a.clip_ratio);
            const float ce = cv - in.ret;
            if (ce * ce > value_loss) {
                value_loss = ce * ce;
                dv = (d >= -a.clip_ratio && d <= a.clip_ratio) ? 2.0f * ce : 0.0f;
            }
        }
        value_loss = a.value_loss_scale * value_loss;
        dv *= a.value_loss_scale;
        if (lane == 0) a.dvalue[i * a.ld_dvalue] = scale * a.value_coefficient * dv;
        const float dlp = scale * dratio * ratio;
        // KL(N_old || N_new) = log(s / s0) + (s0^2 + (m0 - m)^2) / (2 s^2) - 1/2 (ppo.py:207-230)
        if (one_dim) {
            if (mine) {
                const float residual = (in.act - in.mu) * own.inv_std;
                a.dmean[i * a.action_dim + lane] = dlp * residual * own.inv_std;
                const float dstd = (dlp * (residual * residual - 1.0f) - scale * a.entropy_coefficient) * own.dls_dp;
                if (a.fused) {
                    std_col += dstd;
                    const float sd_ratio = in.old_sd / own.std;
                    const float delta = (in.old_mu - in.mu) / own.std;
                    sums[4] += 0.5f * (sd_ratio * sd_ratio + delta * delta - 1.0f) - logf(sd_ratio);
                } else {
                    a.dstd_rows[i * a.action_dim + lane] = dstd;
                }
            }
        } else {
            for (int j = lane; j < a.action_dim; j += kWave) {
                const DimTerms d = dim_terms(a, j);
                const float residual = (a.actions[i * a.action_dim + j] - a.mean[i * a.ld_mean + j]) * d.inv_std;
                a.dmean[i * a.action_dim + j] = dlp * residual * d.inv_std;
                const float dstd = (dlp * (residual * residual - 1.0f) - scale * a.entropy_coefficient) * d.dls_dp;
                if (a.fused) {
                    std_col += dstd;
                    const float sd_ratio = a.old_std[i * a.action_dim + j] / d.std;
                    const float delta = (a.old_mean[i * a.action_dim + j] - a.mean[i * a.ld_mean + j]) / d.std;
                    sums[4] += 0.5f * (sd_ratio * sd_ratio + delta * delta - 1.0f) - logf(sd_ratio);
                } else {
                    a.dstd_rows[i * a.action_dim + j] = dstd;
                }
            }
        }
        sums[0] += scale * (policy_loss + a.value_coefficient * value_loss - a.entropy_coefficient * entropy);
        sums[1] += scale * policy_loss;
        sums[2] += scale * value_loss;
        sums[3] += scale * entropy;
    };
    constexpr int kPerWave = kRowsPerBlock / kRowWaves;
    static_assert(kPerWave * kRowWaves == kRowsPerBlock, "whole rows per wave");
    const long long first = blockIdx.x * static_cast<long long>(kRowsPerBlock) + wave;
    if (one_dim) {
        RowIn in[kPerWave];
#pragma unroll
        for (int q = 0; q < kPerWave; ++q) in[q] = load_row(first + q * kRowWaves);
#pragma unroll
        for (int q = 0; q < kPerWave; ++q) {
            if (first + q * kRowWaves >= a.rows) break;
            process(first + q * kRowWaves, in[q]);
        }
    } else {
        for (int q = 0; q < kPerWave; ++q) {
            if (first + q * kRowWaves >= a.rows) break;
            process(first + q * kRowWaves, load_row(first + q * kRowWaves));
        }
    }
    if (a.fused) {
        sums[4] = wave_sum(sums[4]);  // lanes hold different action dimensions
        std_cols[wave][lane] = std_col;
    }
    if (lane == 0) {
#pragma unroll
        for (int q = 0; q < 5; ++q) waves[q][wave] = sums[q];
    }
    __syncthreads();
    const int terms = a.fused ? 5 : 4;
    if (static_cast<int>(threadIdx.x) < terms) {
        float total = 0.0f;
        for (int w = 0; w < kRowWaves; ++w) total += waves[threadIdx.x][w];
        a.partial[threadIdx.x * static_cast<long long>(gridDim.x) + blockIdx.x] = total;
    }
    if (a.fused && static_cast<int>(threadIdx.x) < a.action_dim) {
        float total = 0.0f;
        for (int w = 0; w < kRowWaves; ++w) total += std_cols[w][threadIdx.x];
        a.partial[(5 + threadIdx.x) * static_cast<long long>(gridDim.x) + blockIdx.x] = total;
    }
}

// Fused minibatch finish over partial [5 + action_dim][blocks]: totals[q] =
// sum_b partial[q, b] (q < 4), the mean KL from column 4 and the adaptive
// learning-rate rule (ppo.py:233-238), and the std-parameter gradient dstd[j] =
// sum_b partial[5 + j, b].  One wave per column: lane l adds blocks l, l + 64,
// ... in order, then the fixed lane reduction of wave_sum.
__global__ __launch_bounds__(kThreads) void loss_finish(const float* partial, long long blocks, long long rows,
                                                        int action_dim, float desired_kl, int adapt, float* totals,
                                                        float* kl_out, float* lr, float* dstd) {
    const int lane = threadIdx.x % kWave;
    const int columns = 5 + action_dim;
    for (int q = threadIdx.x / kWave; q < columns; q += kThreads / kWave) {  // wave-uniform
        const float* column = partial + q * blocks;
        float v = 0.0f;
#pragma unroll 8
        for (long long b = lane; b < blocks; b += kWave) v += column[b];
        v = wave_sum(v);
        if (lane != 0) continue;
        if (q < 4) {
            totals[q] = v;
        } else if (q == 4) {
            const float kl = v / static_cast<float>(rows);
            kl_out[0] = kl;
            if (adapt) {
                if (kl > desired_kl * 2.0f) lr[0] = fmaxf(1.0e-5f, lr[0] / 1.5f);
                else if (kl < desired_kl / 2.0f && kl > 0.0f) lr[0] = fminf(1.0e-2f, lr[0] * 1.5f);
            }
        } else {
            dstd[q - 5] = v;
        }
    }
}

// out[q] = sum_b partial[q, b] in fixed order, for q < count.
__global__ __launch_bounds__(kThreads) void sum_rows_kernel(const float* terms, long long rows, int count, float* out) {
    __shared__ float s[kThreads];
    for (int q = 0; q < count; ++q) {
        float v = 0.0f;
        for (long long i = threadIdx.x; i < rows; i += kThreads) v += terms[q * rows + i];
        v = block_sum(v, s);
        if (threadIdx.x == 0) out[q] = v;
    }
}

// Sum of squares over a flat vector: per-block partials (fixed order), then one block.
__global__ void sumsq_partials(const float* x, long long n, float* partial) {
    __shared__ float s[256];
    const long long start = static_cast<long long>(blockIdx.x) * 4096;
    const float total = block_sum_squares(x, start, min(n, start + 4096), s);
    if (threadIdx.x == 0) partial[blockIdx.x] = total;
}

__global__ __launch_bounds__(kThreads) void sumsq_finish(const float* partial, long long blocks, float* out) {
    __shared__ float s[kThreads];
    float v = 0.0f;
    for (long long i = threadIdx.x; i < blocks; i += kThreads) v += partial[i];
    v = block_sum(v, s);
    if (threadIdx.x == 0) out[0] = v;
}

// g *= min(1, max_norm / (sqrt(sum_squares) + 1e-6)).
__global__ void clip_kernel(float* g, long long n, const float* sum_squares, float max_norm) {
    const float coefficient = fminf(1.0f, max_norm / (sqrtf(sum_squares[0]) + 1.0e-6f));
    for (long long i = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<long long>(gridDim.x) * blockDim.x)
        g[i] *= coefficient;
}

// clip_kernel on sumsq_partials' output: every workgroup adds the partials in
// sumsq_finish's order (so all see the same sum of squares, bitwise that of
// sumsq_finish), workgroup 0 stores it, and each scales its grid-stride share.
__global__ __launch_bounds__(kThreads) void clip_from_partials(float* g, long long n, const float* partial,
                                                               long long blocks, float* sum_squares, float max_norm) {
    __shared__ float s[kThreads];
    float v = 0.0f;
    for (long long i = threadIdx.x; i < blocks; i += kThreads) v += partial[i];
    v = block_sum(v, s);
    if (blockIdx.x == 0 && threadIdx.x == 0) sum_squares[0] = v;
    const float coefficient = fminf(1.0f, max_norm / (sqrtf(v) + 1.0e-6f));
    for (long long i = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<long long>(gridDim.x) * blockDim.x)
        g[i] *= coefficient;
}

// dx *= elu'(y) = 1 if y > 0 else y + 1 (ELU with alpha 1, from its output).
__global__ void elu_backward_kernel(float* dx, const float* y, long long n) {
    for (long long i = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<long long>(gridDim.x) * blockDim.x)
        dx[i] *= y[i] > 0.0f ? 1.0f : y[i] + 1.0f;
}

// Rollout action sampling (robolearn/warp/ppo.py:26-58 _sample, called by act
// :488-507): per action dimension std = exp(p) ("log") or clamp(p, lo, hi)
// ("scalar"), actions = mean + std * noise, log_prob = sum_j -(noise^2 +
// 2 log std + ln 2 pi) / 2, values = value[:, 0], sampled_std = std.  One wave
// per environment row, lanes over the action dimensions.  noise == nullptr is
// the deterministic case (zero noise).  The draw counter of the noise is
// advanced here, after the launch that drew with it.
struct SampleArgs {
    const float* mean;
    long long ld_mean;
    const float* value;
    long long ld_value;
    const float* parameter;
    const float* noise;
    long long rows;
    int action_dim;
    int scalar_std;
    float min_std, max_std;
    float* actions;
    float* log_probs;
    float* values;
    float* sampled_std;
    long long* counter;
};

__global__ __launch_bounds__(kGatherRows* kWave) void rollout_sample(SampleArgs a) {
    if (a.counter && blockIdx.x == 0 && threadIdx.x == 0) a.counter[0] += 1;
    const long long r = static_cast<long long>(blockIdx.x) * kGatherRows + threadIdx.x / kWave;
    if (r >= a.rows) return;  // wave-uniform
    const int lane = threadIdx.x % kWave;
    constexpr float kLogTwoPi = 1.8378770664093453f;
    float log_prob = 0.0f;
    for (int j = lane; j < a.action_dim; j += kWave) {
        const float p = a.parameter[j];
        const float std = a.scalar_std ? fminf(fmaxf(p, a.min_std), a.max_std) : expf(p);
        const float log_std = a.scalar_std ? logf(std) : p;
        const float noise = a.noise ? a.noise[r * a.action_dim + j] : 0.0f;
        a.actions[r * a.action_dim + j] = a.mean[r * a.ld_mean + j] + std * noise;
        log_prob -= 0.5f * (noise * noise + 2.0f * log_std + kLogTwoPi);
        if (r == 0) a.sampled_std[j] = std;
    }
    log_prob = wave_sum(log_prob);
    if (lane == 0) {
        a.log_probs[r] = log_prob;
        a.values[r] = a.value[r * a.ld_value];
    }
}

// Rollout store of step t (robolearn/warp/ppo.py:61-99 _store, called by store
// :509-550): row k = t E + i of every rollout buffer takes environment i's
// observation, sampled action, log-prob, value, reward, done flags, bootstrap
// value of the pre-reset next observation, mean and the sampled std.
struct StoreArgs {
    long long row0;  // t * E
    long long num_envs;
    int obs_dim, action_dim;
    const float* observations;
    const float* actions;
    const float* log_probs;
    const float* values;
    const float* rewards;
    const int* terminated;
    const int* truncated;
    const float* next_values;
    long long ld_next_values;
    const float* mean;
    long long ld_mean;
    const float* sampled_std;
    float* rollout_obs;
    float* rollout_actions;
    float* rollout_log_probs;
    float* rollout_values;
    float* rollout_rewards;
    int* rollout_terminated;
    int* rollout_truncated;
    float* rollout_next_values;
    float* rollout_means;
    float* rollout_stds;
};

__global__ __launch_bounds__(kGatherRows* kWave) void rollout_store(StoreArgs a) {
    const long long i = static_cast<long long>(blockIdx.x) * kGatherRows + threadIdx.x / kWave;
    if (i >= a.num_envs) return;  // wave-uniform
    const int lane = threadIdx.x % kWave;
    const long long k = a.row0 + i;
    for (int j = lane; j < a.obs_dim; j += kWave) a.rollout_obs[k * a.obs_dim + j] = a.observations[i * a.obs_dim + j];
    for (int j = lane; j < a.action_dim; j += kWave) {
        a.rollout_actions[k * a.action_dim + j] = a.actions[i * a.action_dim + j];
        a.rollout_means[k * a.action_dim + j] = a.mean[i * a.ld_mean + j];
        a.rollout_stds[k * a.action_dim + j] = a.sampled_std[j];
    }
    if (lane == 0) {
        a.rollout_log_probs[k] = a.log_probs[i];
        a.rollout_values[k] = a.values[i];
        a.rollout_rewards[k] = a.rewards[i];
        a.rollout_terminated[k] = a.terminated[i];
        a.rollout_truncated[k] = a.truncated[i];
        a.rollout_next_values[k] = a.next_values[i * a.ld_next_values];
    }
}

}  // namespace ppo
}  // namespace rl

namespace Q = rl::ppo;

RL_API int rl_ppo_sample(const float* mean, long long ld_mean, const float* value, long long ld_value,
                         const float* parameter, int scalar_std, float min_std, float max_std, const float* noise,
                         long long rows, int action_dim, float* actions, float* log_probs, float* values,
                         float* sampled_std, long long* counter, void* stream) noexcept {
    return rl::guarded("rl_ppo_sample", [&] {
        rl::require(mean && value && parameter && actions && log_probs && values && sampled_std,
                    "PPO sampling needs the mean, value, distribution parameter and outputs.");
        rl::require(rows > 0 && action_dim > 0 && ld_mean >= action_dim && ld_value >= 1,
                    "PPO sampling shapes are invalid.");
        Q::SampleArgs a{mean, ld_mean, value, ld_value, parameter, noise, rows, action_dim, scalar_std, min_std,
                        max_std, actions, log_probs, values, sampled_std, counter};
        hipLaunchKernelGGL(Q::rollout_sample, dim3(rl::ceil_div(rows, Q::kGatherRows)),
                           dim3(Q::kGatherRows * rl::kWave), 0, rl::as_stream(stream), a);
        rl::check_launch("Launch PPO rollout sampling");
    });
}

RL_API int rl_ppo_store(int step, long long num_envs, int obs_dim, int action_dim, const float* observations,
                        const float* actions, const float* log_probs, const float* values, const float* rewards,
                        const int* terminated, const int* truncated, const float* next_values,
                        long long ld_next_values, const float* mean, long long ld_mean, const float* sampled_std,
                        float* rollout_obs, float* rollout_actions, float* rollout_log_probs, float* rollout_values,
                        float* rollout_rewards, int* rollout_terminated, int* rollout_truncated,
                        float* rollout_next_values, float* rollout_means, float* rollout_stds,
                        void* stream) noexcept {
    return rl::guarded("rl_ppo_store", [&] {
        rl::require(step >= 0 && num_envs > 0 && obs_dim > 0 && action_dim > 0 && ld_mean >= action_dim &&
                        ld_next_values >= 1,
                    "PPO store shapes are invalid.");
        rl::require(observations && actions && log_probs && values && rewards && terminated && truncated &&
                        next_values && mean && sampled_std,
                    "PPO store needs every per-step input.");
        rl::require(rollout_obs && rollout_actions && rollout_log_probs && rollout_values && rollout_rewards &&
                        rollout_terminated && rollout_truncated && rollout_next_values && rollout_means && rollout_stds,
                    "PPO store needs every rollout buffer.");
        Q::StoreArgs a{static_cast<long long>(step) * num_envs, num_envs, obs_dim, action_dim, observations, actions,
                       log_probs, values, rewards, terminated, truncated, next_values, ld_next_values, mean, ld_mean,
                       sampled_std, rollout_obs, rollout_actions, rollout_log_probs, rollout_values, rollout_rewards,
                       rollout_terminated, rollout_truncated, rollout_next_values, rollout_means, rollout_stds};
        hipLaunchKernelGGL(Q::rollout_store, dim3(rl::ceil_div(num_envs, Q::kGatherRows)),
                           dim3(Q::kGatherRows * rl::kWave), 0, rl::as_stream(stream), a);
        rl::check_launch("Launch PPO rollout store");
    });
}

RL_API int rl_gae(int horizon, int num_envs, float gamma, float lambda, int current_timeout_bootstrap,
                  const float* rewards, const float* values, const float* next_values, const int* terminated,
                  const int* truncated, float* advantages, float* returns, void* stream) noexcept {
    return rl::guarded("rl_gae", [&] {
        rl::require(horizon > 0 && num_envs > 0, "GAE needs a positive horizon and environment count.");
        rl::require(rewards && values && next_values && terminated && truncated && advantages && returns,
                    "GAE needs every rollout buffer.");
        hipLaunchKernelGGL(Q::gae_kernel, dim3(rl::ceil_div(num_envs, 256)), dim3(256), 0, rl::as_stream(stream),
                           horizon, num_envs, gamma, lambda, current_timeout_bootstrap, rewards, values, next_values,
                           terminated, truncated, advantages, returns);
        rl::check_launch("Launch GAE");
    });
}

RL_API int rl_normalize_advantages(float* advantages, long long n, int sample_std, float* stats, void* stream) noexcept {
    return rl::guarded("rl_normalize_advantages", [&] {
        rl::require(advantages && n > 0, "Advantage normalization needs a nonempty vector.");
        hipLaunchKernelGGL(Q::normalize_kernel, dim3(1), dim3(Q::kThreads), 0, rl::as_stream(stream), advantages, n,
                           sample_std, stats);
        rl::check_launch("Launch advantage normalization");
    });
}

RL_API int rl_permutation(long long n, unsigned long long seed, const int* seed_counter, long long* perm64,
                          int* perm32, void* stream) noexcept {
    return rl::guarded("rl_permutation", [&] {
        rl::require(n > 0 && n < (1ll << 40) && (perm64 || perm32), "Permutation needs 0 < n < 2^40 and an output.");
        int bits = 1;
        while ((1ll << bits) < n) ++bits;
        const int h = (bits + 1) / 2;
        hipLaunchKernelGGL(Q::permutation_kernel, dim3(rl::ceil_div(n, 256)), dim3(256), 0, rl::as_stream(stream), n,
                           h, seed, seed_counter, perm64, perm32);
        rl::check_launch("Launch permutation");
    });
}

RL_API int rl_advance_int(int* value, void* stream) noexcept {
    return rl::guarded("rl_advance_int", [&] {
        rl::require(value != nullptr, "Counter must be nonnull.");
        hipLaunchKernelGGL(Q::advance_int, dim3(1), dim3(1), 0, rl::as_stream(stream), value);
        rl::check_launch("Launch counter advance");
    });
}

RL_API int rl_ppo_gather(const int* indices, long long offset, long long rows, int obs_dim, int action_dim, int obs_ld,
                         const float* obs, const float* actions, const float* log_probs, const float* values,
                         const float* advantages, const float* returns, const float* means, const float* stds,
                         float* b_obs, float* b_actions, float* b_log_probs, float* b_values, float* b_advantages,
                         float* b_returns, float* b_means, float* b_stds, void* stream) noexcept {
    return rl::guarded("rl_ppo_gather", [&] {
        rl::require(indices && rows > 0 && rows <= (1LL << 32) && obs_dim > 0 && action_dim > 0 && obs_ld >= obs_dim,
                    "PPO gather shapes are invalid.");
        Q::GatherArgs a{indices, offset, rows, obs_dim, action_dim, obs_ld, obs, actions, log_probs, values, advantages,
                        returns, means, stds, b_obs, b_actions, b_log_probs, b_values, b_advantages, b_returns, b_means,
                        b_stds};
        if (obs_dim <= 4 * rl::kWave && action_dim <= rl::kWave) {
            hipLaunchKernelGGL(Q::gather_kernel, dim3(rl::ceil_div(rows, Q::kGatherRows * Q::kGatherWaves)),
                               dim3(Q::kGatherWaves * rl::kWave), 0, rl::as_stream(stream), a);
        } else {
            hipLaunchKernelGGL(Q::gather_rows_kernel, dim3(rl::ceil_div(rows, Q::kGatherWaves)),
                               dim3(Q::kGatherWaves * rl::kWave), 0, rl::as_stream(stream), a);
        }
        rl::check_launch("Launch PPO gather");
    });
}

RL_API int rl_ppo_kl_adapt(const float* mean, long long ld_mean, const float* std_param, const float* old_mean,
                           const float* old_std, long long rows, int action_dim, int std_type, float std_min,
                           float std_max, float desired_kl, int adapt, float* partial, float* kl_out, float* lr,
                           void* stream) noexcept {
    return rl::guarded("rl_ppo_kl_adapt", [&] {
        rl::require(mean && std_param && old_mean && old_std && partial && kl_out && (!adapt || lr) && rows > 0 &&
                        action_dim > 0,
                    "KL needs means, std parameters, partial scratch and outputs.");
        const long long blocks = (rows + Q::kRowsPerBlock - 1) / Q::kRowsPerBlock;
        rl::require(blocks <= (1LL << 30), "KL row count is too large.");
        const hipStream_t st = rl::as_stream(stream);
        hipLaunchKernelGGL(Q::kl_partials, dim3(static_cast<unsigned>(blocks)), dim3(Q::kRowThreads), 0, st, mean,
                           ld_mean, std_param, old_mean, old_std, rows, action_dim, std_type, std_min, std_max,
                           partial);
        rl::check_launch("Launch KL partials");
        hipLaunchKernelGGL(Q::kl_finish, dim3(1), dim3(Q::kThreads), 0, st, partial, static_cast<int>(blocks), rows,
                           desired_kl, adapt, kl_out, lr);
        rl::check_launch("Launch KL adapt");
    });
}

RL_API int rl_ppo_loss(const float* mean, long long ld_mean, const float* value, const float* std_param,
                       const float* actions, const float* old_log_probs, const float* old_values,
                       const float* advantages, const float* returns, long long rows, int action_dim, int std_type,
                       float std_min, float std_max, float clip_ratio, float value_coefficient,
                       float entropy_coefficient, float value_loss_scale, int clip_value, float* dmean, float* dvalue,
                       float* dstd_rows, float* row_terms, float* totals, void* stream) noexcept {
    return rl::guarded("rl_ppo_loss", [&] {
        rl::require(mean && value && std_param && actions && old_log_probs && old_values && advantages && returns &&
                        dmean && dvalue && dstd_rows && row_terms && totals && rows > 0 && action_dim > 0,
                    "PPO loss needs every input and output buffer.");
        const long long blocks = (rows + Q::kRowsPerBlock - 1) / Q::kRowsPerBlock;
        rl::require(blocks <= (1LL << 30), "PPO loss row count is too large.");
        Q::LossArgs a{mean, ld_mean, value, 1, std_param, actions, old_log_probs, old_values, advantages, returns,
                      rows, action_dim, std_type, std_min, std_max, clip_ratio, value_coefficient,
                      entropy_coefficient, value_loss_scale, clip_value, dmean, dvalue, 1, dstd_rows, row_terms,
                      nullptr, nullptr, false};
        const hipStream_t st = rl::as_stream(stream);
        hipLaunchKernelGGL(Q::loss_kernel, dim3(static_cast<unsigned>(blocks)), dim3(Q::kRowThreads), 0, st, a);
        rl::check_launch("Launch PPO loss");
        hipLaunchKernelGGL(Q::sum_rows_kernel, dim3(1), dim3(Q::kThreads), 0, st, row_terms, blocks, 4, totals);
        rl::check_launch("Launch PPO loss reduction");
    });
}

RL_API int rl_ppo_minibatch_loss(const float* mean, long long ld_mean, const float* value, long long ld_value,
                                 const float* std_param, const float* actions, const float* old_log_probs,
                                 const float* old_values, const float* advantages, const float* returns,
                                 const float* old_mean, const float* old_std, long long rows, int action_dim,
                                 int std_type, float std_min, float std_max, float clip_ratio, float value_coefficient,
                                 float entropy_coefficient, float value_loss_scale, int clip_value, float desired_kl,
                                 int adapt, float* dmean, float* dvalue, long long ld_dvalue, float* dstd,
                                 float* partial, float* totals, float* kl, float* lr, void* stream) noexcept {
    return rl::guarded("rl_ppo_minibatch_loss", [&] {
        rl::require(mean && value && std_param && actions && old_log_probs && old_values && advantages && returns &&
                        old_mean && old_std && dmean && dvalue && dstd && partial && totals && kl && lr && rows > 0,
                    "PPO minibatch loss needs every input and output buffer.");
        rl::require(action_dim > 0 && action_dim <= rl::kWave, "PPO minibatch loss supports 1..64 action dimensions.");
        const long long blocks = (rows + Q::kRowsPerBlock - 1) / Q::kRowsPerBlock;
        rl::require(blocks <= (1LL << 30), "PPO loss row count is too large.");
        rl::require(ld_value >= 1 && ld_dvalue >= 1, "PPO minibatch loss value pitches must be positive.");
        Q::LossArgs a{mean, ld_mean, value, ld_value, std_param, actions, old_log_probs, old_values, advantages,
                      returns, rows, action_dim, std_type, std_min, std_max, clip_ratio, value_coefficient,
                      entropy_coefficient, value_loss_scale, clip_value, dmean, dvalue, ld_dvalue, nullptr, partial,
                      old_mean, old_std, true};
        const hipStream_t st = rl::as_stream(stream);
        hipLaunchKernelGGL(Q::loss_kernel, dim3(static_cast<unsigned>(blocks)), dim3(Q::kRowThreads), 0, st, a);
        rl::check_launch("Launch PPO minibatch loss");
        hipLaunchKernelGGL(Q::loss_finish, dim3(1), dim3(Q::kThreads), 0, st, partial, blocks, rows, action_dim,
                           desired_kl, adapt, totals, kl, lr, dstd);
        rl::check_launch("Launch PPO minibatch loss reduction");
    });
}

// Squared L2 norm of a flat vector; partial needs ceil(n / 4096) floats.
RL_API int rl_sum_squares(const float* x, long long n, float* partial, float* out, void* stream) noexcept {
    return rl::guarded("rl_sum_squares", [&] {
        rl::require(x && partial && out && n > 0, "Sum of squares needs buffers.");
        const long long blocks = (n + 4095) / 4096;
        const hipStream_t st = rl::as_stream(stream);
        hipLaunchKernelGGL(Q::sumsq_partials, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st, x, n, partial);
        rl::check_launch("Launch sum of squares");
        hipLaunchKernelGGL(Q::sumsq_finish, dim3(1), dim3(Q::kThreads), 0, st, partial, blocks, out);
        rl::check_launch("Launch sum of squares finish");
    });
}

RL_API int rl_clip_by_norm(float* g, long long n, const float* sum_squares, float max_norm, void* stream) noexcept {
    return rl::guarded("rl_clip_by_norm", [&] {
        rl::require(g && sum_squares && n > 0 && max_norm > 0, "Clipping needs buffers and a positive norm.");
        hipLaunchKernelGGL(Q::clip_kernel, dim3(static_cast<unsigned>(std::min<long long>((n + 255) / 256, 65536))),
                           dim3(256), 0, rl::as_stream(stream), g, n, sum_squares, max_norm);
        rl::check_launch("Launch gradient clipping");
    });
}

RL_API int rl_clip_grad_norm(float* g, long long n, float* partial, float* sum_squares, float max_norm,
                             void* stream) noexcept {
    return rl::guarded("rl_clip_grad_norm", [&] {
        rl::require(g && partial && sum_squares && n > 0 && max_norm > 0,
                    "Gradient-norm clipping needs buffers and a positive norm.");
        const long long blocks = (n + 4095) / 4096;
        const hipStream_t st = rl::as_stream(stream);
        hipLaunchKernelGGL(Q::sumsq_partials, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st, g, n, partial);
        rl::check_launch("Launch sum of squares");
        hipLaunchKernelGGL(Q::clip_from_partials, dim3(static_cast<unsigned>(std::min<long long>((n + 255) / 256, 1024))),
                           dim3(Q::kThreads), 0, st, g, n, partial, blocks, sum_squares, max_norm);
        rl::check_launch("Launch gradient clipping");
    });
}

RL_API int rl_elu_backward(float* dx, const float* y, long long n, void* stream) noexcept {
    return rl::guarded("rl_elu_backward", [&] {
        rl::require(dx && y && n > 0, "ELU backward needs buffers.");
        hipLaunchKernelGGL(Q::elu_backward_kernel,
                           dim3(static_cast<unsigned>(std::min<long long>((n + 255) / 256, 65536))), dim3(256), 0,
                           rl::as_stream(stream), dx, y, n);
        rl::check_launch("Launch ELU backward");
    });
}
