// Replay ingest: n-step staging and commit into the device ring, and the
// return statistics behind reward normalization.
//
// Ingest follows robolearn/flashsac/replay.py:107-174 (TorchUniformBuffer.add
// and _get_n_step_prev_transition) with the persistent device staging of
// robolearn/warp/_flash_replay.py:26-113: one vector step of E transitions is
// staged in slot (additions % n) of an n-slot ring, and once n - 1 earlier
// steps are staged the oldest one is committed with its n-step return.  The
// walk goes from the newest transition back; a done (terminated or truncated)
// transition restarts the return at its own reward and supplies the terminal
// flags and the bootstrap observation.  Products and sums are rounded one at a
// time in the reference's order (contraction into fused multiply-adds is off in
// these kernels), so committed rewards and discounts are bit-identical to the
// fp32 reference.
//
// Counters (int64[3], device): [0] vector steps added, [1] next ring row,
// [2] committed rows (at most the capacity).
//
// Return statistics follow robolearn/flashsac/_utils/reward_normalization.py:
// 14-25 (G_r update and running maximum), 42-66 and 187-197 (RunningMeanStd
// merge with epsilon 1e-4); device state as robolearn/warp/_flash_replay.py:
// 347-389 (returns [E], maximum [1], running = [mean, var, count]).  The batch
// mean and variance are fixed-order block reductions (the reference's device
// path uses atomics).

#include "common.hpp"

namespace rl {
namespace replay {

constexpr int kThreads = 256;

struct IngestArgs {
    const float* observation;
    const float* action;
    const float* reward;
    const float* terminated;
    const float* truncated;
    const float* next_observation;
    float* pending_observation;       // [n][E][O]
    float* pending_action;            // [n][E][A]
    float* pending_next_observation;  // [n][E][O]
    float* pending_scalars;           // [n][E][3]: reward, terminated, truncated
    float* observation_store;         // [capacity][O]
    float* action_store;              // [capacity][A]
    float* reward_store;
    float* terminated_store;
    float* truncated_store;
    float* next_observation_store;    // [capacity][O]
    float* discount_store;
    const long long* counters;
    long long num_envs;
    long long capacity;
    int obs_dim;
    int action_dim;
    int width;  // max(obs_dim, action_dim)
    int n_step;
    float gamma;
};

// One thread per (environment, column < width).  Every thread reads the newest
// transition from the inputs and older ones from the staging ring, so no thread
// depends on a value another thread of this launch writes.
__global__ __launch_bounds__(kThreads) void ingest_kernel(IngestArgs a) {
#pragma clang fp contract(off)
    const long long t = blockIdx.x * static_cast<long long>(kThreads) + threadIdx.x;
    if (t >= a.num_envs * a.width) return;
    const long long i = t / a.width;
    const int j = static_cast<int>(t % a.width);
    const int n = a.n_step;
    const int O = a.obs_dim;
    const int A = a.action_dim;
    const long long additions = a.counters[0];
    const int latest = static_cast<int>(additions % n);
    const auto row = [&](int slot) { return static_cast<long long>(slot) * a.num_envs + i; };

    const float reward = a.reward[i];
    const float terminated = a.terminated[i];
    const float truncated = a.truncated[i];
    if (j < O) {
        a.pending_observation[row(latest) * O + j] = a.observation[i * O + j];
        a.pending_next_observation[row(latest) * O + j] = a.next_observation[i * O + j];
    }
    if (j < A) a.pending_action[row(latest) * A + j] = a.action[i * A + j];
    if (j == 0) {
        float* s = a.pending_scalars + row(latest) * 3;
        s[0] = reward;
        s[1] = terminated;
        s[2] = truncated;
    }
    if (additions < n - 1) return;  // fewer than n steps staged: nothing to commit yet

    float total = reward;
    float factor = a.gamma;
    float terminal = terminated;
    float timeout = truncated;
    int next_slot = latest;
    for (int offset = 1; offset < n; ++offset) {
        const int slot = (latest - offset + n) % n;
        const float* s = a.pending_scalars + row(slot) * 3;
        const float r = s[0];
        if (s[1] != 0.0f || s[2] != 0.0f) {
            total = r;
            factor = a.gamma;
            terminal = s[1];
            timeout = s[2];
            next_slot = slot;
        } else {
            total = r + a.gamma * total;
            factor = a.gamma * factor;
        }
    }
    const int oldest = (latest + 1) % n;  // equals latest only when n == 1
    const long long target = (a.counters[1] + i) % a.capacity;
    if (j < O) {
        a.observation_store[target * O + j] =
            oldest == latest ? a.observation[i * O + j] : a.pending_observation[row(oldest) * O + j];
        a.next_observation_store[target * O + j] =
            next_slot == latest ? a.next_observation[i * O + j] : a.pending_next_observation[row(next_slot) * O + j];
    }
    if (j < A) {
        a.action_store[target * A + j] = oldest == latest ? a.action[i * A + j] : a.pending_action[row(oldest) * A + j];
    }
    if (j == 0) {
        a.reward_store[target] = total;
        a.terminated_store[target] = terminal;
        a.truncated_store[target] = timeout;
        a.discount_store[target] = factor;
    }
}

// Runs after ingest_kernel on the same stream.
__global__ void advance_kernel(long long* counters, int n_step, long long num_envs, long long capacity) {
    if (blockIdx.x != 0 || threadIdx.x != 0) return;
    const long long additions = counters[0];
    if (additions >= n_step - 1) {
        counters[1] = (counters[1] + num_envs) % capacity;
        counters[2] = min(counters[2] + num_envs, capacity);
    }
    counters[0] = additions + 1;
}

constexpr int kStatThreads = 1024;

__device__ __forceinline__ float block_max(float value, float* scratch) {
    value = wave_max(value);
    const int wave = threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    __syncthreads();
    if (lane == 0) scratch[wave] = value;
    __syncthreads();
    float result = scratch[0];
#pragma unroll
    for (int w = 1; w < kStatThreads / kWave; ++w) result = fmaxf(result, scratch[w]);
    return result;
}

// One workgroup: G_r = gamma (1 - done) G_r + r per environment, the running
// maximum of |G_r|, then the batch mean and (population) variance of G_r
// merged into running = [mean, var, count].
__global__ __launch_bounds__(kStatThreads) void reward_stats_kernel(long long num_envs, float gamma,
                                                                     const float* reward, const float* terminated,
                                                                     const float* truncated, float* returns,
                                                                     float* maximum, float* running) {
#pragma clang fp contract(off)
    __shared__ float scratch[3][kStatThreads / kWave];
    float sum = 0.0f;
    float largest = 0.0f;
    for (long long i = threadIdx.x; i < num_envs; i += kStatThreads) {
        const bool done = terminated[i] != 0.0f || truncated[i] != 0.0f;
        const float keep = gamma * (done ? 0.0f : 1.0f);
        const float value = keep * returns[i] + reward[i];
        returns[i] = value;
        sum += value;
        largest = fmaxf(largest, fabsf(value));
    }
    const float count = static_cast<float>(num_envs);
    const float mean = block_sum<kStatThreads>(sum, scratch[0]) / count;
    largest = block_max(largest, scratch[1]);
    float squares = 0.0f;
    for (long long i = threadIdx.x; i < num_envs; i += kStatThreads) {  // this thread's own values, written above
        const float d = returns[i] - mean;
        squares += d * d;
    }
    const float variance = block_sum<kStatThreads>(squares, scratch[2]) / count;
    if (threadIdx.x == 0) {
        maximum[0] = fmaxf(maximum[0], largest);
        const float old_mean = running[0];
        const float old_var = running[1];
        const float old_count = running[2];
        const float delta = mean - old_mean;
        const float total = old_count + count;
        const float ratio = count / total;
        const float m_a = old_var * (old_count + 1.0e-4f);
        const float m_b = variance * count;
        running[0] = old_mean + delta * ratio;
        running[1] = (m_a + m_b + delta * delta * old_count * ratio) / total;
        running[2] = total;
    }
}

}  // namespace replay
}  // namespace rl

namespace R = rl::replay;

RL_API int rl_replay_ingest(long long num_envs, int obs_dim, int action_dim, int n_step, long long capacity,
                            float gamma, const float* observation, const float* action, const float* reward,
                            const float* terminated, const float* truncated, const float* next_observation,
                            float* pending_observation, float* pending_action, float* pending_next_observation,
                            float* pending_scalars, float* observation_store, float* action_store, float* reward_store,
                            float* terminated_store, float* truncated_store, float* next_observation_store,
                            float* discount_store, long long* counters, void* stream) noexcept {
    return rl::guarded("rl_replay_ingest", [&] {
        rl::require(num_envs > 0 && obs_dim > 0 && action_dim > 0 && n_step > 0, "Replay ingest needs positive sizes.");
        rl::require(capacity >= num_envs, "Replay capacity must hold one vector step.");
        rl::require(observation && action && reward && terminated && truncated && next_observation,
                    "Replay ingest needs every transition field.");
        rl::require(pending_observation && pending_action && pending_next_observation && pending_scalars,
                    "Replay ingest needs the n-step staging buffers.");
        rl::require(observation_store && action_store && reward_store && terminated_store && truncated_store &&
                        next_observation_store && discount_store && counters,
                    "Replay ingest needs the storage fields and counters.");
        const int width = std::max(obs_dim, action_dim);
        R::IngestArgs a{observation, action, reward, terminated, truncated, next_observation,
                        pending_observation, pending_action, pending_next_observation, pending_scalars,
                        observation_store, action_store, reward_store, terminated_store, truncated_store,
                        next_observation_store, discount_store, counters, num_envs, capacity, obs_dim, action_dim,
                        width, n_step, gamma};
        hipStream_t st = rl::as_stream(stream);
        hipLaunchKernelGGL(R::ingest_kernel, dim3(rl::ceil_div(num_envs * width, R::kThreads)), dim3(R::kThreads), 0,
                           st, a);
        rl::check_launch("Launch replay ingest");
        hipLaunchKernelGGL(R::advance_kernel, dim3(1), dim3(1), 0, st, counters, n_step, num_envs, capacity);
        rl::check_launch("Launch replay counter advance");
    });
}

RL_API int rl_reward_stats_update(long long num_envs, float gamma, const float* reward, const float* terminated,
                                  const float* truncated, float* returns, float* maximum, float* running,
                                  void* stream) noexcept {
    return rl::guarded("rl_reward_stats_update", [&] {
        rl::require(num_envs > 0, "Reward statistics need at least one environment.");
        rl::require(reward && terminated && truncated && returns && maximum && running,
                    "Reward statistics need rewards, flags and state buffers.");
        hipLaunchKernelGGL(R::reward_stats_kernel, dim3(1), dim3(R::kStatThreads), 0, rl::as_stream(stream), num_envs,
                           gamma, reward, terminated, truncated, returns, maximum, running);
        rl::check_launch("Launch reward statistics");
    });
}
