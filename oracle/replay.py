"""CPU restatement of replay ingest and reward statistics (TEST INFRASTRUCTURE ONLY).

numpy float32 arithmetic, rounded one operation at a time in the reference's
order:
  NStepReplay.add     robolearn/flashsac/replay.py:107-174 (TorchUniformBuffer.add
                      and _get_n_step_prev_transition): a deque of the last n
                      vector steps; once full, the oldest step is committed with
                      its n-step return, discount, terminal flags and bootstrap
                      observation at ring rows (position + e) % capacity
  NStepReplay.sample  robolearn/flashsac/replay.py:179-194 with injected indices
  RewardStats.update  robolearn/flashsac/_utils/reward_normalization.py:14-25
                      (_update_reward_stats), 108-122 (update_reward_stats) and
                      42-66, 187-197 (RunningMeanStd.update, epsilon 1e-4)
  RewardStats.scale   reward_normalization.py:28-38 (_scale_reward)

Parity pinning (tests/test_oracle.py):
  * NStepReplay against the reference's known answer
    tests/test_flashsac.py:197-231 (n = 3, gamma = 0.5: rewards 2 / 3 / 2,
    bootstrap observations 20 / 31 / 22, discounts 0.25 / 0.125 / 0.25, the
    timeout keeps its bootstrap, the termination suppresses it), and against a
    float64 brute force that recomputes every committed row from the full
    transition history (first done within the window, discounted sum up to it);
  * RewardStats against the closed forms: G_r is the per-environment discounted
    return since the last done; the running mean is the mean of every G_r value
    seen so far; running_var * count equals the total sum of squares about that
    mean plus 1e-4 times the sum of the previous running variances (the
    epsilon term of the merge), starting from var = 1, count = 0.
"""

import numpy as np

f32 = np.float32


class NStepReplay:
    """TorchUniformBuffer with float32 storage and injected sample indices."""

    FIELDS = ("observation", "action", "reward", "terminated", "truncated", "next_observation", "discount")

    def __init__(self, obs_dim, action_dim, n_step, gamma, capacity):
        self.n_step, self.gamma, self.capacity = int(n_step), f32(gamma), int(capacity)
        self.storage = {
            "observation": np.zeros((capacity, obs_dim), np.float32),
            "action": np.zeros((capacity, action_dim), np.float32),
            "next_observation": np.zeros((capacity, obs_dim), np.float32),
            **{k: np.zeros(capacity, np.float32) for k in ("reward", "terminated", "truncated", "discount")},
        }
        self.window = []  # deque(maxlen=n_step), oldest first
        self.count = 0
        self.position = 0

    def add(self, observation, action, reward, terminated, truncated, next_observation):
        step = {
            "observation": np.array(observation, np.float32),
            "action": np.array(action, np.float32),
            "reward": np.array(reward, np.float32),
            "terminated": np.array(terminated, np.float32),
            "truncated": np.array(truncated, np.float32),
            "next_observation": np.array(next_observation, np.float32),
        }
        self.window.append(step)
        if len(self.window) > self.n_step:
            self.window.pop(0)
        if len(self.window) < self.n_step:
            return
        g = self.gamma
        last = self.window[-1]
        reward = last["reward"].copy()
        term = last["terminated"].copy()
        trunc = last["truncated"].copy()
        next_obs = last["next_observation"].copy()
        discount = np.full_like(reward, g)
        for idx in reversed(range(self.n_step - 1)):  # replay.py:133-148
            t = self.window[idx]
            done = (t["terminated"] != 0) | (t["truncated"] != 0)
            keep = (f32(1.0) - done.astype(np.float32))
            reward = (t["reward"] + (g * reward) * keep).astype(np.float32)
            discount = np.where(done, g, (g * discount).astype(np.float32)).astype(np.float32)
            term[done] = t["terminated"][done]
            trunc[done] = t["truncated"][done]
            next_obs[done] = t["next_observation"][done]
        first = self.window[0]
        n = len(reward)
        rows = (np.arange(n) + self.position) % self.capacity
        s = self.storage
        s["observation"][rows] = first["observation"]
        s["action"][rows] = first["action"]
        s["next_observation"][rows] = next_obs
        s["reward"][rows] = reward
        s["terminated"][rows] = term
        s["truncated"][rows] = trunc
        s["discount"][rows] = discount
        self.count = min(self.count + n, self.capacity)
        self.position = (self.position + n) % self.capacity

    def sample(self, idx):
        idx = np.asarray(idx, np.int64)
        return {k: self.storage[k][idx] for k in self.FIELDS}


def brute_force_commit(history, n_step, gamma):
    """Committed row of each environment for the window ending at the last step of
    `history` (a list of steps, oldest first), recomputed in float64: the return
    sums rewards from the window's first step up to and including its first
    done step (or the window's last step), discounted by gamma per step."""
    window = history[-n_step:]
    envs = len(window[0]["reward"])
    out = {k: [] for k in ("reward", "discount", "terminated", "truncated", "next_observation")}
    for e in range(envs):
        total, stop = 0.0, n_step - 1
        for k, t in enumerate(window):
            total += gamma ** k * float(t["reward"][e])
            if t["terminated"][e] != 0 or t["truncated"][e] != 0:
                stop = k
                break
        out["reward"].append(total)
        out["discount"].append(gamma ** (stop + 1))
        out["terminated"].append(float(window[stop]["terminated"][e]))
        out["truncated"].append(float(window[stop]["truncated"][e]))
        out["next_observation"].append(np.asarray(window[stop]["next_observation"][e], np.float64))
    return {k: np.array(v) for k, v in out.items()}


class RewardStats:
    """RewardNormalizer: per-environment returns, running max |G_r| and RunningMeanStd."""

    def __init__(self, num_envs, gamma, epsilon=1e-4):
        self.gamma = f32(gamma)
        self.returns = np.zeros(num_envs, np.float32)
        self.maximum = np.zeros(1, np.float32)
        self.running = np.array([0.0, 1.0, 0.0], np.float32)  # mean, var, count
        self.epsilon = f32(epsilon)

    def update(self, reward, terminated, truncated):
        reward = np.asarray(reward, np.float32)
        done = ((np.asarray(terminated) != 0) | (np.asarray(truncated) != 0)).astype(np.float32)
        keep = (self.gamma * (f32(1.0) - done)).astype(np.float32)
        self.returns = ((keep * self.returns).astype(np.float32) + reward).astype(np.float32)
        self.maximum = np.maximum(self.maximum, np.abs(self.returns).max()).astype(np.float32)
        x = self.returns
        count = f32(x.shape[0])
        mean = f32(x.mean(dtype=np.float32))
        var = f32(((x - mean) ** 2).mean(dtype=np.float32))
        old_mean, old_var, old_count = self.running
        delta = f32(mean - old_mean)
        total = f32(old_count + count)
        ratio = f32(count / total)
        m_a = f32(old_var * f32(old_count + self.epsilon))
        m_b = f32(var * count)
        self.running = np.array([old_mean + delta * ratio,
                                 (m_a + m_b + delta * delta * old_count * ratio) / total, total], np.float32)

    def scale(self, rewards, g_max, eps=1e-8):
        denominator = np.maximum(np.sqrt(self.running[1] + f32(eps)), self.maximum[0] / f32(g_max))
        return (np.asarray(rewards, np.float32) / denominator).astype(np.float32)
