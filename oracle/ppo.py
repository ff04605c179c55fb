"""CPU restatement of the PPO update (TEST INFRASTRUCTURE ONLY).

Follows robolearn/warp/ppo.py:
  _gae :101-133                  reverse scan, time-major k = t E + i, timeout modes
  _advantage_* :136-159          two-pass normalization (population or sample std)
  launch_update :586-695         one permutation reused across all epochs;
                                 per minibatch: KL on the pre-step policy and the
                                 adaptive LR rule (:207-238), clipped surrogate /
                                 clipped value / entropy loss (:255-310),
                                 gradient clipping (:241-252, 676-693), Adam
  _mlp :313-350                  Linear + ELU/Tanh MLPs, U(+-1/sqrt(fan_in)) init
  _sample :26-58                 rollout actions, log-probs and values (sample)
with the Torch formulas of the reference's own parity harness
(examples/diagnose_ppo_update.py:75-162), including torch.optim.Adam.

Parity pinning: GAE, advantage normalization and the loss with its gradients
are pinned by the reference's known-answer tests (tests/test_warp_ppo.py:23-119,
restated in tests/test_oracle.py); the KL expression by the closed form of the
Gaussian KL; Adam by torch.optim.Adam itself; the rollout log-prob by
torch.distributions.Normal.log_prob of the same actions.  Gradient clipping
(``clip_gradients``) is pinned by its closed form in tests/test_oracle.py: below
the threshold the gradients are unchanged, above it the post-clip norm is
max_norm ||g|| / (||g|| + 1e-6), for one group and for the combined group.
The combined (non-separate) mode applies that rule to all parameters as one
group, standing in for Warp-NN's Adam ``max_norm`` option, whose source is not
in the reference tree (warp-nn 0.4.0, uv.lock:1244-1245): where Warp-NN places
its epsilon stays parity unpinned.  The minibatch permutation is injected (the
device one is read back).
"""

import math

import numpy as np
import torch
import torch.nn.functional as F


def init_mlp(input_dim, output_dim, hidden_dims, rng: np.random.Generator):
    """Weights then bias per layer from U(-1/sqrt(in), 1/sqrt(in)), as ppo.py:333-343."""
    params = []
    widths = (input_dim, *hidden_dims, output_dim)
    for in_dim, out_dim in zip(widths[:-1], widths[1:]):
        bound = 1.0 / math.sqrt(in_dim)
        params.append(rng.uniform(-bound, bound, (out_dim, in_dim)).astype(np.float32))
        params.append(rng.uniform(-bound, bound, (out_dim,)).astype(np.float32))
    return params


def init_parameters(observation_dim, action_dim, cfg):
    """Actor MLP, critic MLP, distribution parameter (WarpPPO.__init__, ppo.py:396-424)."""
    rng = np.random.default_rng(cfg.seed)
    actor = init_mlp(observation_dim, action_dim, cfg.hidden_dims, rng)
    critic = init_mlp(observation_dim, 1, cfg.hidden_dims, rng)
    std = math.log(cfg.initial_std) if cfg.std_type == "log" else cfg.initial_std
    return actor + critic + [np.full(action_dim, std, dtype=np.float32)]


def mlp(inputs, layers, activation):
    x = inputs
    for index in range(0, len(layers), 2):
        x = F.linear(x, layers[index], layers[index + 1])
        if index < len(layers) - 2:
            x = F.elu(x) if activation == "elu" else torch.tanh(x)
    return x


def gae(rewards, values, next_values, terminated, truncated, horizon, num_envs, gamma, lam,
        timeout_bootstrap="next"):
    """_gae (ppo.py:101-133) over time-major flat arrays; returns (advantages, returns)."""
    rewards, values, next_values = (torch.as_tensor(a).double() for a in (rewards, values, next_values))
    terminated = torch.as_tensor(terminated).long()
    truncated = torch.as_tensor(truncated).long()
    advantages = torch.zeros_like(rewards)
    returns = torch.zeros_like(rewards)
    for i in range(num_envs):
        advantage = 0.0
        for step in reversed(range(horizon)):
            k = step * num_envs + i
            bootstrap = 0.0 if terminated[k] != 0 else 1.0
            continuation = 0.0 if (terminated[k] != 0 or truncated[k] != 0) else 1.0
            next_value = next_values[k]
            if timeout_bootstrap == "current" and truncated[k] != 0:
                next_value = values[k]
                bootstrap = 1.0
            delta = rewards[k] + gamma * bootstrap * next_value - values[k]
            advantage = delta + gamma * lam * continuation * advantage
            advantages[k] = advantage
            returns[k] = advantage + values[k]
    return advantages, returns


def normalize(advantages, sample_std: bool):
    """_advantage_sum/_variance/_normalize (ppo.py:136-159)."""
    n = advantages.numel()
    mean = advantages.sum() / n
    sq = ((advantages - mean) ** 2).sum()
    if sample_std:
        return (advantages - mean) / (torch.sqrt(sq / max(n - 1.0, 1.0)) + 1e-8)
    return (advantages - mean) / torch.sqrt(sq / n + 1e-8)


def std_of(parameter, cfg):
    if cfg.std_type == "scalar":
        return parameter.clamp(*cfg.std_range)
    return torch.exp(parameter)


def sample(mean, value, parameter, noise, cfg):
    """Rollout sampling, ppo.py:26-58: actions = mean + std * noise, the Gaussian log-prob summed over
    action dimensions (log std = p for "log", log(clamp(p)) for "scalar"), values = value[:, 0]."""
    std = std_of(parameter, cfg)
    log_std = torch.log(std) if cfg.std_type == "scalar" else parameter
    actions = mean + std * noise
    log_probs = (-0.5 * (noise * noise + 2.0 * log_std + math.log(2.0 * math.pi))).sum(-1)
    return actions, log_probs, value[:, 0], std


def loss_terms(mean, value, parameter, actions, old_log_probs, old_values, advantages, returns, cfg):
    """loss_kernel (ppo.py:255-310); returns (loss, policy, value, entropy) means."""
    std = std_of(parameter, cfg)
    log_std = torch.log(std)
    residual = (actions - mean) * torch.exp(-log_std)
    log_prob = (-0.5 * (residual * residual + 2.0 * log_std + math.log(2 * math.pi))).sum(-1)
    entropy = (log_std + 0.5 * math.log(2 * math.pi * math.e)).sum(-1).expand_as(log_prob)
    ratio = torch.exp(log_prob - old_log_probs)
    policy = -torch.minimum(ratio * advantages,
                            ratio.clamp(1.0 - cfg.clip_ratio, 1.0 + cfg.clip_ratio) * advantages)
    value = value[:, 0]
    value_loss = (value - returns) ** 2
    if cfg.clip_value:
        clipped = old_values + (value - old_values).clamp(-cfg.clip_ratio, cfg.clip_ratio)
        value_loss = torch.maximum(value_loss, (clipped - returns) ** 2)
    value_loss = cfg.value_loss_scale * value_loss
    total = policy + cfg.value_coefficient * value_loss - cfg.entropy_coefficient * entropy
    return total.mean(), policy.mean(), value_loss.mean(), entropy.mean()


def gaussian_kl(old_mean, old_std, mean, std):
    """KL(N_old || N_new) summed over actions, as kl_kernel (ppo.py:207-230)."""
    ratio = old_std / std
    delta = (old_mean - mean) / std
    return (0.5 * (ratio * ratio + delta * delta - 1.0) - torch.log(ratio)).sum(-1)


def adapt_learning_rate(learning_rate: float, kl: float, desired_kl: float) -> float:
    """_adapt_learning_rate (robolearn/warp/ppo.py:233-238): lr / 1.5, floored at 1e-5, when the
    minibatch KL exceeds twice the target; lr * 1.5, capped at 1e-2, when 0 < KL < target / 2; both
    comparisons strict, otherwise unchanged."""
    if kl > desired_kl * 2.0:
        return max(1.0e-5, learning_rate / 1.5)
    if kl < desired_kl / 2.0 and kl > 0.0:
        return min(1.0e-2, learning_rate * 1.5)
    return learning_rate


def clip_gradients(params, max_norm: float) -> float:
    """g <- g * min(1, max_norm / (||g|| + 1e-6)) over one group (robolearn/warp/ppo.py:241-252,
    676-693, the separate-group form; the combined form clips all parameters as one group with the
    same rule, as Warp-NN's Adam(max_norm) is used at ppo.py:431-437).  Returns ||g|| before clipping."""
    return float(torch.nn.utils.clip_grad_norm_(params, max_norm))


class PPOOracle:
    def __init__(self, observation_dim, action_dim, num_envs, horizon, cfg, parameters, dtype=torch.float64):
        self.cfg = cfg
        self.num_envs, self.horizon = num_envs, horizon
        self.batch_size = num_envs * horizon
        self.mini_batch_size = self.batch_size // cfg.num_mini_batches
        self.dtype = dtype
        self.params = [torch.nn.Parameter(torch.as_tensor(np.asarray(p)).to(dtype).clone()) for p in parameters]
        layers = 2 * (len(cfg.hidden_dims) + 1)
        self.actor = self.params[:layers]
        self.critic = self.params[layers: 2 * layers]
        self.std_parameter = self.params[-1]
        self.optimizer = torch.optim.Adam(self.params, lr=cfg.learning_rate, foreach=False, fused=False)
        self.learning_rate = cfg.learning_rate
        self.last = {}

    def prepare(self, rollout: dict):
        """GAE and advantage normalization of a rollout (ppo.py:101-159); keeps the arrays."""
        cfg = self.cfg
        data = {k: torch.as_tensor(np.asarray(v)) for k, v in rollout.items()}
        advantages, returns = gae(data["rewards"], data["values"], data["next_values"], data["terminated"],
                                  data["truncated"], self.horizon, self.num_envs, cfg.gamma, cfg.gae_lambda,
                                  cfg.timeout_bootstrap)
        if cfg.normalize_advantages:
            advantages = normalize(advantages, cfg.advantage_sample_std)
        self.advantages, self.returns = advantages.clone(), returns.clone()
        self._data = data
        self._obs = data["observations"].to(self.dtype)

    def minibatch_step(self, idx) -> None:
        """One minibatch of launch_update (ppo.py:586-695) on the prepared rollout: the pre-step KL and
        adaptive learning rate, the loss, backward, gradient clipping and the Adam step."""
        cfg, dt, data = self.cfg, self.dtype, self._data
        idx = torch.as_tensor(np.asarray(idx, dtype=np.int64))
        mean = mlp(self._obs[idx], self.actor, cfg.activation)
        if cfg.schedule == "adaptive":
            with torch.no_grad():
                kl = gaussian_kl(data["means"][idx].to(dt), data["stds"][idx].to(dt), mean,
                                 std_of(self.std_parameter, cfg)).mean().item()
                self.learning_rate = adapt_learning_rate(self.learning_rate, kl, cfg.desired_kl)
                self.last["kl"] = kl
            for group in self.optimizer.param_groups:
                group["lr"] = self.learning_rate
        value = mlp(self._obs[idx], self.critic, cfg.activation)
        loss, policy, value_loss, entropy = loss_terms(
            mean, value, self.std_parameter, data["actions"][idx].to(dt), data["log_probs"][idx].to(dt),
            data["values"][idx].to(dt), self.advantages[idx].to(dt), self.returns[idx].to(dt), cfg)
        self.optimizer.zero_grad()
        loss.backward()
        if cfg.separate_grad_clipping:
            clip_gradients(self.actor + [self.std_parameter], cfg.max_grad_norm)
            clip_gradients(self.critic, cfg.max_grad_norm)
        else:
            clip_gradients(self.params, cfg.max_grad_norm)
        self.optimizer.step()
        self.last.update(loss=loss.item(), policy_loss=policy.item(), value_loss=value_loss.item(),
                         entropy=entropy.item())

    def update(self, rollout: dict, permutation) -> dict:
        """One launch_update (ppo.py:586-695) on a fixed rollout and permutation: the same permutation
        for every epoch, minibatches in order."""
        self.prepare(rollout)
        permutation = np.asarray(permutation, dtype=np.int64)
        size = self.mini_batch_size
        for _ in range(self.cfg.epochs):
            for mb in range(self.cfg.num_mini_batches):
                self.minibatch_step(permutation[mb * size: (mb + 1) * size])
        return dict(self.last, learning_rate=self.learning_rate)

    def set_state(self, parameters, moments, steps: int, learning_rate: float) -> None:
        """Parameters, Adam moments, Adam step count and learning rate taken from another
        implementation (to check one step from its state)."""
        with torch.no_grad():
            for p, value in zip(self.params, parameters):
                p.copy_(torch.as_tensor(np.asarray(value)).reshape(p.shape).to(self.dtype))
        for p, (m1, m2) in zip(self.params, moments):
            self.optimizer.state[p] = {
                "step": torch.tensor(float(steps)),
                "exp_avg": torch.as_tensor(np.asarray(m1)).reshape(p.shape).to(self.dtype).clone(),
                "exp_avg_sq": torch.as_tensor(np.asarray(m2)).reshape(p.shape).to(self.dtype).clone(),
            }
        self.learning_rate = float(learning_rate)
        for group in self.optimizer.param_groups:
            group["lr"] = self.learning_rate

    def moments(self):
        out = []
        for p in self.params:
            st = self.optimizer.state[p]
            out.append((st["exp_avg"].detach().clone(), st["exp_avg_sq"].detach().clone()))
        return out
