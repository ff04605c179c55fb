"""Replay ingest (n-step staging and commit) and return statistics on the GPU,
against the reference's known answer and the CPU oracle (oracle.replay).

Committed rows are compared bit for bit: the kernel rounds every product and
sum in the reference's order.  The running mean/variance of the return
statistics are fixed-order block sums, within 1e-5 relative of the oracle.
"""

import numpy as np
import pytest
import torch

from oracle import replay as OR
from robolearn_amd import _native
from robolearn_amd import kernels as K

pytestmark = pytest.mark.gpu

FIELDS = ("observation", "action", "reward", "terminated", "truncated", "next_observation", "discount")


class DeviceReplay:
    """Storage, staging ring and counters laid out as the C-ABI expects."""

    def __init__(self, device, envs, obs_dim, action_dim, n_step, capacity, gamma):
        self.envs, self.obs_dim, self.action_dim = envs, obs_dim, action_dim
        self.n_step, self.capacity, self.gamma = n_step, capacity, gamma
        z = lambda *shape: torch.full(shape, float("nan"), device=device)  # unwritten rows stay NaN
        self.store = {"observation": z(capacity, obs_dim), "action": z(capacity, action_dim),
                      "reward": z(capacity), "terminated": z(capacity), "truncated": z(capacity),
                      "next_observation": z(capacity, obs_dim), "discount": z(capacity)}
        self.pending = {"observation": z(n_step, envs, obs_dim), "action": z(n_step, envs, action_dim),
                        "next_observation": z(n_step, envs, obs_dim), "scalars": z(n_step, envs, 3)}
        self.counters = torch.zeros(3, dtype=torch.long, device=device)
        self.device = device

    def add(self, step):
        t = {k: torch.as_tensor(np.asarray(v, np.float32)).to(self.device).contiguous() for k, v in step.items()}
        s, p = self.store, self.pending
        _native.call("rl_replay_ingest", self.envs, self.obs_dim, self.action_dim, self.n_step, self.capacity,
                     float(self.gamma), t["observation"].data_ptr(), t["action"].data_ptr(), t["reward"].data_ptr(),
                     t["terminated"].data_ptr(), t["truncated"].data_ptr(), t["next_observation"].data_ptr(),
                     p["observation"].data_ptr(), p["action"].data_ptr(), p["next_observation"].data_ptr(),
                     p["scalars"].data_ptr(), *[s[k].data_ptr() for k in FIELDS], self.counters.data_ptr(),
                     K.stream())
        torch.cuda.synchronize()


def _step(rng, envs, obs_dim, action_dim, done_prob):
    return dict(observation=rng.standard_normal((envs, obs_dim)).astype(np.float32),
                action=rng.uniform(-1, 1, (envs, action_dim)).astype(np.float32),
                reward=(rng.standard_normal(envs) * 3).astype(np.float32),
                terminated=(rng.random(envs) < done_prob).astype(np.float32),
                truncated=(rng.random(envs) < done_prob).astype(np.float32),
                next_observation=rng.standard_normal((envs, obs_dim)).astype(np.float32))


def test_replay_ingest_reference_known_answer(gpu):
    """tests/test_flashsac.py:197-231 of the reference, through the C-ABI."""
    print("case ingest known answer n=3 gamma=0.5", flush=True)
    replay = DeviceReplay(gpu, 3, 1, 1, n_step=3, capacity=16, gamma=0.5)
    for step, rewards in enumerate(([1.0, 1.0, 1.0], [2.0, 2.0, 2.0], [100.0, 4.0, 100.0])):
        replay.add(dict(observation=[[step * 10.0], [step * 10.0 + 1], [step * 10.0 + 2]],
                        action=np.zeros((3, 1)), reward=rewards,
                        terminated=[0.0, 0.0, float(step == 1)], truncated=[float(step == 1), 0.0, 0.0],
                        next_observation=[[(step + 1) * 10.0], [(step + 1) * 10.0 + 1], [(step + 1) * 10.0 + 2]]))
        assert replay.counters.tolist() == [step + 1, 0 if step < 2 else 3, 0 if step < 2 else 3]
    s = {k: v[:3].cpu() for k, v in replay.store.items()}
    torch.testing.assert_close(s["reward"], torch.tensor([2.0, 3.0, 2.0]), rtol=0, atol=0)
    torch.testing.assert_close(s["next_observation"], torch.tensor([[20.0], [31.0], [22.0]]), rtol=0, atol=0)
    torch.testing.assert_close(s["discount"], torch.tensor([0.25, 0.125, 0.25]), rtol=0, atol=0)
    torch.testing.assert_close(s["terminated"], torch.tensor([0.0, 0.0, 1.0]), rtol=0, atol=0)
    torch.testing.assert_close(s["truncated"], torch.tensor([1.0, 0.0, 0.0]), rtol=0, atol=0)
    torch.testing.assert_close(s["observation"], torch.tensor([[0.0], [1.0], [2.0]]), rtol=0, atol=0)
    assert torch.isnan(replay.store["reward"][3:]).all()


@pytest.mark.parametrize("n_step,envs,obs_dim,action_dim,capacity", [
    (1, 37, 11, 3, 100), (3, 37, 11, 3, 100), (5, 64, 4, 9, 256), (2, 1, 1, 1, 3)])
def test_replay_ingest_matches_oracle(gpu, n_step, envs, obs_dim, action_dim, capacity):
    print(f"case ingest n={n_step} envs={envs} obs={obs_dim} act={action_dim} cap={capacity}", flush=True)
    rng = np.random.default_rng(n_step * 100 + envs)
    gamma = 0.99
    replay = DeviceReplay(gpu, envs, obs_dim, action_dim, n_step, capacity, gamma)
    oracle = OR.NStepReplay(obs_dim, action_dim, n_step, gamma, capacity)
    for step in range(12):
        t = _step(rng, envs, obs_dim, action_dim, done_prob=0.25)
        replay.add(t)
        oracle.add(**t)
        assert replay.counters.tolist() == [step + 1, oracle.position, oracle.count], step
        rows = np.arange(oracle.count)
        for key in FIELDS:
            got = replay.store[key].cpu().numpy()[rows]
            np.testing.assert_array_equal(got, oracle.storage[key][rows], err_msg=f"{key} after step {step}")


@pytest.mark.parametrize("envs", [5, 1000, 4099])
def test_reward_stats_match_oracle(gpu, envs):
    print(f"case reward statistics envs={envs}", flush=True)
    rng = np.random.default_rng(envs)
    gamma = 0.99
    oracle = OR.RewardStats(envs, gamma)
    returns = torch.zeros(envs, device=gpu)
    maximum = torch.zeros(1, device=gpu)
    running = torch.tensor([0.0, 1.0, 0.0], device=gpu)
    for step in range(10):
        reward = (rng.standard_normal(envs) * 2).astype(np.float32)
        term = (rng.random(envs) < 0.05).astype(np.float32)
        trunc = (rng.random(envs) < 0.05).astype(np.float32)
        r, te, tr = (torch.as_tensor(v).to(gpu) for v in (reward, term, trunc))
        _native.call("rl_reward_stats_update", envs, gamma, r.data_ptr(), te.data_ptr(), tr.data_ptr(),
                     returns.data_ptr(), maximum.data_ptr(), running.data_ptr(), K.stream())
        oracle.update(reward, term, trunc)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(returns.cpu().numpy(), oracle.returns, err_msg=f"returns, step {step}")
        np.testing.assert_array_equal(maximum.cpu().numpy(), oracle.maximum)
        np.testing.assert_allclose(running.cpu().numpy(), oracle.running, rtol=1e-5, atol=1e-7)
    # the normalized batch the update consumes (reward_normalization.py:28-38)
    batch = torch.randn(257, generator=torch.Generator().manual_seed(1))
    device_batch = batch.to(gpu)
    _native.call("rl_scale_rewards", device_batch.data_ptr(), 257, running[1:2].data_ptr(), maximum.data_ptr(),
                 5.0, 1e-8, K.stream())
    expected = batch.numpy() / np.maximum(np.sqrt(running[1].item() + np.float32(1e-8)),
                                          maximum.item() / np.float32(5.0))
    np.testing.assert_allclose(device_batch.cpu().numpy(), expected, rtol=1e-6)


def _small_agent(n_step=3, normalize_reward=True, envs=8):
    from robolearn_amd.config import FlashSACConfig
    from robolearn_amd.flashsac import FlashSAC

    cfg = FlashSACConfig(seed=3, n_step=n_step, normalize_reward=normalize_reward, sample_batch_size=16,
                         buffer_max_length=64, buffer_min_length=16, actor_hidden_dim=32, actor_num_blocks=1,
                         critic_hidden_dim=32, critic_num_blocks=1, critic_num_bins=21)
    return FlashSAC(5, 2, num_envs=envs, cfg=cfg)


def test_agent_observe_commits_n_step_returns_and_updates(gpu):
    print("case agent observe n_step=3 normalize_reward", flush=True)
    agent = _small_agent()
    rng = np.random.default_rng(7)
    oracle = OR.NStepReplay(5, 2, 3, agent.cfg.gamma, agent.capacity)
    stats = OR.RewardStats(agent.num_envs, agent.cfg.gamma)
    for step in range(6):
        t = _step(rng, agent.num_envs, 5, 2, done_prob=0.2)
        t["terminated"] = t["terminated"].astype(bool)  # flags may arrive as booleans
        agent.process_transition(t)
        oracle.add(**t)
        stats.update(t["reward"], t["terminated"], t["truncated"])
    torch.cuda.synchronize()
    assert agent._num_in_buffer_host == oracle.count == 32 and agent.ready
    assert agent.replay_counters.tolist() == [6, oracle.position, oracle.count]
    for key in FIELDS:
        np.testing.assert_array_equal(agent.replay[key][:32].cpu().numpy(), oracle.storage[key][:32], err_msg=key)
    np.testing.assert_array_equal(agent.reward_returns.cpu().numpy(), stats.returns)
    np.testing.assert_allclose(agent.reward_running.cpu().numpy(), stats.running, rtol=1e-5)
    metrics = agent.update(capture=False)
    assert metrics and all(np.isfinite(v) for v in metrics.values())

    # a checkpoint with replay continues the staging exactly
    state = agent.state_dict(include_replay=True)
    restored = _small_agent()
    restored.load_state_dict(state)
    for step in range(3):
        t = _step(rng, agent.num_envs, 5, 2, done_prob=0.2)
        fields = [t[k] for k in ("observation", "action", "reward", "terminated", "truncated", "next_observation")]
        agent.observe(*fields)
        restored.observe(*fields)
    torch.cuda.synchronize()
    assert restored.replay_counters.tolist() == agent.replay_counters.tolist()
    for key in FIELDS:
        torch.testing.assert_close(restored.replay[key], agent.replay[key], rtol=0, atol=0, equal_nan=True)


def test_agent_observe_rejects_wrong_environment_count(gpu):
    agent = _small_agent(envs=4)
    t = _step(np.random.default_rng(0), 3, 5, 2, done_prob=0.0)
    with pytest.raises(ValueError):
        agent.process_transition(t)
