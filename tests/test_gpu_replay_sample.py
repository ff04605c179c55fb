"""Replay sampling (hot-path row a1) on the GPU.

* Indices: rl_replay_sample_indices equals the NumPy Philox restatement
  (oracle/philox.py, pinned by the generator authors' known answers) bit for
  bit, every index lies in [0, count) also when count < capacity, and a
  chi-square test over 2^20 draws accepts uniformity.
* Gather: rl_replay_gather equals torch indexing of the stores with the same
  indices (TorchUniformBuffer.sample(sample_idxs=...), robolearn/flashsac/
  replay.py:179-194, restated by oracle.flashsac.sample) bit for bit, at the G1
  replay size (1,048,576 rows, obs 123, act 37, batch 8192).
* The agent's own sampling inside update(), on a ring that has wrapped with a
  capacity that the environment count does not divide (as
  examples/diagnose_flash_replay.py:210-229 checks): the device indices equal
  the oracle's for the update's draw counter and the gathered batch equals the
  oracle replay's rows (oracle/replay.py NStepReplay) bit for bit.
* The update-to-data-2 pair graph (the benchmarked step) equals two eager
  update() calls bit for bit and keeps the host update step in line.
"""

import numpy as np
import pytest
import torch

from oracle import flashsac as O
from oracle import philox as PH
from oracle import replay as OR
from robolearn_amd import _native
from robolearn_amd import kernels as K
from robolearn_amd.config import FlashSACConfig

pytestmark = pytest.mark.gpu

FIELDS = ("observation", "action", "reward", "terminated", "truncated", "next_observation", "discount")


def _device_indices(gpu, seed, draw, stream_id, count, n):
    counter = torch.tensor([draw], dtype=torch.long, device=gpu)
    count_t = torch.tensor([count], dtype=torch.long, device=gpu)
    idx = torch.empty(n, dtype=torch.long, device=gpu)
    K.sample_indices(idx, seed=seed, count=count_t, counter=counter, stream_id=stream_id)
    torch.cuda.synchronize()
    return idx.cpu().numpy()


@pytest.mark.parametrize("seed,draw,stream_id,count,n", [
    (1, 0, 1, 1_048_576, 8192),          # G1: full 1,048,576-row replay, batch 8192
    (7919 * 3 + 1, 5, 1, 1000, 4097),    # count below capacity, ragged n
    (2**40 + 17, 2**33 + 9, 7, 32_000, 512),  # 64-bit seed and draw counter (c0 replay size)
    (3, 1, 1, 1, 300),                   # a single stored row
    (11, 2, 1, 3_000_000_019, 1000),     # count above 2^31
])
def test_device_indices_equal_philox_oracle(gpu, seed, draw, stream_id, count, n):
    print(f"case sample indices seed={seed} draw={draw} count={count} n={n}", flush=True)
    got = _device_indices(gpu, seed, draw, stream_id, count, n)
    expected = PH.replay_indices(seed, draw, stream_id, count, n)
    np.testing.assert_array_equal(got, expected)
    assert got.min() >= 0 and got.max() < count


def test_device_indices_are_uniform(gpu):
    print("case sample indices chi-square", flush=True)
    bins, n = 1000, 1 << 20
    got = _device_indices(gpu, 12345, 0, 1, bins, n)
    counts = np.bincount(got, minlength=bins)
    assert counts.size == bins
    expected = n / bins
    chi2 = float(((counts - expected) ** 2 / expected).sum())
    # 999 degrees of freedom: mean 999, standard deviation 44.7; accept within 6 sd
    assert abs(chi2 - (bins - 1)) < 6 * np.sqrt(2 * (bins - 1)), chi2
    # successive draws of the counter are different streams
    other = _device_indices(gpu, 12345, 1, 1, bins, 4096)
    assert (other != got[:4096]).mean() > 0.99


def _gather(gpu, store, idx, batch):
    out = {k: torch.full((batch,) + tuple(v.shape[1:]), float("nan"), device=gpu) for k, v in store.items()}
    error = torch.zeros(1, dtype=torch.int32, device=gpu)
    obs_dim, act_dim = store["observation"].shape[1], store["action"].shape[1]
    capacity = store["reward"].shape[0]
    _native.call("rl_replay_gather", idx.data_ptr(), batch, capacity, obs_dim, act_dim,
                 store["observation"].data_ptr(), store["next_observation"].data_ptr(), store["action"].data_ptr(),
                 store["reward"].data_ptr(), store["terminated"].data_ptr(), store["truncated"].data_ptr(),
                 store["discount"].data_ptr(), out["observation"].data_ptr(), out["next_observation"].data_ptr(),
                 out["action"].data_ptr(), out["reward"].data_ptr(), out["terminated"].data_ptr(),
                 out["truncated"].data_ptr(), out["discount"].data_ptr(), error.data_ptr(), K.stream())
    torch.cuda.synchronize()
    return out, int(error.item())


def test_gather_bit_exact_at_g1_replay_size(gpu):
    print("case gather G1 capacity=1048576 obs=123 act=37 batch=8192", flush=True)
    capacity, obs_dim, act_dim, batch = 1 << 20, 123, 37, 8192
    store = O.synthetic_replay(capacity, obs_dim, act_dim, seed=0, gamma=0.99, reward_std=0.5, done_prob=0.005)
    store["truncated"] = (torch.rand(capacity, generator=torch.Generator().manual_seed(9)) < 0.01).float()
    store["discount"] = torch.rand(capacity, generator=torch.Generator().manual_seed(10))
    device_store = {k: v.to(gpu) for k, v in store.items()}
    idx_host = PH.replay_indices(1, 3, 1, capacity, batch)
    idx = torch.as_tensor(idx_host).to(gpu)
    K.sample_indices(idx, seed=1, count=torch.tensor([capacity], device=gpu),
                     counter=torch.tensor([3], device=gpu), stream_id=1)
    np.testing.assert_array_equal(idx.cpu().numpy(), idx_host)
    out, error = _gather(gpu, device_store, idx, batch)
    assert error == 0
    expected = O.sample(store, idx_host)
    for key in FIELDS:
        got = out[key].cpu()
        assert got.dtype == expected[key].dtype and got.shape == expected[key].shape, key
        assert torch.equal(got, expected[key]), key


def test_gather_flags_indices_outside_the_store(gpu):
    print("case gather out-of-range index flag", flush=True)
    store = {k: v.to(gpu) for k, v in O.synthetic_replay(64, 5, 2, seed=1, gamma=0.99).items()}
    idx = torch.tensor([3, 64, -1, 7], dtype=torch.long, device=gpu)
    out, error = _gather(gpu, store, idx, 4)
    assert error == 1
    # rows with a bad index read row 0; the others are exact
    assert torch.equal(out["observation"][1], store["observation"][0])
    assert torch.equal(out["observation"][2], store["observation"][0])
    assert torch.equal(out["observation"][3], store["observation"][7])


def _agent_config(**overrides):
    base = dict(seed=5, normalize_reward=False, n_step=3, sample_batch_size=64, buffer_max_length=100,
                buffer_min_length=32, actor_hidden_dim=16, actor_num_blocks=1, critic_hidden_dim=32,
                critic_num_blocks=1, critic_num_bins=11, critic_min_v=-5.0, critic_max_v=5.0)
    base.update(overrides)
    return FlashSACConfig(**base)


def test_agent_sampling_on_a_wrapped_nondivisible_ring(gpu):
    print("case agent sampling, 3 envs, capacity 100, n_step 3, wrapped ring", flush=True)
    from robolearn_amd.flashsac import FlashSAC

    cfg = _agent_config()
    envs, obs_dim, act_dim = 3, 5, 2
    assert cfg.buffer_max_length % envs != 0
    agent = FlashSAC(obs_dim, act_dim, num_envs=envs, cfg=cfg)
    oracle = OR.NStepReplay(obs_dim, act_dim, cfg.n_step, cfg.gamma, cfg.buffer_max_length)
    rng = np.random.default_rng(4)
    for _ in range(45):  # 43 committed steps x 3 envs = 129 rows through a 100-row ring
        step = dict(observation=rng.standard_normal((envs, obs_dim)).astype(np.float32),
                    action=rng.uniform(-1, 1, (envs, act_dim)).astype(np.float32),
                    reward=rng.standard_normal(envs).astype(np.float32),
                    terminated=(rng.random(envs) < 0.2).astype(np.float32),
                    truncated=(rng.random(envs) < 0.2).astype(np.float32),
                    next_observation=rng.standard_normal((envs, obs_dim)).astype(np.float32))
        agent.observe(*(torch.as_tensor(step[k]).to(gpu) for k in ("observation", "action", "reward", "terminated",
                                                                   "truncated", "next_observation")))
        oracle.add(**step)
    assert oracle.count == cfg.buffer_max_length and oracle.position == 29
    assert agent.replay_counters.tolist() == [45, oracle.position, oracle.count]
    for capture in (False, True, True):
        draw = int(agent.update_counters[0].item())
        agent.update(capture=capture)
        torch.cuda.synchronize()
        idx = agent.indices.cpu().numpy()
        expected_idx = PH.replay_indices(cfg.seed * 7919 + 1, draw, 1, oracle.count, cfg.sample_batch_size)
        np.testing.assert_array_equal(idx, expected_idx)
        expected = oracle.sample(expected_idx)
        for key in FIELDS:
            np.testing.assert_array_equal(agent.batch[key].cpu().numpy(), expected[key], err_msg=key)
        assert int(agent.gather_error.item()) == 0


def test_pair_graph_equals_two_eager_updates(gpu):
    print("case update-to-data-2 pair graph vs eager", flush=True)
    from robolearn_amd.flashsac import FlashSAC

    cfg = _agent_config(buffer_max_length=256, buffer_min_length=64, n_step=1)
    store = {k: v.numpy() for k, v in O.synthetic_replay(256, 6, 3, seed=2, gamma=cfg.gamma, done_prob=0.1).items()}
    pair, eager = FlashSAC(6, 3, cfg=cfg), FlashSAC(6, 3, cfg=cfg)
    for agent in (pair, eager):
        agent.load_replay(store)
    eager.load_state_dict(pair.state_dict(include_replay=False))
    for round_index in range(2):
        got = pair.update_pair()
        first = eager.update(capture=False)
        second = eager.update(capture=False)
        torch.cuda.synchronize()
        assert pair._update_step == eager._update_step == 2 * (round_index + 1)
        assert got["critic/loss"] == second["critic/loss"]
        assert got["actor/loss"] == first["actor/loss"]
        a, b = pair.state_dict(include_replay=False), eager.state_dict(include_replay=False)
        for key in a:
            np.testing.assert_array_equal(a[key], b[key], err_msg=f"{key} after pair {round_index}")
    # a later single update takes the actor phase the step gives it, on both
    third_pair = pair.update(capture=True)
    third_eager = eager.update(capture=False)
    assert third_pair.keys() == third_eager.keys() and "actor/loss" in third_pair
    a, b = pair.state_dict(include_replay=False), eager.state_dict(include_replay=False)
    for key in a:
        np.testing.assert_array_equal(a[key], b[key], err_msg=key)
