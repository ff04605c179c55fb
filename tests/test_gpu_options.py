"""Reference options the benchmarked configurations leave off, end to end against the float64 oracle.

One agent turns on, together:

* asymmetric critic observations: the replay holds critic_observation_dim columns, the actor reads
  their observation_dim prefix (robolearn/flashsac/agent.py:316-327, 485-487);
* the behaviour-cloning term actor_bc_alpha > 0: the actor loss gains
  bc_alpha |Q|.mean() ((a - a_batch)^2).mean() (robolearn/flashsac/updates.py:130-134);
* normalize_reward: observe() feeds the per-environment returns into the running statistics
  (agent.py:463-468) and the update divides the batch rewards by
  max(sqrt(var + 1e-8), G_r_max / normalized_G_max) (agent.py:493-495,
  _utils/reward_normalization.py:28-38);
* n_step 3 with terminations and truncations, and a replay that is not yet full (the sampler's
  range is the committed count, not the capacity).

The environment steps go through observe(); the update pair runs through update_pair (the captured
update-to-data-2 graph, device sampling and device noise).  The oracle gets the same transitions
(oracle/replay.py), the indices from the NumPy Philox restatement (checked bit for bit against the
device's), the noise regenerated on the device from the same keys (checked bit for bit against the
update's buffers) and the rewards scaled by its own running statistics.  Metrics are held to 1e-4
relative; gradients, Adam moments and parameters to the reference-relative rule of tests/parity.py
(1e-4 relative L2 against float64, or 3x the reference's own fp32 path where that errs more).
"""

import numpy as np
import pytest
import torch

from oracle import flashsac as O
from oracle import philox as PH
from oracle import replay as OR
from robolearn_amd import kernels as K
from robolearn_amd.config import FlashSACConfig

from parity import compare

pytestmark = pytest.mark.gpu

ACTOR_OBS, CRITIC_OBS, ACT, ENVS = 6, 11, 3, 8


def _device_normal(gpu, shape, seed, draw, stream_id):
    out = torch.empty(shape, device=gpu)
    K.philox_normal(out, seed=seed, counter=torch.tensor([draw], dtype=torch.long, device=gpu), stream_id=stream_id)
    return out


def _store_from(replay):
    return {k: torch.as_tensor(v.copy()) for k, v in replay.storage.items()}


def test_asymmetric_bc_normalized_reward_pair_graph_matches_oracle(gpu):
    print("case options: asymmetric observations, actor_bc_alpha 0.4, normalize_reward, n_step 3, "
          "update_pair vs float64 oracle", flush=True)
    from robolearn_amd.flashsac import FlashSAC

    torch.set_num_threads(8)
    cfg = FlashSACConfig(seed=9, normalize_reward=True, normalized_G_max=5.0, n_step=3, sample_batch_size=64,
                         buffer_max_length=300, buffer_min_length=64, actor_hidden_dim=32, actor_num_blocks=1,
                         critic_hidden_dim=64, critic_num_blocks=2, critic_num_bins=31, critic_min_v=-6.0,
                         critic_max_v=6.0, actor_bc_alpha=0.4, learning_rate_init=3e-4, learning_rate_peak=3e-4,
                         learning_rate_end=3e-4, use_amp=False, actor_update_period=2)
    agent = FlashSAC(ACTOR_OBS, ACT, num_envs=ENVS, cfg=cfg, critic_observation_dim=CRITIC_OBS)
    assert agent.cfg.asymmetric_observation
    replay = OR.NStepReplay(CRITIC_OBS, ACT, cfg.n_step, cfg.gamma, cfg.buffer_max_length)
    stats = OR.RewardStats(ENVS, cfg.gamma)
    rng = np.random.default_rng(11)
    for _ in range(22):  # 20 committed steps x 8 envs = 160 of 300 rows
        step = dict(observation=rng.standard_normal((ENVS, CRITIC_OBS)).astype(np.float32),
                    action=rng.uniform(-1, 1, (ENVS, ACT)).astype(np.float32),
                    reward=(2.0 * rng.standard_normal(ENVS) + 0.5).astype(np.float32),
                    terminated=(rng.random(ENVS) < 0.1).astype(np.float32),
                    truncated=(rng.random(ENVS) < 0.05).astype(np.float32),
                    next_observation=rng.standard_normal((ENVS, CRITIC_OBS)).astype(np.float32))
        agent.observe(*(torch.as_tensor(step[k]).to(gpu) for k in ("observation", "action", "reward", "terminated",
                                                                   "truncated", "next_observation")))
        replay.add(**step)
        stats.update(step["reward"], step["terminated"], step["truncated"])
    torch.cuda.synchronize()
    count = replay.count
    assert count == 160 < cfg.buffer_max_length and agent.ready
    assert agent.replay_counters.tolist() == [22, replay.position, count]
    np.testing.assert_array_equal(agent.reward_max.cpu().numpy(), stats.maximum)
    np.testing.assert_allclose(agent.reward_running.cpu().numpy(), stats.running, rtol=1e-5)

    state = O.OracleState(O.dims_from_config(ACTOR_OBS, ACT, agent.cfg, CRITIC_OBS), agent.cfg,
                          dtype=torch.float64)
    state.load_flat(agent.state_dict(include_replay=False))
    before = state.flat()
    draw = int(agent.update_counters[0].item())
    metrics = agent.update_pair(tensor_metrics=False)
    torch.cuda.synchronize()
    B, seed = cfg.sample_batch_size, cfg.seed
    idx = [PH.replay_indices(seed * 7919 + 1, draw + u, 1, count, B) for u in range(2)]
    assert all(i.max() < count for i in idx)
    np.testing.assert_array_equal(agent.indices.cpu().numpy(), idx[1])
    assert int(agent.gather_error.item()) == 0
    actor_noise = _device_normal(gpu, (2 * B, ACT), seed * 7919 + 11, draw, 11)
    next_noise = [_device_normal(gpu, (B, ACT), seed * 7919 + 23, draw + u, 23) for u in range(2)]
    torch.cuda.synchronize()
    assert torch.equal(actor_noise, agent.actor_noise)
    assert torch.equal(next_noise[1], agent.next_noise)

    # the rewards the update saw: the second update's batch, scaled on the device, against the oracle's scale
    store = _store_from(replay)
    batches = []
    for u in range(2):
        batch = O.sample(store, idx[u])
        batch["reward"] = torch.as_tensor(stats.scale(batch["reward"].numpy(), cfg.normalized_G_max))
        batches.append(batch)
    np.testing.assert_allclose(agent.reward_used.cpu().numpy(), batches[1]["reward"].numpy(), rtol=2e-6)
    assert not np.allclose(batches[1]["reward"].numpy(), O.sample(store, idx[1])["reward"].numpy())

    inputs = [(batches[0], actor_noise.cpu(), next_noise[0].cpu(), True),
              (batches[1], actor_noise.cpu(), next_noise[1].cpu(), False)]
    records = [{}, {}]
    info = [O.update(state, b, an, nn, do_actor_update=actor, record=r)
            for (b, an, nn, actor), r in zip(inputs, records)]
    expected = {k: float(v) for k, v in info[0].items() if not k.startswith("critic/")}
    expected.update({k: float(v) for k, v in info[1].items()})
    assert set(metrics) == set(expected)
    for key, value in expected.items():
        assert metrics[key] == pytest.approx(value, rel=1e-4, abs=1e-6), (key, metrics[key], value)

    fp32 = O.OracleState(state.d, agent.cfg, dtype=torch.float32)
    fp32.load_flat(before)
    fp32_records = [{}, {}]
    for (b, an, nn, actor), r in zip(inputs, fp32_records):
        O.update(fp32, b, an, nn, do_actor_update=actor, record=r)
    report = []
    compare("actor grad (update 1)", {k: v.cpu() for k, v in agent.actor.grads().items()},
            fp32_records[0]["actor_grads"], records[0]["actor_grads"], report)
    compare("critic grad (update 2)", {k: v.cpu() for k, v in agent.critic.grads().items()},
            fp32_records[1]["critic_grads"], records[1]["critic_grads"], report)
    after, gpu_state = state.flat(), agent.state_dict(include_replay=False)
    params = {k: v for k, v in after.items() if "running" not in k}
    compare("parameters", gpu_state, fp32.flat(), params, report)
    for key in (k for k in after if "running" in k):
        err = (torch.as_tensor(gpu_state[key]).double() - after[key]).abs().max().item()
        assert err <= 1e-4 * after[key].abs().max().item() + 1e-7, (key, err)
    report.sort(key=lambda r: -r[4])
    for label, name, gpu_max, cpu_max, gpu_l2, cpu_l2 in report[:6]:
        print(f"  {label:22s} {name:40s} rel L2 GPU {gpu_l2:.2e} fp32 Torch {cpu_l2:.2e}", flush=True)
