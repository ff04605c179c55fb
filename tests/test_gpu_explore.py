"""Acting: the fp32 eval-mode actor and the exploration-noise repeats on the GPU,
against the CPU oracle (oracle.explore, oracle.flashsac.actor_forward).

* With injected uniforms and fresh noise the device repeat state and held
  noise equal the oracle's exactly (same CDF, same decisions).
* With the device's own Philox draws the schedule is self-consistent (noise
  changes exactly on refresh, lengths within 1..max_n) and the draws are
  standard normal to sampling accuracy.
* act() matches the float64 oracle actor in eval mode within 1e-5: tanh(mean)
  when deterministic, tanh(mean + std * held noise) when training, in both
  precision modes (acting is fp32, as in the reference).
"""

import numpy as np
import pytest
import torch

from oracle import explore as OX
from oracle import flashsac as O
from robolearn_amd import _native
from robolearn_amd import kernels as K

pytestmark = pytest.mark.gpu


def _call(seed, step, cdf, state, noise, uniform=None, fresh=None):
    _native.call("rl_exploration_noise", seed, step.data_ptr(), cdf.data_ptr(), cdf.numel(), state.data_ptr(),
                 noise.data_ptr(), noise.numel(), uniform.data_ptr() if uniform is not None else None,
                 fresh.data_ptr() if fresh is not None else None, K.stream())


def test_exploration_repeat_matches_oracle_with_injected_draws(gpu):
    print("case exploration repeat, injected draws, mu=1.5 max_n=6", flush=True)
    cdf_host = OX.zeta_cdf(1.5, 6)
    cdf = cdf_host.to(gpu)
    state = torch.tensor([0, 1, 0], dtype=torch.int32, device=gpu)
    step = torch.zeros(1, dtype=torch.long, device=gpu)
    noise = torch.zeros(13, 3, device=gpu)
    oracle = OX.Exploration((13, 3))
    g = torch.Generator().manual_seed(4)
    for t in range(40):
        u = torch.rand(1, generator=g)
        fresh = torch.randn(13, 3, generator=g)
        _call(99, step, cdf, state, noise, uniform=u.to(gpu), fresh=fresh.to(gpu))
        refreshed = oracle.step(float(u), fresh, cdf_host)
        torch.cuda.synchronize()
        assert state.tolist() == [oracle.count, oracle.n, int(refreshed)], t
        torch.testing.assert_close(noise.cpu(), oracle.noise, rtol=0, atol=0)
    assert step.item() == 40


def test_exploration_repeat_philox_schedule(gpu):
    print("case exploration repeat, device draws, 4096 x 37", flush=True)
    max_n = 8
    cdf = OX.zeta_cdf(1.0, max_n).to(gpu)
    state = torch.tensor([0, 1, 0], dtype=torch.int32, device=gpu)
    step = torch.zeros(1, dtype=torch.long, device=gpu)
    noise = torch.zeros(4096, 37, device=gpu)
    previous, lengths, refreshes = None, [], 0
    for t in range(120):
        _call(7, step, cdf, state, noise)
        torch.cuda.synchronize()
        count, length, refresh = state.tolist()
        assert 1 <= length <= max_n and 1 <= count <= length
        current = noise.clone()
        if previous is not None:
            assert bool(refresh) == (not torch.equal(current, previous)), t
        if refresh:
            refreshes += 1
            lengths.append(length)
            assert count == 1
            assert abs(current.mean().item()) < 0.02 and abs(current.std().item() - 1.0) < 0.02
        previous = current
    assert refreshes == len(lengths) and sum(lengths[:-1]) < 120 <= sum(lengths)
    assert step.item() == 120


def _agent(use_amp, envs=6):
    from robolearn_amd.config import FlashSACConfig
    from robolearn_amd.flashsac import FlashSAC

    cfg = FlashSACConfig(seed=9, use_amp=use_amp, sample_batch_size=32, buffer_max_length=64, buffer_min_length=32,
                         actor_hidden_dim=64, actor_num_blocks=2, critic_hidden_dim=32, critic_num_blocks=1,
                         critic_num_bins=21, actor_noise_zeta_mu=0.0, actor_noise_zeta_max=3)
    return FlashSAC(7, 3, num_envs=envs, cfg=cfg)


@pytest.mark.parametrize("use_amp", [False, True])
def test_act_matches_oracle_actor(gpu, use_amp):
    print(f"case act vs oracle actor, use_amp={use_amp}", flush=True)
    agent = _agent(use_amp)
    state = agent.state_dict(include_replay=False)
    g = torch.Generator().manual_seed(2)
    for key in list(state):  # non-trivial eval-mode BN statistics
        if key.startswith("actor.") and key.endswith("running_mean"):
            state[key] = (torch.randn(state[key].shape, generator=g) * 0.3).numpy()
        elif key.startswith("actor.") and key.endswith("running_var"):
            state[key] = (torch.rand(state[key].shape, generator=g) + 0.5).numpy()
    agent.load_state_dict(state)
    oracle = O.OracleState(O.dims_from_config(7, 3, agent.cfg), agent.cfg, dtype=torch.float64)
    oracle.load_flat(agent.state_dict(include_replay=False))
    obs = torch.randn(6, 9, generator=g)  # wider than the actor's prefix: act() slices it
    _, _, mean, std = O.actor_forward(oracle.actor, oracle.actor_buffers, obs[:, :7].double(), False, None,
                                      oracle.d)
    deterministic = agent.act(obs.to(gpu), training=False).cpu().double()
    torch.testing.assert_close(deterministic, torch.tanh(mean), rtol=1e-5, atol=1e-5)
    assert agent.exploration_state.tolist() == [0, 1, 0]  # inference leaves exploration alone
    held = None
    for t in range(8):
        actions = agent.act(obs.to(gpu), training=True).cpu().double()
        count, length, refresh = agent.exploration_state.tolist()
        noise = agent.exploration_noise.cpu().double()
        if refresh:
            held = noise
        torch.testing.assert_close(noise, held, rtol=0, atol=0)
        torch.testing.assert_close(actions, torch.tanh(mean + std * held), rtol=1e-5, atol=1e-5)
    with pytest.raises(ValueError):
        agent.act(obs[:4].to(gpu), training=True)
