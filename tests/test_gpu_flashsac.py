"""FlashSAC learner on the GPU against the CPU oracle on identical inputs.

Inputs (initial weights, replay batch, reparameterization noise) are injected
into both sides.  The oracle runs in float64; the HIP fp32 path must match
losses, gradients and Adam moments to 1e-4 relative (tensor max-norm), and
post-update parameter deltas by the reference's delta policy
(examples/diagnose_warp_flashsac.py:114-129: atol 5e-7, rtol 0.02 of the
tensor's largest delta).  The bf16-operand mode must match losses to 1e-2.
"""

from dataclasses import replace

import numpy as np
import pytest
import torch

from oracle import flashsac as O
from robolearn_amd.config import FlashSACConfig

pytestmark = pytest.mark.gpu

OBS, ACT = 6, 3


def _config(**overrides):
    base = dict(seed=3, normalize_reward=False, n_step=1, sample_batch_size=32, buffer_max_length=256,
                buffer_min_length=32, actor_hidden_dim=16, actor_num_blocks=1, critic_hidden_dim=32,
                critic_num_blocks=2, critic_num_bins=21, critic_min_v=-10.0, critic_max_v=10.0,
                critic_target_update_tau=0.005, learning_rate_init=3e-4, learning_rate_peak=3e-4,
                learning_rate_end=1.5e-4, learning_rate_decay_step=50)
    base.update(overrides)
    return FlashSACConfig(**base)


def _tensor_rel(actual, expected):
    actual = torch.as_tensor(actual).double().cpu()
    expected = torch.as_tensor(expected).double().cpu()
    scale = expected.abs().max().item()
    return (actual - expected).abs().max().item() / max(scale, 1e-30)


def _make(cfg):
    from robolearn_amd.flashsac import FlashSAC

    agent = FlashSAC(OBS, ACT, cfg=cfg)
    state = O.OracleState(O.dims_from_config(OBS, ACT, agent.cfg), agent.cfg, dtype=torch.float64)
    state.load_flat({k: v for k, v in agent.state_dict(include_replay=False).items()})
    return agent, state


def _inputs(cfg, step, rows=None):
    rows = rows or cfg.sample_batch_size
    g = torch.Generator().manual_seed(100 + step)
    store = O.synthetic_replay(256, OBS, ACT, seed=7, gamma=cfg.gamma, done_prob=0.1)
    idx = torch.randint(0, 256, (rows,), generator=g)
    batch = O.sample(store, idx)
    actor_noise = torch.randn(2 * rows, ACT, generator=g)
    next_noise = torch.randn(rows, ACT, generator=g)
    return batch, actor_noise, next_noise


def test_gradients_match_oracle(gpu):
    """Actor-phase and critic-phase gradients, each from the same initial state."""
    cfg = _config()
    batch, an, nn = _inputs(cfg, 0)
    host_batch = {k: v.numpy() for k, v in batch.items()}
    # actor phase: actor gradients and temperature gradient (BN batch statistics; frozen eval critic)
    agent, state = _make(cfg)
    metrics = agent.update_from_batch(host_batch, actor_noise=an.numpy(), next_noise=nn.numpy(),
                                      do_actor_update=True, apply_optimizer=False, tensor_metrics=False)
    record = {}
    info = O.update(state, batch, an, nn, do_actor_update=True, record=record)
    torch.cuda.synchronize()
    for key in ("actor/loss", "actor/entropy", "actor/mean_action", "temperature/loss", "temperature/value"):
        assert metrics[key] == pytest.approx(float(info[key]), rel=1e-4, abs=1e-6), key
    for name, grad in agent.actor.grads().items():
        assert _tensor_rel(grad, record["actor_grads"][name]) < 1e-4, f"actor grad {name}"
    assert _tensor_rel(agent.temperature.grad[:1], record["temperature_grad"]) < 1e-4
    # critic phase alone
    agent, state = _make(cfg)
    metrics = agent.update_from_batch(host_batch, actor_noise=an.numpy(), next_noise=nn.numpy(),
                                      do_actor_update=False, apply_optimizer=False, tensor_metrics=False)
    record = {}
    info = O.update(state, batch, an, nn, do_actor_update=False, record=record)
    torch.cuda.synchronize()
    for key in ("critic/loss", "critic/max_entropy_bonus"):
        assert metrics[key] == pytest.approx(float(info[key]), rel=1e-4, abs=1e-6), key
    assert _tensor_rel(agent.target_probabilities, record["target_probs"]) < 1e-5
    for name, grad in agent.critic.grads().items():
        assert _tensor_rel(grad, record["critic_grads"][name]) < 1e-4, f"critic grad {name}"


@pytest.mark.parametrize("steps", [3])
def test_full_updates_match_oracle(gpu, steps):
    cfg = _config()
    agent, state = _make(cfg)
    for step in range(steps):
        batch, an, nn = _inputs(cfg, step)
        metrics = agent.update_from_batch({k: v.numpy() for k, v in batch.items()}, actor_noise=an.numpy(),
                                          next_noise=nn.numpy(), tensor_metrics=False)
        before = state.flat()
        info = O.update(state, batch, an, nn)
        for key, value in info.items():
            assert metrics[key] == pytest.approx(float(value), rel=1e-4, abs=1e-6), (step, key)
        gpu_state = agent.state_dict(include_replay=False)
        after = state.flat()
        flips = 0
        for key, expected in after.items():
            actual = torch.as_tensor(gpu_state[key]).double()
            if "running" in key:
                # batch means of zero-mean BN outputs are O(1e-19) in float64 and O(1e-10)
                # in fp32, so the running statistics get an absolute floor
                err = (actual - expected).abs().max().item()
                assert err <= 1e-4 * expected.abs().max().item() + 1e-7, (step, key, err)
                continue
            delta_ref = expected - before[key]
            delta_gpu = actual - before[key]
            bound = 5e-7 + 0.02 * delta_ref.abs().max().item()
            err = (delta_gpu - delta_ref).abs()
            flips += int((err > bound).sum())
            assert err.max().item() <= bound, (step, key, err.max().item(), bound)
        moments = state.moments()
        for label, store in (("actor", agent.actor), ("critic", agent.critic)):
            m1, m2 = store.moments()
            for name in store.shapes:
                assert _tensor_rel(m1[name], moments[f"{label}.{name}.m1"]) < 1e-4, (step, label, name, "m1")
                assert _tensor_rel(m2[name], moments[f"{label}.{name}.m2"]) < 1e-4, (step, label, name, "m2")
        print(f"step {step}: parameter elements beyond the delta policy: {flips}")


def test_bf16_mode_losses_within_1e2(gpu):
    cfg = _config(use_amp=True)
    agent, state = _make(cfg)
    for step in range(2):
        batch, an, nn = _inputs(cfg, step)
        metrics = agent.update_from_batch({k: v.numpy() for k, v in batch.items()}, actor_noise=an.numpy(),
                                          next_noise=nn.numpy(), tensor_metrics=False)
        info = O.update(state, batch, an, nn)
        for key, value in info.items():
            assert metrics[key] == pytest.approx(float(value), rel=1e-2, abs=1e-3), (step, key)


def test_captured_graph_matches_eager(gpu):
    cfg = _config(buffer_min_length=64)
    store = O.synthetic_replay(256, OBS, ACT, seed=7, gamma=cfg.gamma, done_prob=0.1)
    from robolearn_amd.flashsac import FlashSAC

    eager = FlashSAC(OBS, ACT, cfg=cfg)
    graph = FlashSAC(OBS, ACT, cfg=cfg)
    for agent in (eager, graph):
        agent.load_replay({k: v.numpy() for k, v in store.items()})
    graph.load_state_dict(eager.state_dict(include_replay=False))
    for _ in range(4):
        a = eager.update(capture=False)
        b = graph.update(capture=True)
        assert a.keys() == b.keys()
    torch.cuda.synchronize()
    s1, s2 = eager.state_dict(include_replay=False), graph.state_dict(include_replay=False)
    for key in s1:
        np.testing.assert_array_equal(s1[key], s2[key], err_msg=key)


def test_checkpoint_roundtrip_preserves_graph(gpu, tmp_path):
    cfg = _config(buffer_min_length=64)
    store = O.synthetic_replay(256, OBS, ACT, seed=7, gamma=cfg.gamma)
    from robolearn_amd.flashsac import FlashSAC

    agent = FlashSAC(OBS, ACT, cfg=cfg)
    agent.load_replay({k: v.numpy() for k, v in store.items()})
    agent.update()
    agent.save(tmp_path / "ckpt")
    saved = agent.state_dict(include_replay=False)
    agent.update()
    agent.update()
    agent.load(tmp_path / "ckpt")
    restored = agent.state_dict(include_replay=False)
    for key in saved:
        np.testing.assert_array_equal(saved[key], restored[key], err_msg=key)
    agent.update()  # the captured graph still points at the restored buffers
    torch.cuda.synchronize()


def test_constructor_target_entropy_is_the_normal_entropy(gpu):
    """cfg.temp_target_entropy of a constructed learner is A times the entropy of Normal(0, sigma)
    (robolearn/flashsac/agent.py:329), for the configured temp_target_sigma."""
    from robolearn_amd.flashsac import FlashSAC

    for sigma in (0.15, 0.4):
        agent = FlashSAC(OBS, ACT, cfg=_config(temp_target_sigma=sigma))
        normal = ACT * torch.distributions.Normal(torch.tensor(0.0, dtype=torch.float64),
                                                  torch.tensor(sigma, dtype=torch.float64)).entropy().item()
        assert agent.cfg.temp_target_entropy == pytest.approx(normal, rel=1e-12)


@pytest.mark.parametrize("bins", [1024, 4096])
def test_wide_categorical_heads_match_oracle(gpu, bins):
    """Critics with more bins than the register-row kernels hold take the one-workgroup-per-row
    categorical kernels (head forward, Q backward, TD target + cross-entropy): an actor-phase update and
    a critic-only update against the float64 oracle with the device's ReLU decisions, 1e-4."""
    from parity import forced_update_check

    print(f"case flashsac with {bins}-bin critics vs float64 oracle (forced ReLU decisions)", flush=True)
    cfg = _config(critic_num_bins=bins)
    agent, _ = _make(cfg)
    for step, actor_phase in enumerate((True, False)):
        batch, an, nn = _inputs(cfg, step)
        forced_update_check(agent, batch, an, nn, bound=1e-4, label=f"{bins} bins update {step + 1}",
                            actor_phase=actor_phase)
