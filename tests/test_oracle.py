"""Pins the CPU oracle: reference golden vectors, reference known answers,
closed forms and brute force.  CPU only."""

import math
from collections import OrderedDict
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import flashsac as O
from oracle import ppo as OP
from robolearn_amd.config import FlashSACConfig, PPOConfig

GOLDEN = np.load(Path(__file__).resolve().parent / "golden" / "flashsac_modules.npz", allow_pickle=False)


def _group(prefix):
    return OrderedDict((k[len(prefix):], torch.tensor(GOLDEN[k])) for k in GOLDEN.files if k.startswith(prefix))


def _dims():
    return O.Dims(actor_obs=4, critic_obs=4, action=2, actor_hidden=16, actor_blocks=1, critic_hidden=16,
                  critic_blocks=2, bins=11, min_v=-10.0, max_v=10.0)


def _split(state, shapes):
    params = OrderedDict((k, state[k].clone().requires_grad_(True)) for k in shapes)
    buffers = OrderedDict((k, v.clone()) for k, v in state.items() if k not in shapes)
    return params, buffers


def test_actor_forward_backward_matches_reference_modules():
    d = _dims()
    params, buffers = _split(_group("actor.init."), O.actor_parameter_shapes(d))
    x, noise = torch.tensor(GOLDEN["actor.train.x"]), torch.tensor(GOLDEN["actor.train.noise"])
    actions, log_prob, _, _ = O.actor_forward(params, buffers, x, True, noise, d)
    torch.testing.assert_close(actions, torch.tensor(GOLDEN["actor.train.actions"]), rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(log_prob, torch.tensor(GOLDEN["actor.train.log_prob"]), rtol=1e-5, atol=1e-5)
    coef = torch.tensor(GOLDEN["actor.train.coef"])
    loss = (0.3 * log_prob).mean() + (coef * actions).mean()
    grads = torch.autograd.grad(loss, list(params.values()))
    for (name, _), grad in zip(params.items(), grads):
        torch.testing.assert_close(grad, torch.tensor(GOLDEN[f"actor.grad.{name}"]), rtol=1e-4, atol=1e-6,
                                   msg=name)
    for name, value in buffers.items():
        torch.testing.assert_close(value, torch.tensor(GOLDEN[f"actor.after.{name}"]), rtol=1e-6, atol=1e-7,
                                   msg=name)
    xe, ne = torch.tensor(GOLDEN["actor.eval.x"]), torch.tensor(GOLDEN["actor.eval.noise"])
    with torch.no_grad():
        a, lp, mean, std = O.actor_forward(params, buffers, xe, False, ne, d)
    torch.testing.assert_close(a, torch.tensor(GOLDEN["actor.eval.actions"]), rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(lp, torch.tensor(GOLDEN["actor.eval.log_prob"]), rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(mean, torch.tensor(GOLDEN["actor.eval.mean"]), rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(std, torch.tensor(GOLDEN["actor.eval.std"]), rtol=1e-6, atol=1e-7)


def test_critic_forward_backward_matches_reference_modules():
    d = _dims()
    state = _group("critic.init.")
    state.pop("predictor.bin_values")
    params, buffers = _split(state, O.critic_parameter_shapes(d))
    obs, act = torch.tensor(GOLDEN["critic.train.obs"]), torch.tensor(GOLDEN["critic.train.act"])
    q, lp = O.critic_forward(params, buffers, obs, act, True, d)
    torch.testing.assert_close(q, torch.tensor(GOLDEN["critic.train.q"]), rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(lp, torch.tensor(GOLDEN["critic.train.log_prob"]), rtol=1e-5, atol=1e-6)
    loss = (torch.tensor(GOLDEN["critic.train.cq"]) * q).sum() + (torch.tensor(GOLDEN["critic.train.clp"]) * lp).sum() * 0.05
    grads = torch.autograd.grad(loss, list(params.values()))
    for (name, _), grad in zip(params.items(), grads):
        torch.testing.assert_close(grad, torch.tensor(GOLDEN[f"critic.grad.{name}"]), rtol=1e-4, atol=1e-5,
                                   msg=name)
    for name, value in buffers.items():
        torch.testing.assert_close(value, torch.tensor(GOLDEN[f"critic.after.{name}"]), rtol=1e-6, atol=1e-7,
                                   msg=name)
    with torch.no_grad():
        q2, lp2 = O.critic_forward(params, buffers, obs, act, False, d)
    torch.testing.assert_close(q2, torch.tensor(GOLDEN["critic.eval.q"]), rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(lp2, torch.tensor(GOLDEN["critic.eval.log_prob"]), rtol=1e-5, atol=1e-6)


def test_projection_and_ema_match_reference_network():
    before = _group("project.before.")
    O.normalize_parameters(before)
    for name, value in before.items():
        torch.testing.assert_close(value, torch.tensor(GOLDEN[f"project.after.{name}"]), rtol=1e-6, atol=1e-7,
                                   msg=name)
    target = _group("ema.before.")
    source = _group("project.after.")
    O.ema_update(target, source, 0.005)
    for name, value in target.items():
        torch.testing.assert_close(value, torch.tensor(GOLDEN[f"ema.after.{name}"]), rtol=0, atol=0, msg=name)


def test_projection_invariants():
    g = torch.Generator().manual_seed(0)
    params = OrderedDict(
        (k, torch.randn(v, generator=g)) for k, v in O.critic_parameter_shapes(_dims()).items())
    O.normalize_parameters(params)
    w = params["encoder.0.w1.weight"]
    torch.testing.assert_close(w.norm(dim=-1), torch.ones(w.shape[:-1]), rtol=1e-6, atol=1e-6)
    bn_w, bn_b = params["encoder.0.norm1.weight"], params["encoder.0.norm1.bias"]
    torch.testing.assert_close((bn_w ** 2 + bn_b ** 2).sum(-1), torch.full((2,), float(bn_w.shape[-1])), rtol=1e-5,
                               atol=1e-5)
    rms = params["post_norm.weight"]
    torch.testing.assert_close((rms ** 2).sum(-1), torch.full((2,), float(rms.shape[-1])), rtol=1e-5, atol=1e-5)


def test_schedule_matches_reference_and_closed_form():
    steps = GOLDEN["schedule.steps"]
    for label in ("a", "b"):
        f = O.warmup_cosine(*GOLDEN[f"schedule.{label}.args"])
        np.testing.assert_allclose([f(int(s)) for s in steps], GOLDEN[f"schedule.{label}.values"], rtol=0, atol=0)
    f = O.warmup_cosine(1e-5, 3e-4, 1e-4, 10, 110)
    assert f(5) == pytest.approx(1e-5 + (3e-4 - 1e-5) * 0.5)
    assert f(60) == pytest.approx(1e-4 + (3e-4 - 1e-4) * 0.5)  # cosine midpoint
    assert f(200) == 1e-4


def test_log_det_and_temperature_match_reference():
    x = torch.tensor(GOLDEN["logdet.x"])
    torch.testing.assert_close(O.safe_tanh_log_det_jacobian(x), torch.tensor(GOLDEN["logdet.y"]), rtol=0, atol=0)
    # closed form log(1 - tanh(x)^2) away from saturation
    xs = torch.linspace(-3, 3, 13, dtype=torch.float64)
    torch.testing.assert_close(O.safe_tanh_log_det_jacobian(xs), torch.log(1 - torch.tanh(xs) ** 2))
    assert float(GOLDEN["temperature.value"][0]) == pytest.approx(math.exp(math.log(0.01)), rel=1e-7)


# ---------------------------------------------------------------------------
# categorical TD projection: closed forms
# ---------------------------------------------------------------------------
def _td(reward, done, entropy, gamma, lp, bins=11, min_v=-10.0, max_v=10.0):
    return O.categorical_td_target(lp, reward, done, entropy, gamma, bins, min_v, max_v)


def test_td_target_mass_and_grid_points():
    g = torch.Generator().manual_seed(1)
    rows, bins = 64, 11
    lp = torch.log_softmax(torch.randn(rows, bins, generator=g, dtype=torch.float64), -1)
    reward = torch.randn(rows, generator=g, dtype=torch.float64) * 5
    done = (torch.rand(rows, generator=g) < 0.3).double()
    entropy = torch.randn(rows, generator=g, dtype=torch.float64) * 0.1
    t = _td(reward, done, entropy, torch.full((rows,), 0.99, dtype=torch.float64), lp)
    torch.testing.assert_close(t.sum(-1), torch.ones(rows, dtype=torch.float64))
    assert (t >= 0).all()
    # terminal rows collapse all mass onto the reward (two-hot of one value)
    expected_mean = torch.clamp(reward, -10, 10)
    support = torch.linspace(-10, 10, bins, dtype=torch.float64)
    term = done == 1
    torch.testing.assert_close((t[term] * support).sum(-1), expected_mean[term])
    # values exactly on the grid: reward on a bin center, gamma 0 -> one-hot
    reward = torch.tensor([-10.0, -6.0, 0.0, 4.0, 10.0], dtype=torch.float64)
    t = _td(reward, torch.zeros(5, dtype=torch.float64), torch.zeros(5, dtype=torch.float64),
            torch.zeros(5, dtype=torch.float64), lp[:5])
    for row, r in enumerate(reward):
        k = int(round((float(r) + 10) / 2))
        assert t[row, k] == pytest.approx(1.0)
    # everything beyond max_v lands in the last bin
    t = _td(torch.full((3,), 50.0, dtype=torch.float64), torch.zeros(3, dtype=torch.float64),
            torch.zeros(3, dtype=torch.float64), torch.full((3,), 0.99, dtype=torch.float64), lp[:3])
    torch.testing.assert_close(t[:, -1], torch.ones(3, dtype=torch.float64))


def test_td_target_brute_force():
    """Direct per-atom two-hot accumulation on tiny inputs."""
    g = torch.Generator().manual_seed(2)
    rows, bins = 7, 5
    lp = torch.log_softmax(torch.randn(rows, bins, generator=g, dtype=torch.float64), -1)
    reward = torch.randn(rows, generator=g, dtype=torch.float64) * 3
    done = torch.tensor([0, 1, 0, 0, 1, 0, 0], dtype=torch.float64)
    entropy = torch.randn(rows, generator=g, dtype=torch.float64) * 0.2
    gamma = torch.full((rows,), 0.9, dtype=torch.float64)
    t = _td(reward, done, entropy, gamma, lp, bins=bins, min_v=-4.0, max_v=4.0)
    support = np.linspace(-4, 4, bins)
    for i in range(rows):
        expected = np.zeros(bins)
        for j in range(bins):
            v = reward[i].item() + gamma[i].item() * (support[j] - entropy[i].item()) * (1 - done[i].item())
            v = min(max(v, -4.0), 4.0)
            b = (v + 4.0) / 2.0
            lo = int(math.floor(b))
            hi = min(lo + 1, bins - 1)
            p = math.exp(lp[i, j].item())
            expected[lo] += p * (1 - (b - lo))
            expected[hi] += p * (b - lo)
        np.testing.assert_allclose(t[i].numpy(), expected, atol=1e-12)


def test_select_min_q_prefers_first_critic_on_ties():
    q = torch.tensor([[1.0, 2.0, 3.0], [1.0, 1.0, 4.0]])
    lp = torch.stack([torch.zeros(3, 4), torch.ones(3, 4)])
    out = O.select_min_q_log_probs(q, lp)
    assert out[0].eq(0).all() and out[1].eq(1).all() and out[2].eq(0).all()


# ---------------------------------------------------------------------------
# composite update: finite differences on a tiny network (float64)
# ---------------------------------------------------------------------------
def _tiny_config():
    cfg = FlashSACConfig(seed=0, normalize_reward=False, n_step=1, sample_batch_size=6, buffer_max_length=32,
                         buffer_min_length=6, actor_hidden_dim=4, actor_num_blocks=1, critic_hidden_dim=4,
                         critic_num_blocks=1, critic_num_bins=5, critic_min_v=-4.0, critic_max_v=4.0)
    from dataclasses import replace

    return replace(cfg, temp_target_entropy=O.target_entropy(2, cfg.temp_target_sigma))


def test_actor_and_critic_loss_gradients_match_finite_differences():
    cfg = _tiny_config()
    d = O.dims_from_config(3, 2, cfg)
    state = O.init_state(d, cfg, seed=4, dtype=torch.float64)
    store = O.synthetic_replay(32, 3, 2, seed=1, gamma=0.99, done_prob=0.2)
    batch = {k: v.double() for k, v in O.sample(store, torch.arange(6)).items()}
    g = torch.Generator().manual_seed(3)
    noise = torch.randn(12, 2, generator=g, dtype=torch.float64)

    def actor_loss():
        actions, log_probs, _, _ = O.actor_forward(state.actor, OrderedDict((k, v.clone()) for k, v in state.actor_buffers.items()),
                                                   torch.cat([batch["observation"], batch["next_observation"]]), True,
                                                   noise, d)
        qs, _ = O.critic_forward(state.critic, state.critic_buffers, batch["observation"], actions[:6], False, d)
        return (log_probs[:6] * 0.01 - torch.minimum(qs[0], qs[1])).mean()

    for name in ("embedder.w.w.weight", "encoder.0.norm1.bias", "predictor.std_w.w.weight", "predictor.mean_bias"):
        param = state.actor[name]
        (grad,) = torch.autograd.grad(actor_loss(), [param])
        flat = param.detach().view(-1)
        for index in (0, flat.numel() // 2, flat.numel() - 1):
            saved = flat[index].item()
            with torch.no_grad():
                flat[index] = saved + 1e-6
                plus = actor_loss().item()
                flat[index] = saved - 1e-6
                minus = actor_loss().item()
                flat[index] = saved
            assert grad.view(-1)[index].item() == pytest.approx((plus - minus) / 2e-6, rel=1e-4, abs=1e-8), name


# ---------------------------------------------------------------------------
# PPO: reference known answers (tests/test_warp_ppo.py)
# ---------------------------------------------------------------------------
def test_ppo_gae_known_answer():
    reward = np.array([[1, 2], [3, 4], [5, 6]], dtype=np.float32)
    value = np.array([[0.1, 0.2], [0.3, 0.4], [0.5, 0.6]], dtype=np.float32)
    next_value = np.array([[0.3, 0.4], [9, 10], [11, 12]], dtype=np.float32)
    terminated = np.array([[0, 0], [1, 0], [0, 0]], dtype=np.int32)
    truncated = np.array([[0, 0], [0, 1], [0, 0]], dtype=np.int32)
    adv, ret = OP.gae(reward.flatten(), value.flatten(), next_value.flatten(), terminated.flatten(),
                      truncated.flatten(), 3, 2, 0.99, 0.95)
    expected = np.zeros_like(reward)
    tail = np.zeros(2, dtype=np.float32)
    for t in range(2, -1, -1):
        delta = reward[t] + 0.99 * (1 - terminated[t]) * next_value[t] - value[t]
        tail = delta + 0.99 * 0.95 * (1 - np.maximum(terminated[t], truncated[t])) * tail
        expected[t] = tail
    np.testing.assert_allclose(adv.numpy().reshape(3, 2), expected, rtol=1e-6)
    np.testing.assert_allclose(ret.numpy().reshape(3, 2), expected + value, rtol=1e-6)


def test_ppo_timeout_current_bootstrap_uses_own_value():
    adv, _ = OP.gae([1.0], [0.5], [9.0], [0], [1], 1, 1, 0.9, 0.95, "current")
    assert adv[0].item() == pytest.approx(1.0 + 0.9 * 0.5 - 0.5)


def test_ppo_advantage_normalization_at_large_offset():
    adv, ret = OP.gae(np.array([10000.0, 10001.0]), np.zeros(2), np.zeros(2), np.zeros(2), np.zeros(2), 1, 2,
                      0.0, 0.95)
    np.testing.assert_allclose(OP.normalize(adv.float(), False).numpy(), [-1.0, 1.0], rtol=1e-6)


def test_ppo_loss_and_gradients_match_reference_known_answer():
    mean = torch.tensor([[0.4, 0.1], [-0.3, 0.2], [0.2, -0.2]], dtype=torch.float64, requires_grad=True)
    action = torch.tensor([[0.0, 0.5], [0.6, 0.1], [-0.5, 0.4]], dtype=torch.float64)
    old_lp = torch.tensor([-2.4, -1.8, -2.0], dtype=torch.float64)
    advantage = torch.tensor([1.0, -0.8, 0.4], dtype=torch.float64)
    value = torch.tensor([[0.8], [1.0], [-0.5]], dtype=torch.float64, requires_grad=True)
    old_value = torch.tensor([0.2, 1.3, -0.4], dtype=torch.float64)
    returns = torch.tensor([0.7, -0.2, 1.0], dtype=torch.float64)
    log_std = torch.tensor([-0.2, 0.1], dtype=torch.float64, requires_grad=True)
    cfg = PPOConfig(clip_ratio=0.2, value_coefficient=0.5, entropy_coefficient=0.01, value_loss_scale=0.5)
    loss, *_ = OP.loss_terms(mean, value, log_std, action, old_lp, old_value, advantage, returns, cfg)

    def reference(m=mean.detach().numpy(), v=value.detach().numpy(), s=log_std.detach().numpy()):
        a = action.numpy()
        lp = (-0.5 * (((a - m) * np.exp(-s)) ** 2 + 2 * s + np.log(2 * np.pi))).sum(1)
        ratio = np.exp(lp - old_lp.numpy())
        policy = -np.minimum(ratio * advantage.numpy(), np.clip(ratio, 0.8, 1.2) * advantage.numpy()).mean()
        clipped = old_value.numpy() + np.clip(v[:, 0] - old_value.numpy(), -0.2, 0.2)
        vl = 0.5 * np.maximum((v[:, 0] - returns.numpy()) ** 2, (clipped - returns.numpy()) ** 2).mean()
        return policy + 0.5 * vl - 0.01 * (s + 0.5 * np.log(2 * np.pi * np.e)).sum()

    assert loss.item() == pytest.approx(reference(), rel=1e-10)
    grads = torch.autograd.grad(loss, [mean, value, log_std])
    for key, data, grad in (("m", mean, grads[0]), ("v", value, grads[1]), ("s", log_std, grads[2])):
        base = data.detach().numpy()
        numerical = np.zeros_like(base)
        for index in np.ndindex(base.shape):
            plus, minus = base.copy(), base.copy()
            plus[index] += 1e-6
            minus[index] -= 1e-6
            numerical[index] = (reference(**{key: plus}) - reference(**{key: minus})) / 2e-6
        np.testing.assert_allclose(grad.numpy(), numerical, atol=1e-7, rtol=1e-6)


@pytest.mark.parametrize("scale", [1e-3, 0.5, 3.0, 40.0])
def test_ppo_gradient_clipping_closed_form(scale):
    """clip_gradients (robolearn/warp/ppo.py:241-252, 676-693): unchanged below the threshold; above it
    g * max_norm / (||g|| + 1e-6), so the post-clip norm is max_norm ||g|| / (||g|| + 1e-6).  Checked for
    one group and for the combined group of several tensors (the c3 default)."""
    g = torch.Generator().manual_seed(int(scale * 1000))
    max_norm = 1.0
    shapes = [(7, 3), (3,), (5, 7), (1,)]
    params = [torch.nn.Parameter(torch.randn(s, generator=g, dtype=torch.float64)) for s in shapes]
    grads = [torch.randn(s, generator=g, dtype=torch.float64) for s in shapes]
    total = math.sqrt(sum(float((x * x).sum()) for x in grads))
    grads = [x * (scale / total) for x in grads]
    norm = math.sqrt(sum(float((x * x).sum()) for x in grads))
    for p, x in zip(params, grads):
        p.grad = x.clone()
    returned = OP.clip_gradients(params, max_norm)
    assert returned == pytest.approx(norm, rel=1e-12)
    after = math.sqrt(sum(float((p.grad * p.grad).sum()) for p in params))
    if norm + 1e-6 <= max_norm:
        for p, x in zip(params, grads):
            assert torch.equal(p.grad, x)
    else:
        assert after == pytest.approx(max_norm * norm / (norm + 1e-6), rel=1e-12)
        coefficient = max_norm / (norm + 1e-6)
        for p, x in zip(params, grads):
            torch.testing.assert_close(p.grad, x * coefficient, rtol=1e-14, atol=0)


def test_ppo_step_from_injected_state_continues_the_update():
    """set_state + minibatch_step (the per-step check of the GPU update) continue a run exactly: an
    update of 2 epochs x 2 minibatches equals its first three steps followed by the fourth step run
    from the parameters, moments, step count and learning rate copied into a fresh oracle."""
    cfg = PPOConfig(hidden_dims=(16, 8), epochs=2, num_mini_batches=2, schedule="adaptive", desired_kl=0.01)
    envs, horizon, obs_dim, act_dim = 8, 4, 5, 3
    n = envs * horizon
    rng = np.random.default_rng(4)
    rollout = dict(observations=rng.standard_normal((n, obs_dim)), actions=rng.standard_normal((n, act_dim)),
                   means=rng.standard_normal((n, act_dim)) * 0.1, stds=np.full((n, act_dim), 1.1),
                   values=rng.standard_normal(n), log_probs=rng.standard_normal(n) - 4.0,
                   rewards=rng.standard_normal(n), next_values=rng.standard_normal(n),
                   terminated=(rng.random(n) < 0.1).astype(np.int32), truncated=np.zeros(n, np.int32))
    params = OP.init_parameters(obs_dim, act_dim, cfg)
    permutation = rng.permutation(n)
    full = OP.PPOOracle(obs_dim, act_dim, envs, horizon, cfg, params)
    full.update(rollout, permutation)
    first = OP.PPOOracle(obs_dim, act_dim, envs, horizon, cfg, params)
    first.prepare(rollout)
    half = n // 2
    for idx in (permutation[:half], permutation[half:], permutation[:half]):
        first.minibatch_step(idx)
    second = OP.PPOOracle(obs_dim, act_dim, envs, horizon, cfg, params)
    second.prepare(rollout)
    second.set_state([p.detach() for p in first.params], first.moments(), 3, first.learning_rate)
    second.minibatch_step(permutation[half:])
    for a, b in zip(full.params, second.params):
        assert torch.equal(a.detach(), b.detach())
    for (a1, a2), (b1, b2) in zip(full.moments(), second.moments()):
        assert torch.equal(a1, b1) and torch.equal(a2, b2)
    assert full.learning_rate == second.learning_rate


def test_gaussian_kl_closed_form():
    old_mean, new_mean = torch.tensor([[0.3]]), torch.tensor([[-0.1]])
    old_std, new_std = torch.tensor([[0.7]]), torch.tensor([[1.2]])
    kl = OP.gaussian_kl(old_mean, old_std, new_mean, new_std)
    expected = torch.distributions.kl_divergence(torch.distributions.Normal(old_mean, old_std),
                                                 torch.distributions.Normal(new_mean, new_std)).sum(-1)
    torch.testing.assert_close(kl, expected)


# ---------------------------------------------------------------------------
# native optimizer plans: Adam, loss scaling
# ---------------------------------------------------------------------------
from oracle import optim as OO  # noqa: E402


def test_native_adam_matches_torch_adam():
    rng = np.random.default_rng(3)
    shapes = [(7,), (33, 5)]
    params = [rng.standard_normal(s).astype(np.float32) for s in shapes]
    torch_params = [torch.tensor(p.copy(), requires_grad=True) for p in params]
    adam = torch.optim.Adam(torch_params, lr=3e-3, betas=(0.9, 0.999), eps=1e-8)
    m1 = [np.zeros_like(p) for p in params]
    m2 = [np.zeros_like(p) for p in params]
    state = {"timestep": np.float32(0)}
    for _ in range(6):
        grads = [rng.standard_normal(s).astype(np.float32) for s in shapes]
        OO.native_adam_step(params, grads, m1, m2, state, 3e-3, 0.9, 0.999, 1e-8)
        for tp, g in zip(torch_params, grads):
            tp.grad = torch.tensor(g)
        adam.step()
    assert state["timestep"] == 6
    for p, tp in zip(params, torch_params):
        np.testing.assert_allclose(p, tp.detach().numpy(), rtol=1e-6, atol=1e-7)


def test_native_adam_first_step_closed_form():
    g = np.array([3.0, -0.5, 1e-3, 0.0], np.float32)
    p = np.zeros(4, np.float32)
    OO.native_adam_step([p], [g.copy()], [np.zeros(4, np.float32)], [np.zeros(4, np.float32)],
                        {"timestep": np.float32(0)}, 0.1, 0.9, 0.99, 1e-8)
    np.testing.assert_allclose(p, -0.1 * g / (np.abs(g) + 1e-8), rtol=1e-5)


def _torch_scale_sequence(found, scale, growth, backoff, interval):
    s = torch.tensor([scale], dtype=torch.float32)
    tracker = torch.zeros(1, dtype=torch.int32)
    out = []
    for f in found:
        torch._amp_update_scale_(s, tracker, torch.tensor([float(f)]), growth, backoff, interval)
        out.append((float(s[0]), int(tracker[0])))
    return out


def test_scaled_prepare_matches_torch_update_scale():
    found = [0, 0, 1, 0, 0, 0, 1, 1, 0, 0, 0, 0, 0]
    state = {"loss_scale": np.float32(65536.0), "growth_tracker": 0, "step_skipped": 0, "attempted": 0,
             "skipped": 0}
    expected = _torch_scale_sequence(found, 65536.0, 2.0, 0.5, 3)
    for f, (scale, tracker) in zip(found, expected):
        ran = OO.scaled_prepare(state, f, 2.0, 0.5, 3)
        assert ran == (f == 0)
        assert state["loss_scale"] == np.float32(scale) and state["growth_tracker"] == tracker
    assert state["attempted"] == len(found) and state["skipped"] == sum(found)


def test_scaled_prepare_floor_and_overflow_guard():
    state = {"loss_scale": np.float32(2.0**-125), "growth_tracker": 0, "step_skipped": 0, "attempted": 0,
             "skipped": 0}
    for _ in range(4):
        OO.scaled_prepare(state, 1, 2.0, 0.5, 1)
    assert state["loss_scale"] == np.float32(2.0**-126)
    state["loss_scale"] = np.float32(3.0e38)
    OO.scaled_prepare(state, 0, 2.0, 0.5, 1)
    assert state["loss_scale"] == np.float32(3.0e38) and state["growth_tracker"] == 0


@pytest.mark.parametrize("poison", [None, np.inf, -np.inf, np.nan])
def test_unscale_matches_torch_check(poison):
    rng = np.random.default_rng(4)
    grads = [rng.standard_normal(n).astype(np.float32) * 1024 for n in (5, 300)]
    if poison is not None:
        grads[1][17] = poison
    torch_grads = [torch.tensor(g.copy()) for g in grads]
    found_t = torch.zeros(1)
    torch._amp_foreach_non_finite_check_and_unscale_(torch_grads, found_t, torch.tensor([1.0 / 1024]))
    found = OO.unscale(grads, 1024.0)
    assert found == int(found_t[0])
    for g, t in zip(grads, torch_grads):
        np.testing.assert_array_equal(np.isfinite(g), np.isfinite(t.numpy()))
        np.testing.assert_array_equal(g[np.isfinite(g)], t.numpy()[np.isfinite(g)])


def test_unscale_reference_only_cases():
    # finite gradient whose unscaled value overflows; non-positive scale
    assert OO.unscale([np.array([3.0e38], np.float32)], 0.5) == 1
    assert OO.unscale([np.array([1.0], np.float32)], 0.0) == 1
    assert OO.unscale([np.array([1.0], np.float32)], -2.0) == 1
    assert OO.unscale([np.array([1.0, 2.0], np.float32)], 4.0) == 0


# ---------------------------------------------------------------------------
# replay ingest (n-step commit) and reward statistics
# ---------------------------------------------------------------------------
from oracle import replay as OR  # noqa: E402


def test_n_step_replay_known_answer():
    """The reference's known answer, tests/test_flashsac.py:197-231."""
    replay = OR.NStepReplay(1, 1, n_step=3, gamma=0.5, capacity=16)
    for step, rewards in enumerate(([1.0, 1.0, 1.0], [2.0, 2.0, 2.0], [100.0, 4.0, 100.0])):
        replay.add([[step * 10.0], [step * 10.0 + 1], [step * 10.0 + 2]], np.zeros((3, 1)), rewards,
                   [False, False, step == 1], [step == 1, False, False],
                   [[(step + 1) * 10.0], [(step + 1) * 10.0 + 1], [(step + 1) * 10.0 + 2]])
    batch = replay.sample([0, 1, 2])
    np.testing.assert_array_equal(batch["reward"], [2.0, 3.0, 2.0])
    np.testing.assert_array_equal(batch["next_observation"], [[20.0], [31.0], [22.0]])
    np.testing.assert_array_equal(batch["discount"], [0.25, 0.125, 0.25])
    np.testing.assert_array_equal(batch["terminated"], [0.0, 0.0, 1.0])
    np.testing.assert_array_equal(batch["truncated"], [1.0, 0.0, 0.0])
    target = batch["reward"] + batch["discount"] * (1.0 - batch["terminated"]) * batch["next_observation"][:, 0]
    np.testing.assert_allclose(target, [7.0, 6.875, 2.0])
    assert replay.count == 3 and replay.position == 3


def _random_step(rng, envs, obs_dim, action_dim, done_prob):
    return dict(observation=rng.standard_normal((envs, obs_dim)).astype(np.float32),
                action=rng.uniform(-1, 1, (envs, action_dim)).astype(np.float32),
                reward=rng.standard_normal(envs).astype(np.float32),
                terminated=(rng.random(envs) < done_prob).astype(np.float32),
                truncated=(rng.random(envs) < done_prob).astype(np.float32),
                next_observation=rng.standard_normal((envs, obs_dim)).astype(np.float32))


@pytest.mark.parametrize("n_step", [1, 2, 3, 5])
def test_n_step_replay_matches_brute_force(n_step):
    rng = np.random.default_rng(n_step)
    envs, obs_dim, action_dim, capacity, gamma = 7, 3, 2, 40, 0.9
    replay = OR.NStepReplay(obs_dim, action_dim, n_step, gamma, capacity)
    history = []
    for step in range(15):
        t = _random_step(rng, envs, obs_dim, action_dim, done_prob=0.3)
        history.append(t)
        position = replay.position
        replay.add(**t)
        if step < n_step - 1:
            assert replay.count == 0
            continue
        rows = (np.arange(envs) + position) % capacity
        expected = OR.brute_force_commit(history, n_step, gamma)
        got = replay.sample(rows)
        np.testing.assert_allclose(got["reward"], expected["reward"], rtol=1e-6, atol=1e-6)
        np.testing.assert_allclose(got["discount"], expected["discount"], rtol=1e-6)
        np.testing.assert_array_equal(got["terminated"], expected["terminated"])
        np.testing.assert_array_equal(got["truncated"], expected["truncated"])
        np.testing.assert_array_equal(got["next_observation"], np.stack(expected["next_observation"]))
        np.testing.assert_array_equal(got["observation"], history[-n_step]["observation"])
        np.testing.assert_array_equal(got["action"], history[-n_step]["action"])
    assert replay.count == min(capacity, envs * (15 - n_step + 1))


def test_reward_stats_closed_forms():
    rng = np.random.default_rng(3)
    envs, gamma, steps = 9, 0.97, 12
    stats = OR.RewardStats(envs, gamma)
    returns = np.zeros(envs)
    seen, previous_vars = [], []
    for _ in range(steps):
        reward = rng.standard_normal(envs).astype(np.float32)
        term = (rng.random(envs) < 0.2).astype(np.float32)
        trunc = (rng.random(envs) < 0.1).astype(np.float32)
        previous_vars.append(float(stats.running[1]))
        stats.update(reward, term, trunc)
        done = (term != 0) | (trunc != 0)
        returns = np.where(done, 0.0, gamma * returns) + reward
        seen.append(returns.copy())
        np.testing.assert_allclose(stats.returns, returns, rtol=1e-5, atol=1e-6)
        values = np.concatenate(seen)
        assert stats.maximum[0] == pytest.approx(np.abs(values).max(), rel=1e-6)
        assert stats.running[2] == len(values)
        assert stats.running[0] == pytest.approx(values.mean(), rel=1e-5, abs=1e-6)
        total_squares = ((values - values.mean()) ** 2).sum() + 1e-4 * sum(previous_vars)
        assert stats.running[1] * len(values) == pytest.approx(total_squares, rel=1e-5)
    scaled = stats.scale(np.array([1.0, -2.0], np.float32), g_max=5.0)
    denominator = max(math.sqrt(stats.running[1] + 1e-8), stats.maximum[0] / 5.0)
    np.testing.assert_allclose(scaled, np.array([1.0, -2.0]) / denominator, rtol=1e-6)


# ---------------------------------------------------------------------------
# exploration-noise repeats (agent.py:159-214)
# ---------------------------------------------------------------------------
from oracle import explore as OX  # noqa: E402


@pytest.mark.parametrize("mu,max_n", [(2.0, 16), (0.0, 5), (1.5, 1)])
def test_zeta_cdf_closed_form(mu, max_n):
    cdf = OX.zeta_cdf(mu, max_n)
    harmonic = np.cumsum([k ** (-mu) for k in range(1, max_n + 1)])
    np.testing.assert_allclose(cdf.numpy(), harmonic / harmonic[-1], rtol=1e-6)
    if mu == 0.0:
        np.testing.assert_allclose(cdf.numpy(), np.arange(1, max_n + 1) / max_n, rtol=1e-6)


def test_sample_length_brute_force_and_all_false_mask():
    cdf = OX.zeta_cdf(2.0, 8)
    for u in np.linspace(0.0, float(cdf[-1]) - 1e-6, 57):
        assert OX.sample_length(float(u), cdf) == 1 + int((cdf.numpy() <= np.float32(u)).sum())
    # u beyond the last entry: the mask is all false and torch.argmax picks index 0
    assert int(torch.argmax(torch.zeros(8, dtype=torch.int32))) == 0
    assert OX.sample_length(float(cdf[-1]), cdf) == 1


def test_exploration_refresh_schedule():
    cdf = OX.zeta_cdf(0.0, 4)  # uniform lengths 1..4: u in [(L-1)/4, L/4) gives L
    lengths = [3, 1, 4, 2, 2, 1]
    state = OX.Exploration((2, 3))
    refresh_at, t = set(), 0
    for length in lengths:
        refresh_at.add(t)
        t += length
    schedule = iter(lengths)
    u_for = {L: (L - 0.5) / 4.0 for L in range(1, 5)}
    held = None
    for step in range(sum(lengths)):
        fresh = torch.full((2, 3), float(step))
        u = u_for[next(schedule)] if step in refresh_at else 0.9
        refreshed = state.step(u, fresh, cdf)
        assert refreshed == (step in refresh_at), step
        if refreshed:
            held = fresh
        torch.testing.assert_close(state.noise, held)
    mean, std = torch.zeros(2, 3), torch.full((2, 3), 0.5)
    torch.testing.assert_close(state.actions(mean, std), torch.tanh(0.5 * held))


@pytest.mark.parametrize("std_type", ["log", "scalar"])
def test_ppo_rollout_sample_log_prob_matches_normal(std_type):
    cfg = PPOConfig(std_type=std_type)
    g = torch.Generator().manual_seed(8)
    mean, noise = torch.randn(6, 5, generator=g, dtype=torch.float64), torch.randn(6, 5, generator=g, dtype=torch.float64)
    value = torch.randn(6, 1, generator=g, dtype=torch.float64)
    parameter = torch.randn(5, generator=g, dtype=torch.float64) * 0.5 + (0.0 if std_type == "log" else 0.6)
    actions, log_probs, values, std = OP.sample(mean, value, parameter, noise, cfg)
    expected_std = torch.exp(parameter) if std_type == "log" else parameter.clamp(*cfg.std_range)
    torch.testing.assert_close(std, expected_std)
    torch.testing.assert_close(actions, mean + expected_std * noise)
    reference = torch.distributions.Normal(mean, expected_std).log_prob(actions).sum(-1)
    torch.testing.assert_close(log_probs, reference, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(values, value[:, 0])
