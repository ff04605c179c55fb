"""PPO update on the GPU: the reference's known answers and parity with the CPU oracle."""

import math

import numpy as np
import pytest
import torch

from oracle import ppo as OP
from robolearn_amd import _native
from robolearn_amd import kernels as K
from robolearn_amd.config import PPOConfig

pytestmark = pytest.mark.gpu


def _agent(obs, act, envs, horizon, cfg):
    from robolearn_amd.ppo import WarpPPO

    return WarpPPO(obs, act, envs, horizon, cfg)


def test_gae_distinguishes_termination_timeout_and_rollout_boundary(gpu):
    """Known answer of tests/test_warp_ppo.py:23-46."""
    agent = _agent(1, 1, 2, 3, PPOConfig(hidden_dims=(), normalize_advantages=False, activation="elu"))
    reward = np.array([[1, 2], [3, 4], [5, 6]], dtype=np.float32)
    value = np.array([[0.1, 0.2], [0.3, 0.4], [0.5, 0.6]], dtype=np.float32)
    next_value = np.array([[0.3, 0.4], [9, 10], [11, 12]], dtype=np.float32)
    terminated = np.array([[0, 0], [1, 0], [0, 0]], dtype=np.int32)
    truncated = np.array([[0, 0], [0, 1], [0, 0]], dtype=np.int32)
    for name, data in (("rewards", reward), ("values", value), ("next_values", next_value),
                       ("terminated", terminated), ("truncated", truncated)):
        getattr(agent, name).copy_(torch.as_tensor(data.flatten()))
    expected = np.zeros_like(reward)
    tail = np.zeros(2, dtype=np.float32)
    for t in range(2, -1, -1):
        delta = reward[t] + 0.99 * (1 - terminated[t]) * next_value[t] - value[t]
        tail = delta + 0.99 * 0.95 * (1 - np.maximum(terminated[t], truncated[t])) * tail
        expected[t] = tail
    agent.compute_returns()
    np.testing.assert_allclose(agent.advantages.cpu().numpy().reshape(3, 2), expected, rtol=1e-6)
    np.testing.assert_allclose(agent.returns.cpu().numpy().reshape(3, 2), expected + value, rtol=1e-6)


def test_advantage_normalization_preserves_small_variance_at_large_offset(gpu):
    """Known answer of tests/test_warp_ppo.py:49-56."""
    agent = _agent(1, 1, 2, 1, PPOConfig(hidden_dims=(), gamma=0.0, activation="elu"))
    rewards = np.array([10000.0, 10001.0], dtype=np.float32)
    agent.rewards.copy_(torch.as_tensor(rewards))
    agent.compute_returns()
    np.testing.assert_allclose(agent.advantages.cpu().numpy(), [-1.0, 1.0], rtol=1e-6)
    np.testing.assert_array_equal(agent.returns.cpu().numpy(), rewards)


def test_clipped_gaussian_loss_and_gradient_match_reference(gpu):
    """Known answer + central finite differences of tests/test_warp_ppo.py:59-119."""
    mean_np = np.array([[0.4, 0.1], [-0.3, 0.2], [0.2, -0.2]], dtype=np.float32)
    action_np = np.array([[0.0, 0.5], [0.6, 0.1], [-0.5, 0.4]], dtype=np.float32)
    old_lp_np = np.array([-2.4, -1.8, -2.0], dtype=np.float32)
    advantage_np = np.array([1.0, -0.8, 0.4], dtype=np.float32)
    value_np = np.array([[0.8], [1.0], [-0.5]], dtype=np.float32)
    old_value_np = np.array([0.2, 1.3, -0.4], dtype=np.float32)
    return_np = np.array([0.7, -0.2, 1.0], dtype=np.float32)
    log_std_np = np.array([-0.2, 0.1], dtype=np.float32)
    d = lambda a: torch.as_tensor(a).to(gpu).contiguous()  # noqa: E731
    dmean, dvalue, dstd_rows = d(np.zeros((3, 2), np.float32)), d(np.zeros(3, np.float32)), d(np.zeros((3, 2), np.float32))
    row_terms, totals = d(np.zeros((4, 3), np.float32)), d(np.zeros(4, np.float32))
    args = [d(mean_np), d(value_np), d(log_std_np), d(action_np), d(old_lp_np), d(old_value_np), d(advantage_np),
            d(return_np)]
    _native.call("rl_ppo_loss", args[0].data_ptr(), 2, args[1].data_ptr(), args[2].data_ptr(), args[3].data_ptr(),
                 args[4].data_ptr(), args[5].data_ptr(), args[6].data_ptr(), args[7].data_ptr(), 3, 2, 0, 1e-6, 1e6,
                 0.2, 0.5, 0.01, 0.5, 1, dmean.data_ptr(), dvalue.data_ptr(), dstd_rows.data_ptr(),
                 row_terms.data_ptr(), totals.data_ptr(), K.stream())
    torch.cuda.synchronize()

    def reference(mean_values=mean_np, value_values=value_np, std_values=log_std_np):
        lp = (-0.5 * (((action_np - mean_values) * np.exp(-std_values)) ** 2 + 2 * std_values + np.log(2 * np.pi))).sum(1)
        ratio = np.exp(lp - old_lp_np)
        policy = -np.minimum(ratio * advantage_np, np.clip(ratio, 0.8, 1.2) * advantage_np).mean()
        clipped_value = old_value_np + np.clip(value_values[:, 0] - old_value_np, -0.2, 0.2)
        value_loss = 0.5 * np.maximum((value_values[:, 0] - return_np) ** 2, (clipped_value - return_np) ** 2).mean()
        entropy = (std_values + 0.5 * np.log(2 * np.pi * np.e)).sum()
        return policy + 0.5 * value_loss - 0.01 * entropy

    np.testing.assert_allclose(totals.cpu().numpy()[0], reference(), rtol=1e-5, atol=1e-7)
    gradients = {"mean_values": dmean.cpu().numpy(), "value_values": dvalue.cpu().numpy().reshape(3, 1),
                 "std_values": dstd_rows.cpu().numpy().sum(0)}
    for argument, data in (("mean_values", mean_np), ("value_values", value_np), ("std_values", log_std_np)):
        numerical = np.zeros_like(data)
        for index in np.ndindex(data.shape):
            plus, minus = data.copy(), data.copy()
            plus[index] += 1e-3
            minus[index] -= 1e-3
            numerical[index] = (reference(**{argument: plus}) - reference(**{argument: minus})) / 2e-3
        np.testing.assert_allclose(gradients[argument], numerical, atol=2e-4, rtol=2e-3, err_msg=argument)


def _config(**overrides):
    base = dict(hidden_dims=(16, 8), activation="elu", std_type="scalar", epochs=5, num_mini_batches=4,
                learning_rate=1.0e-3, schedule="adaptive", desired_kl=0.01, value_coefficient=1.0,
                value_loss_scale=1.0, entropy_coefficient=0.008, advantage_sample_std=True,
                timeout_bootstrap="current", separate_grad_clipping=True)
    base.update(overrides)
    return PPOConfig(**base)


def _rollout(agent, seed=29):
    """The fixed rollout of examples/diagnose_ppo_update.py:50-72 (synthetic, seeded)."""
    rng = np.random.default_rng(seed)
    n, obs_dim, act_dim = agent.batch_size, agent.observation_dim, agent.action_dim
    observations = rng.normal(size=(n, obs_dim)).astype(np.float32)
    means = rng.normal(scale=0.3, size=(n, act_dim)).astype(np.float32)
    actions = means + rng.normal(size=(n, act_dim)).astype(np.float32)
    data = {
        "observations": observations, "actions": actions, "means": means, "stds": np.ones_like(means),
        "values": rng.normal(scale=0.5, size=n).astype(np.float32),
        "log_probs": (-0.5 * ((actions - means) ** 2 + math.log(2 * math.pi))).sum(1).astype(np.float32),
        "rewards": rng.normal(0.2, 0.05, size=n).astype(np.float32),
        "next_values": rng.normal(0.0, 0.2, size=n).astype(np.float32),
        "terminated": np.zeros(n, dtype=np.int32), "truncated": np.zeros(n, dtype=np.int32),
    }
    data["terminated"][min(18, n - 1)] = 1
    data["truncated"][min(39, n - 2)] = 1
    for key, value in data.items():
        getattr(agent, key).copy_(torch.as_tensor(value))
    return data


@pytest.mark.parametrize("separate", [True, False])
def test_update_matches_oracle(gpu, separate):
    cfg = _config(separate_grad_clipping=separate)
    agent = _agent(7, 3, 16, 4, cfg)
    initial = agent.state_dict()
    data = _rollout(agent)
    agent.launch_update()
    torch.cuda.synchronize()
    permutation = agent._perm.cpu().numpy().astype(np.int64)
    assert np.array_equal(np.sort(permutation), np.arange(agent.batch_size))
    oracle = OP.PPOOracle(7, 3, 16, 4, cfg, [initial[f"parameter_{i}"] for i in range(len(agent.parameters))])
    result = oracle.update(data, permutation)
    state = agent.state_dict()
    health = agent.health_metrics()
    assert health["learning_rate"] == pytest.approx(result["learning_rate"], rel=1e-6)
    assert health["kl"] == pytest.approx(result["kl"], rel=1e-4, abs=1e-7)
    assert health["policy_loss"] == pytest.approx(result["policy_loss"], rel=1e-4, abs=1e-6)
    assert health["value_loss"] == pytest.approx(result["value_loss"], rel=1e-4, abs=1e-6)
    assert health["entropy"] == pytest.approx(result["entropy"], rel=1e-4, abs=1e-6)
    np.testing.assert_allclose(agent.advantages.cpu().numpy(), oracle.advantages.numpy(), atol=1e-5)
    np.testing.assert_allclose(agent.returns.cpu().numpy(), oracle.returns.numpy(), atol=1e-5)
    moments = oracle.moments()
    for i, p in enumerate(oracle.params):
        np.testing.assert_allclose(state[f"parameter_{i}"], p.detach().numpy(), atol=2e-4, rtol=0, err_msg=str(i))
        np.testing.assert_allclose(state[f"adam_m1_{i}"].reshape(-1), moments[i][0].numpy().reshape(-1), atol=2e-4)
        np.testing.assert_allclose(state[f"adam_m2_{i}"].reshape(-1), moments[i][1].numpy().reshape(-1), atol=2e-4)


def test_captured_update_matches_eager_and_checkpoint_preserves_graph(gpu, tmp_path):
    """Mirrors tests/test_warp_ppo.py:122-148."""
    config = PPOConfig(hidden_dims=(16,), epochs=2, activation="elu")
    eager = _agent(3, 2, 8, 4, config)
    captured = _agent(3, 2, 8, 4, config)
    captured.load_state_dict(eager.state_dict())
    rng = np.random.default_rng(7)
    for name, shape in (("observations", (32, 3)), ("actions", (32, 2)), ("rewards", (32,))):
        samples = torch.as_tensor(rng.normal(size=shape).astype(np.float32))
        getattr(eager, name).copy_(samples)
        getattr(captured, name).copy_(samples)
    for _ in range(2):
        eager.update(capture=False)
        captured.update()
    for expected, actual in zip(eager.parameters, captured.parameters):
        np.testing.assert_allclose(actual.cpu().numpy(), expected.cpu().numpy(), rtol=2e-5, atol=2e-6)
    checkpoint = tmp_path / "ppo.npz"
    captured.save(checkpoint)
    saved = captured.state_dict()
    captured.update()
    captured.load(checkpoint)
    for key, value in saved.items():
        np.testing.assert_array_equal(captured.state_dict()[key], value)
    captured.update()
    eager.update(capture=False)
    for expected, actual in zip(eager.parameters, captured.parameters):
        np.testing.assert_allclose(actual.cpu().numpy(), expected.cpu().numpy(), rtol=2e-5, atol=2e-6)


@pytest.mark.parametrize("std_type", ["log", "scalar"])
def test_rollout_act_and_store_match_oracle(gpu, std_type):
    """act() (ppo.py:26-58, 488-507) and store() (ppo.py:61-99, 509-550) against oracle.ppo.sample with the
    device's own noise draw read back; the rollout rows land where update() reads them."""
    print(f"case PPO rollout act/store std_type={std_type}", flush=True)
    cfg = PPOConfig(hidden_dims=(16, 8), activation="elu", std_type=std_type, epochs=1, num_mini_batches=2)
    E, T, O, A = 8, 3, 5, 3
    agent = _agent(O, A, E, T, cfg)
    state = agent.state_dict()
    params = [torch.as_tensor(state[f"parameter_{i}"]).double() for i in range(len(agent.parameters))]
    layers = 2 * (len(cfg.hidden_dims) + 1)
    actor, critic, parameter = params[:layers], params[layers:2 * layers], params[-1]
    if std_type == "scalar":  # spread the std parameter across the clamp range
        parameter = torch.tensor([0.005, 0.7, 5.0], dtype=torch.float64)
        agent.distribution_parameter.copy_(parameter.float())
        parameter = parameter.float().double()
    g = torch.Generator().manual_seed(11)
    expected = {k: [] for k in ("observations", "actions", "log_probs", "values", "rewards", "terminated",
                                "truncated", "next_values", "means")}
    for t in range(T):
        obs, next_obs = torch.randn(E, O, generator=g), torch.randn(E, O, generator=g)
        rewards = torch.randn(E, generator=g)
        terminated = (torch.rand(E, generator=g) < 0.3).int()
        truncated = (torch.rand(E, generator=g) < 0.2).int()
        actions = agent.act(obs.to(gpu)).cpu().double()
        sampled = agent._act_state(E)
        noise = sampled["noise"].cpu().double()
        mean = OP.mlp(obs.double(), actor, "elu")
        value = OP.mlp(obs.double(), critic, "elu")
        exp_actions, exp_lp, exp_values, exp_std = OP.sample(mean, value, parameter, noise, cfg)
        torch.testing.assert_close(actions, exp_actions, rtol=1e-5, atol=1e-5)
        torch.testing.assert_close(sampled["log_probs"].cpu().double(), exp_lp, rtol=1e-5, atol=1e-5)
        torch.testing.assert_close(sampled["values"].cpu().double(), exp_values, rtol=1e-5, atol=1e-5)
        torch.testing.assert_close(sampled["std"].cpu().double(), exp_std, rtol=1e-6, atol=0)
        agent.store(t, obs.to(gpu), rewards.to(gpu), terminated.to(gpu), truncated.to(gpu), next_obs.to(gpu))
        for key, value_ in (("observations", obs.double()), ("actions", actions), ("log_probs", exp_lp),
                            ("values", exp_values), ("rewards", rewards.double()),
                            ("terminated", terminated.double()), ("truncated", truncated.double()),
                            ("next_values", OP.mlp(next_obs.double(), critic, "elu")[:, 0]), ("means", mean)):
            expected[key].append(value_)
    torch.cuda.synchronize()
    for key, parts in expected.items():
        got = getattr(agent, key).cpu().double()
        torch.testing.assert_close(got, torch.cat(parts), rtol=1e-5, atol=1e-5, msg=key)
    torch.testing.assert_close(agent.stds.cpu().double(), exp_std.expand(E * T, A), rtol=1e-6, atol=0)
    np.testing.assert_array_equal(agent.observations.cpu().numpy(), torch.cat(expected["observations"]).numpy())
    # deterministic acting uses the mean and leaves the draw counter alone
    counter = agent._act_counter.item()
    obs = torch.randn(E, O, generator=g)
    torch.testing.assert_close(agent.act(obs.to(gpu), deterministic=True).cpu().double(),
                               OP.mlp(obs.double(), actor, "elu"), rtol=1e-5, atol=1e-5)
    assert agent._act_counter.item() == counter == T
    # the device draws are standard normal and change with every call
    big = _agent(O, A, 4096, 1, cfg)
    big.act(torch.randn(4096, O, generator=g).to(gpu))
    first = big._act_state(4096)["noise"].clone()
    big.act(torch.randn(4096, O, generator=g).to(gpu))
    second = big._act_state(4096)["noise"]
    assert abs(first.mean().item()) < 0.03 and abs(first.std().item() - 1.0) < 0.03
    assert not torch.equal(first, second)


@pytest.mark.parametrize("n,scale", [(1000, 1e-3), (232_522 + 227_841, 0.7), (460_363, 25.0), (5, 3.0)])
def test_sum_squares_and_clip_closed_form(gpu, n, scale):
    """rl_sum_squares + rl_clip_by_norm (robolearn/warp/ppo.py:241-252): below the threshold the gradient
    is unchanged; above it g * max_norm / (||g|| + 1e-6), so the post-clip norm is
    max_norm ||g|| / (||g|| + 1e-6).  The middle sizes are the c3 actor + critic parameter count, the
    combined group of the default (non-separate) mode."""
    print(f"case clip n={n} scale={scale}", flush=True)
    g = torch.Generator().manual_seed(n)
    grad = torch.randn(n, generator=g)
    grad = grad * (scale / grad.double().norm().item())
    device = grad.to(gpu)
    partial = torch.empty((n + 4095) // 4096, device=gpu)
    sum_squares = torch.empty(1, device=gpu)
    _native.call("rl_sum_squares", device.data_ptr(), n, partial.data_ptr(), sum_squares.data_ptr(), K.stream())
    _native.call("rl_clip_by_norm", device.data_ptr(), n, sum_squares.data_ptr(), 1.0, K.stream())
    torch.cuda.synchronize()
    norm = grad.double().norm().item()
    assert sum_squares.item() == pytest.approx(norm * norm, rel=1e-5)
    clipped = device.cpu().double()
    if norm + 1e-6 <= 1.0:
        assert torch.equal(device.cpu(), grad)
    else:
        assert clipped.norm().item() == pytest.approx(norm / (norm + 1e-6), rel=1e-5)
        torch.testing.assert_close(clipped, grad.double() / (norm + 1e-6), rtol=1e-5, atol=1e-9)


@pytest.mark.parametrize("n,scale", [(1000, 1e-3), (232_522 + 227_841, 0.7), (460_363, 25.0)])
def test_fused_clip_equals_sum_squares_then_clip(gpu, n, scale):
    """rl_clip_grad_norm (the update's two-launch form) leaves the same sum of squares and the same
    clipped gradient, bit for bit, as rl_sum_squares followed by rl_clip_by_norm."""
    print(f"case fused clip n={n} scale={scale}", flush=True)
    g = torch.Generator().manual_seed(n + 1)
    grad = torch.randn(n, generator=g)
    grad = (grad * (scale / grad.double().norm().item())).float().to(gpu)
    blocks = (n + 4095) // 4096
    a, b = grad.clone(), grad.clone()
    pa, pb = torch.empty(blocks, device=gpu), torch.empty(blocks, device=gpu)
    sa, sb = torch.empty(1, device=gpu), torch.empty(1, device=gpu)
    _native.call("rl_sum_squares", a.data_ptr(), n, pa.data_ptr(), sa.data_ptr(), K.stream())
    _native.call("rl_clip_by_norm", a.data_ptr(), n, sa.data_ptr(), 1.0, K.stream())
    _native.call("rl_clip_grad_norm", b.data_ptr(), n, pb.data_ptr(), sb.data_ptr(), 1.0, K.stream())
    torch.cuda.synchronize()
    assert torch.equal(sa, sb)
    assert torch.equal(a, b)


def _plain_adam_plan(sizes, param, grad, m1, m2, timestep, lr):
    offsets = np.cumsum([0] + sizes[:-1]).tolist()
    ptrs = lambda buf: _native.pointer_array([buf[o:o + s].data_ptr() for o, s in zip(offsets, sizes)])  # noqa
    n = len(sizes)
    return _native.create("rl_fused_optimizer_create", n, _native.int_array([3] * n), _native.ll_array([1] * n),
                          _native.ll_array(sizes), ptrs(param), ptrs(grad), ptrs(m1), ptrs(m2), None, None, None,
                          _native.int_array([-1] * n), timestep.data_ptr(), lr.data_ptr(), 0.9, 0.999, 1e-8, 0.0, 1,
                          0, 0.0, 0.0, 0.0, 0, 1)


@pytest.mark.parametrize("scale", [0.3, 25.0])
def test_clipped_optimizer_step_equals_clip_then_step(gpu, scale):
    """rl_fused_optimizer_step_clipped (clipping folded into the Adam step, the combined-clipping PPO
    update) leaves the same parameters, moments, clipped gradients, sum of squares and timestep, bit for
    bit, as rl_clip_grad_norm followed by rl_fused_optimizer_step, over three steps, below and above the
    norm bound, over tensors of the c3 layer sizes (4-aligned and not)."""
    print(f"case clipped optimizer step scale={scale}", flush=True)
    sizes = [123 * 512, 512, 512 * 256, 256, 37, 256 * 128, 128, 37 * 128, 37, 1]
    g = torch.Generator().manual_seed(17)
    n = sum(sizes)
    param0 = torch.randn(n, generator=g)
    states = []
    for _ in range(2):
        buffers = [param0.clone().to(gpu), torch.zeros(n, device=gpu), torch.zeros(n, device=gpu),
                   torch.zeros(n, device=gpu), torch.zeros(1, device=gpu), torch.full((1,), 1e-3, device=gpu)]
        states.append((buffers, _plain_adam_plan(sizes, *buffers)))
    blocks = (n + 4095) // 4096
    try:
        for step in range(3):
            grad = torch.randn(n, generator=g)
            grad = (grad * (scale / grad.double().norm().item())).float()
            outputs = []
            for variant, (buffers, plan) in enumerate(states):
                buffers[1].copy_(grad)
                partial, sum_squares = torch.empty(blocks, device=gpu), torch.empty(1, device=gpu)
                if variant == 0:
                    _native.call("rl_clip_grad_norm", buffers[1].data_ptr(), n, partial.data_ptr(),
                                 sum_squares.data_ptr(), 1.0, K.stream())
                    _native.call("rl_fused_optimizer_step", plan, 1, 0, 0, None, K.stream())
                else:
                    _native.call("rl_fused_optimizer_step_clipped", plan, 0, 0, buffers[1].data_ptr(), n,
                                 partial.data_ptr(), sum_squares.data_ptr(), 1.0, K.stream())
                torch.cuda.synchronize()
                outputs.append([b.cpu() for b in buffers[:5]] + [sum_squares.cpu()])
            for name, x, y in zip(("param", "grad", "m1", "m2", "timestep", "sum_squares"), *outputs):
                assert torch.equal(x, y), (step, name)
            assert outputs[0][5].item() == pytest.approx(scale * scale, rel=1e-5)
        # a gradient range that misses some of the plan's gradients is refused before any launch
        buffers, plan = states[1]
        partial, sum_squares = torch.empty(blocks, device=gpu), torch.empty(1, device=gpu)
        with pytest.raises(RuntimeError, match="every gradient of the optimizer plan"):
            _native.call("rl_fused_optimizer_step_clipped", plan, 0, 0, buffers[1].data_ptr(), n - 1,
                         partial.data_ptr(), sum_squares.data_ptr(), 1.0, K.stream())
    finally:
        for _, plan in states:
            _native.load().rl_fused_optimizer_destroy(plan)


def _device_kl_adapt(lr, old_mean, desired_kl):
    """rl_ppo_kl_adapt on one row with one action, unit old and new std (std_type 1, clamped): the
    KL is 0.5 d^2 for d = old_mean, exact in fp32 for dyadic d.  Returns (kl, learning rate)."""
    dev = torch.device("cuda:0")
    mean = torch.zeros(1, 1, device=dev)
    std_param = torch.ones(1, device=dev)
    old_m = torch.full((1, 1), float(old_mean), device=dev)
    old_s = torch.ones(1, 1, device=dev)
    partial = torch.zeros(1, device=dev)
    kl = torch.zeros(1, device=dev)
    lr_t = torch.full((1,), float(lr), device=dev)
    _native.call("rl_ppo_kl_adapt", mean.data_ptr(), 1, std_param.data_ptr(), old_m.data_ptr(), old_s.data_ptr(),
                 1, 1, 1, 1e-3, 10.0, float(desired_kl), 1, partial.data_ptr(), kl.data_ptr(), lr_t.data_ptr(),
                 K.stream())
    torch.cuda.synchronize()
    return kl.item(), lr_t.item()


def test_adaptive_learning_rate_rule_known_answers_on_device(gpu):
    """The device rule against hand-worked answers of robolearn/warp/ppo.py:233-238 (tests/test_oracle_pins.py
    holds the same cases for the oracle).  With desired_kl 2^-6 both thresholds are dyadic (2 x target
    = 0.5 * 0.25^2, target / 2 = 0.5 * 0.125^2), so KL lands exactly on them and the strict comparisons
    are exercised; the desired_kl 0.01 cases sit away from the thresholds."""
    f32 = np.float32
    cases = [  # (lr, d, desired_kl, expected lr computed in fp32)
        (1e-3, 0.25, 2.0 ** -6, f32(1e-3)),                                # KL == 2 target: unchanged
        (1e-3, 0.25 * (1 + 2.0 ** -10), 2.0 ** -6, f32(1e-3) / f32(1.5)),  # just above: lowered
        (1e-3, 0.25 * (1 - 2.0 ** -10), 2.0 ** -6, f32(1e-3)),             # just below: unchanged
        (1e-3, 0.125, 2.0 ** -6, f32(1e-3)),                               # KL == target / 2: unchanged
        (1e-3, 0.125 * (1 - 2.0 ** -10), 2.0 ** -6, f32(1e-3) * f32(1.5)),  # just below: raised
        (1e-3, 0.0, 2.0 ** -6, f32(1e-3)),                                 # KL == 0: unchanged
        (1e-3, math.sqrt(2 * 0.0025), 0.01, f32(1e-3) * f32(1.5)),         # KL 0.0025: raised
        (1e-3, math.sqrt(2 * 0.01), 0.01, f32(1e-3)),                      # KL 0.01: unchanged
        (1e-3, math.sqrt(2 * 0.03), 0.01, f32(1e-3) / f32(1.5)),           # KL 0.03: lowered
        (1.2e-5, math.sqrt(2 * 0.03), 0.01, f32(1e-5)),                    # floor
        (8e-3, math.sqrt(2 * 0.001), 0.01, f32(1e-2)),                     # cap
    ]
    for lr, d, desired, expected in cases:
        kl, got = _device_kl_adapt(lr, d, desired)
        # 0.5 (1 + d^2 - 1) cancels in fp32: absolute error about ulp(1) for small d, exact for dyadic d
        assert kl == pytest.approx(0.5 * d * d, rel=1e-6, abs=2e-7), (lr, d, desired)
        assert got == pytest.approx(float(expected), rel=1e-7, abs=0.0), (lr, d, desired, kl, got)
        assert OP.adapt_learning_rate(float(f32(lr)), kl, desired) == pytest.approx(got, rel=1e-6), (lr, d, desired)


@pytest.mark.parametrize("obs_dim, act_dim", [(123, 37), (310, 12), (40, 70)])
def test_minibatch_gather_is_exact_for_narrow_and_wide_rows(gpu, obs_dim, act_dim):
    """rl_ppo_gather copies the permuted rows bit for bit, in the register-batched layout (rows up to
    256 observations and 64 actions) and the per-row strided one beyond it (robolearn/warp/ppo.py:172-204)."""
    print(f"case ppo gather obs {obs_dim} act {act_dim}", flush=True)
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(obs_dim + act_dim)
    n, rows, offset = 1000, 301, 37
    obs_ld = (obs_dim + 3) // 4 * 4
    src = {"obs": torch.randn(n, obs_dim, generator=g), "actions": torch.randn(n, act_dim, generator=g),
           "means": torch.randn(n, act_dim, generator=g), "stds": torch.rand(n, act_dim, generator=g)}
    for key in ("log_probs", "values", "advantages", "returns"):
        src[key] = torch.randn(n, generator=g)
    perm = torch.randperm(n, generator=g).to(torch.int32)
    d = {k: v.to(dev) for k, v in src.items()}
    out = {"obs": torch.full((rows, obs_ld), 7.0, device=dev)}
    for key in ("actions", "means", "stds"):
        out[key] = torch.zeros(rows, act_dim, device=dev)
    for key in ("log_probs", "values", "advantages", "returns"):
        out[key] = torch.zeros(rows, device=dev)
    perm_d = perm.to(dev)
    _native.call("rl_ppo_gather", perm_d.data_ptr(), offset, rows, obs_dim, act_dim, obs_ld, d["obs"].data_ptr(),
                 d["actions"].data_ptr(), d["log_probs"].data_ptr(), d["values"].data_ptr(),
                 d["advantages"].data_ptr(), d["returns"].data_ptr(), d["means"].data_ptr(), d["stds"].data_ptr(),
                 out["obs"].data_ptr(), out["actions"].data_ptr(), out["log_probs"].data_ptr(),
                 out["values"].data_ptr(), out["advantages"].data_ptr(), out["returns"].data_ptr(),
                 out["means"].data_ptr(), out["stds"].data_ptr(), K.stream())
    torch.cuda.synchronize()
    idx = perm[offset: offset + rows].long()
    got_obs = out["obs"].cpu()
    assert torch.equal(got_obs[:, :obs_dim], src["obs"][idx])
    assert torch.all(got_obs[:, obs_dim:] == 7.0)  # padding columns untouched
    for key in ("actions", "means", "stds", "log_probs", "values", "advantages", "returns"):
        assert torch.equal(out[key].cpu(), src[key][idx]), key


def test_update_with_wide_observations_matches_oracle(gpu):
    """A 310-observation policy (wider than the register-batched gather) against the oracle."""
    print("case ppo update obs 310 vs oracle", flush=True)
    cfg = _config()
    agent = _agent(310, 3, 16, 4, cfg)
    initial = agent.state_dict()
    data = _rollout(agent)
    agent.launch_update()
    torch.cuda.synchronize()
    permutation = agent._perm.cpu().numpy().astype(np.int64)
    oracle = OP.PPOOracle(310, 3, 16, 4, cfg, [initial[f"parameter_{i}"] for i in range(len(agent.parameters))])
    result = oracle.update(data, permutation)
    state = agent.state_dict()
    health = agent.health_metrics()
    assert health["learning_rate"] == pytest.approx(result["learning_rate"], rel=1e-6)
    assert health["policy_loss"] == pytest.approx(result["policy_loss"], rel=1e-4, abs=1e-6)
    assert health["value_loss"] == pytest.approx(result["value_loss"], rel=1e-4, abs=1e-6)
    for i, p in enumerate(oracle.params):
        np.testing.assert_allclose(state[f"parameter_{i}"], p.detach().numpy(), atol=2e-4, rtol=0, err_msg=str(i))
