"""Write golden vectors for the FlashSAC network pieces from the reference modules.

Runs only where the reference tree is mounted (this build container); the GPU
box reads the committed ``flashsac_modules.npz`` instead.  Imports, from
/root/reference/src, only modules whose imports are torch/numpy:
  robolearn/flashsac/layers.py, networks.py,
  robolearn/flashsac/_utils/network.py, scheduler.py, distribution.py.
updates.py and agent.py are not imported (they need gymnasium, which the image
lacks, and no stand-in is written for it).

Reparameterization noise is injected by replacing Normal.rsample for the
duration of a call, as examples/diagnose_warp_flashsac.py:311-329 does.

Usage: python tests/golden/make_golden.py [reference_src]
"""

import sys
from contextlib import contextmanager
from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent / "flashsac_modules.npz"


@contextmanager
def injected_noise(noise):
    original = torch.distributions.Normal.rsample

    def rsample(self, sample_shape=torch.Size()):
        return self.loc + noise * self.scale

    torch.distributions.Normal.rsample = rsample
    try:
        yield
    finally:
        torch.distributions.Normal.rsample = original


def main(src: str) -> None:
    sys.dont_write_bytecode = True  # the reference tree is read-only input: leave no __pycache__ in it
    sys.path.insert(0, src)
    from robolearn.flashsac._utils.distribution import safe_tanh_log_det_jacobian
    from robolearn.flashsac._utils.network import Network
    from robolearn.flashsac._utils.scheduler import warmup_cosine_decay_scheduler
    from robolearn.flashsac.networks import FlashSACActor, FlashSACDoubleCritic, FlashSACTemperature

    torch.set_num_threads(1)
    out = {}
    O, A, R, K = 4, 2, 32, 11
    g = torch.Generator().manual_seed(123)

    # ---------------- actor ----------------
    torch.manual_seed(0)
    actor_net = FlashSACActor(num_blocks=1, input_dim=O, hidden_dim=16, action_dim=A)
    actor = Network(network=actor_net, use_weight_normalization=True)
    actor.normalize_parameters()
    for name, value in actor_net.state_dict().items():
        out[f"actor.init.{name}"] = value.numpy().copy()
    x = torch.randn(2 * R, O, generator=g) * 1.5 + 0.3
    noise = torch.randn(2 * R, A, generator=g)
    out["actor.train.x"], out["actor.train.noise"] = x.numpy(), noise.numpy()
    with injected_noise(noise):
        actions, info = actor_net(x, training=True)
    coef = torch.randn(2 * R, A, generator=g)
    loss = (0.3 * info["log_prob"]).mean() + (coef * actions).mean()
    loss.backward()
    out["actor.train.coef"] = coef.numpy()
    out["actor.train.actions"] = actions.detach().numpy()
    out["actor.train.log_prob"] = info["log_prob"].detach().numpy()
    for name, value in actor_net.named_parameters():
        out[f"actor.grad.{name}"] = value.grad.numpy().copy()
    for name, value in actor_net.named_buffers():
        out[f"actor.after.{name}"] = value.numpy().copy()
    x_eval = torch.randn(R, O, generator=g)
    noise_eval = torch.randn(R, A, generator=g)
    out["actor.eval.x"], out["actor.eval.noise"] = x_eval.numpy(), noise_eval.numpy()
    with torch.no_grad(), injected_noise(noise_eval):
        actions_eval, info_eval = actor_net(x_eval, training=False)
        mean_eval, std_eval = actor_net.get_mean_and_std(x_eval, training=False)
    out["actor.eval.actions"] = actions_eval.numpy()
    out["actor.eval.log_prob"] = info_eval["log_prob"].numpy()
    out["actor.eval.mean"], out["actor.eval.std"] = mean_eval.numpy(), std_eval.numpy()

    # ---------------- critic ----------------
    torch.manual_seed(1)
    critic_net = FlashSACDoubleCritic(num_blocks=2, input_dim=O + A, hidden_dim=16, num_bins=K, min_v=-10.0,
                                      max_v=10.0)
    critic = Network(network=critic_net, use_weight_normalization=True)
    critic.normalize_parameters()
    with torch.no_grad():  # non-trivial BN affine and head bias
        for name, value in critic_net.named_parameters():
            if name.endswith("bias"):
                value.copy_(torch.randn(value.shape, generator=g) * 0.1)
    for name, value in critic_net.state_dict().items():
        out[f"critic.init.{name}"] = value.numpy().copy()
    obs = torch.randn(R, O, generator=g)
    act = torch.rand(R, A, generator=g) * 2 - 1
    out["critic.train.obs"], out["critic.train.act"] = obs.numpy(), act.numpy()
    qs, qinfo = critic_net(obs, act, training=True)
    cq = torch.randn(2, R, generator=g)
    clp = torch.randn(2, R, K, generator=g)
    loss = (cq * qs).sum() + (clp * qinfo["log_prob"]).sum() * 0.05
    loss.backward()
    out["critic.train.cq"], out["critic.train.clp"] = cq.numpy(), clp.numpy()
    out["critic.train.q"] = qs.detach().numpy()
    out["critic.train.log_prob"] = qinfo["log_prob"].detach().numpy()
    for name, value in critic_net.named_parameters():
        out[f"critic.grad.{name}"] = value.grad.numpy().copy()
    for name, value in critic_net.named_buffers():
        out[f"critic.after.{name}"] = value.numpy().copy()
    with torch.no_grad():
        qs_eval, qinfo_eval = critic_net(obs, act, training=False)
    out["critic.eval.q"] = qs_eval.numpy()
    out["critic.eval.log_prob"] = qinfo_eval["log_prob"].numpy()

    # ---------------- projection and EMA ----------------
    with torch.no_grad():
        for value in critic_net.parameters():
            value.add_(torch.randn(value.shape, generator=g) * 0.3)
    for name, value in critic_net.named_parameters():
        out[f"project.before.{name}"] = value.detach().numpy().copy()
    critic.normalize_parameters()
    for name, value in critic_net.named_parameters():
        out[f"project.after.{name}"] = value.detach().numpy().copy()
    target_net = FlashSACDoubleCritic(num_blocks=2, input_dim=O + A, hidden_dim=16, num_bins=K, min_v=-10.0,
                                      max_v=10.0)
    target = Network(network=target_net, use_weight_normalization=True, ema_source=critic, ema_tau=0.005)
    for name, value in target_net.named_parameters():
        out[f"ema.before.{name}"] = value.detach().numpy().copy()
    target.ema_update_parameters()
    for name, value in target_net.named_parameters():
        out[f"ema.after.{name}"] = value.detach().numpy().copy()

    # ---------------- schedule, log-det, temperature ----------------
    steps = np.array([0, 1, 2, 5, 9, 10, 11, 50, 99, 100, 150], dtype=np.int64)
    for label, args in (("a", (3e-4, 3e-4, 1.5e-4, 0, 100)), ("b", (1e-5, 3e-4, 1e-4, 10, 100))):
        f = warmup_cosine_decay_scheduler(*args)
        out[f"schedule.{label}.args"] = np.array(args, dtype=np.float64)
        out[f"schedule.{label}.values"] = np.array([f(int(s)) for s in steps], dtype=np.float64)
    out["schedule.steps"] = steps
    z = torch.linspace(-30, 30, 61)
    out["logdet.x"], out["logdet.y"] = z.numpy(), safe_tanh_log_det_jacobian(z).numpy()
    out["temperature.value"] = FlashSACTemperature(0.01)().detach().numpy()
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src")
