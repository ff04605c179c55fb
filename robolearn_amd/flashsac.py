"""FlashSAC learner on MI355X: one gradient update as a fixed sequence of HIP
kernels over persistent buffers, captured once per phase in a HIP graph.

Public interface mirrors the reference learners:
  constructor, update, update_from_batch, launch_update, prepare/warmup,
  capture_update, state_dict/load_state_dict, save/load, parameters,
  get_metrics, act, observe, ready
  (robolearn/warp/flashsac.py:340-1239; robolearn/flashsac/agent.py:295-601).
The update order and losses follow robolearn/flashsac/agent.py:217-281 and
updates.py:83-326: [actor -> temperature] on actor phases, then critic (with
the updated actor and temperature), then the target EMA.  The critic phase
runs the twin critics as one two-member ensemble.

Random draws: replay indices and the reparameterization noise come from a
device Philox stream keyed by the seed and the device update counter, so a
captured graph draws fresh values on every replay.  ``update_from_batch``
injects a batch and noise instead (for parity checks).
"""

import json
import math
import warnings
from dataclasses import asdict, replace
from pathlib import Path

import numpy as np
import torch

from . import _native
from . import kernels as K
from .config import FlashSACConfig
from .networks import FlatStore, FusedOptimizer, Trunk

METRIC_KEYS = ("actor/loss", "actor/entropy", "actor/mean_action", "critic/loss", "critic/max_entropy_bonus",
               "temperature/loss", "temperature/value")
BATCH_KEYS = ("observation", "action", "reward", "terminated", "truncated", "next_observation", "discount")


def target_entropy(action_dim: int, sigma: float) -> float:
    """Temperature target: the differential entropy of an action_dim-dimensional Normal with standard
    deviation sigma per dimension, 0.5 A ln(2 pi e sigma^2) (robolearn/flashsac/agent.py:329)."""
    return 0.5 * action_dim * math.log(2.0 * math.pi * math.e * sigma**2)


def actor_shapes(obs, act, h, blocks):
    from collections import OrderedDict

    s = OrderedDict()
    s["embedder.norm.weight"] = (obs,)
    s["embedder.norm.bias"] = (obs,)
    s["embedder.w.w.weight"] = (h, obs)
    for i in range(blocks):
        s[f"encoder.{i}.w1.w.weight"] = (4 * h, h)
        s[f"encoder.{i}.w2.w.weight"] = (h, 4 * h)
        s[f"encoder.{i}.norm1.weight"] = (4 * h,)
        s[f"encoder.{i}.norm1.bias"] = (4 * h,)
        s[f"encoder.{i}.norm2.weight"] = (h,)
        s[f"encoder.{i}.norm2.bias"] = (h,)
    s["post_norm.weight"] = (h,)
    s["predictor.mean_w.w.weight"] = (act, h)
    s["predictor.mean_bias"] = (act,)
    s["predictor.std_w.w.weight"] = (act, h)
    s["predictor.std_bias"] = (act,)
    return s


def critic_shapes(inp, h, blocks, bins):
    from collections import OrderedDict

    s = OrderedDict()
    s["embedder.norm.weight"] = (2, inp)
    s["embedder.norm.bias"] = (2, inp)
    s["embedder.w.weight"] = (2, h, inp)
    for i in range(blocks):
        s[f"encoder.{i}.w1.weight"] = (2, 4 * h, h)
        s[f"encoder.{i}.w2.weight"] = (2, h, 4 * h)
        s[f"encoder.{i}.norm1.weight"] = (2, 4 * h)
        s[f"encoder.{i}.norm1.bias"] = (2, 4 * h)
        s[f"encoder.{i}.norm2.weight"] = (2, h)
        s[f"encoder.{i}.norm2.bias"] = (2, h)
    s["post_norm.weight"] = (2, h)
    s["predictor.w.weight"] = (2, bins, h)
    s["predictor.bias"] = (2, bins)
    return s


def running_shapes(prefix_widths, ensemble):
    from collections import OrderedDict

    s = OrderedDict()
    for name, width in prefix_widths:
        shape = (width,) if ensemble == 1 else (ensemble, width)
        s[name + ".running_mean"] = shape
        s[name + ".running_var"] = shape
    return s


class _Running:
    """Running BatchNorm statistics as named views of one flat buffer."""

    def __init__(self, shapes, device):
        self.store = FlatStore(shapes, device, adam=False, grads=False)
        self.views = self.store.params()
        for name, value in self.views.items():
            if name.endswith("running_var"):
                value.fill_(1.0)

    def __getitem__(self, name):
        return self.views[name]


class FlashSAC:
    """MI355X FlashSAC learner (drop-in for the reference learner interface).

    ``update`` performs one critic update; the first update and every
    ``actor_update_period`` thereafter also update the actor and temperature.
    ``cfg.use_amp`` selects bf16 operands for the dense-layer GEMMs; with it,
    ``bf16_activations`` (default True) also stores the BatchNorm inputs and the
    ReLU-BatchNorm gradients in bf16, the layout an autocast Linear hands its
    BatchNorm, and False keeps those activations fp32.
    """

    def __init__(self, observation_dim: int, action_dim: int, num_envs: int = 1, cfg: FlashSACConfig | None = None,
                 critic_observation_dim: int | None = None, *, optimized_linear_backward: bool = True,
                 dense_backend: str = "hip", fused_updates: bool = True, cuda_autotune: bool = False,
                 fresh_training_gradients: bool = False, bf16_activations: bool = True):
        cfg = cfg or FlashSACConfig()
        if min(observation_dim, action_dim, num_envs) < 1:
            raise ValueError("Observation, action and environment dimensions must be positive.")
        total_dim = critic_observation_dim or observation_dim
        if total_dim < observation_dim:
            raise ValueError("Critic observations must contain the actor observation prefix.")
        if cfg.temp_initial_value <= 0 or cfg.temp_target_sigma <= 0 or cfg.actor_noise_zeta_max < 1:
            raise ValueError("Temperature and exploration distribution parameters must be positive.")
        if not 0 <= cfg.critic_target_update_tau <= 1:
            raise ValueError("Target EMA tau must lie in [0, 1].")
        if cfg.learning_rate_warmup_step < 0 or cfg.learning_rate_warmup_step >= cfg.learning_rate_decay_step:
            raise ValueError("Learning-rate warmup must be nonnegative and shorter than decay.")
        if not 2 <= cfg.critic_num_bins <= 4096:
            raise ValueError("The categorical TD projection supports 2 to 4096 bins (the reference native limit).")
        if not torch.cuda.is_available():
            raise RuntimeError("FlashSAC on MI355X requires a visible GPU; there is no CPU fallback.")
        _native.load()
        self.cfg = self.config = replace(cfg, asymmetric_observation=critic_observation_dim is not None,
                                         temp_target_entropy=target_entropy(action_dim, cfg.temp_target_sigma))
        self.device = torch.device(cfg.device if str(cfg.device).startswith("cuda") else "cuda:0")
        self.observation_dim = observation_dim
        self.critic_observation_dim = total_dim
        self.action_dim = action_dim
        self.num_envs = num_envs
        self.batch_size = B = cfg.sample_batch_size
        # fp32 configurations form their products on the bf16 matrix cores from exact three-piece
        # splits (fp32-accurate, rl_gemm mode 2)
        self.mode = K.BF16 if cfg.use_amp else K.FP32_SPLIT
        self.compute_dtype = "bfloat16" if cfg.use_amp else "float32"
        self._update_step = 0
        self._graphs = {}
        self._prepared = False
        self.dense_backend = dense_backend
        self.fused_updates = fused_updates
        dev = self.device
        A, Oa, Oc = action_dim, observation_dim, total_dim
        I = Oc + A
        self.critic_in_dim = I
        ha, hc = cfg.actor_hidden_dim, cfg.critic_hidden_dim
        with torch.cuda.device(dev):
            # parameters (mean/std head rows contiguous so one GEMM computes both heads)
            groups = [["predictor.mean_w.w.weight", "predictor.std_w.w.weight"],
                      ["predictor.mean_bias", "predictor.std_bias"]]
            bf = self.mode == K.BF16
            self.actor = FlatStore(actor_shapes(Oa, A, ha, cfg.actor_num_blocks), dev, groups=groups, shadows=bf)
            self.critic = FlatStore(critic_shapes(I, hc, cfg.critic_num_blocks, cfg.critic_num_bins), dev,
                                    target=True, shadows=bf)
            self.log_temperature = torch.full((1,), math.log(cfg.temp_initial_value), device=dev)
            self.temperature = FlatStore({"log_temp": (1,)}, dev)
            self.temperature.param.zero_()
            self.temperature.view(self.temperature.param, "log_temp").copy_(self.log_temperature)
            self.log_temperature = self.temperature.view(self.temperature.param, "log_temp")
            actor_bn = [("embedder.norm", Oa)] + [
                (f"encoder.{i}.{n}", w) for i in range(cfg.actor_num_blocks) for n, w in (("norm1", 4 * ha), ("norm2", ha))]
            critic_bn = [("embedder.norm", I)] + [
                (f"encoder.{i}.{n}", w) for i in range(cfg.critic_num_blocks) for n, w in (("norm1", 4 * hc), ("norm2", hc))]
            self.actor_running = _Running(running_shapes(actor_bn, 1), dev)
            self.critic_running = _Running(running_shapes(critic_bn, 2), dev)
            self.target_running = _Running(running_shapes(critic_bn, 2), dev)
            self._init_parameters(cfg.seed)
            self.actor_p, self.actor_g = self.actor.params(), self.actor.grads()
            # GEMM weight operands: bf16 shadows in bf16 mode, the fp32 masters otherwise
            self.actor_w = self.actor.shadows() or self.actor_p
            heads = ["predictor.mean_w.w.weight", "predictor.std_w.w.weight"]
            head_bias = ["predictor.mean_bias", "predictor.std_bias"]
            self.head_w = self.actor.span(self.actor.param, heads, (2 * A, ha))
            self.head_w_op = self.actor.span(self.actor.shadow, heads, (2 * A, ha)) if bf else self.head_w
            self.head_b = self.actor.span(self.actor.param, head_bias, (2 * A,))
            self.head_dw = self.actor.span(self.actor.grad, heads, (2 * A, ha))
            self.head_db = self.actor.span(self.actor.grad, head_bias, (2 * A,))
            self.critic_p, self.critic_g = self.critic.params(), self.critic.grads()
            self.target_p = self.critic.targets()
            self.critic_w = self.critic.shadows() or self.critic_p
            self.target_w = self.critic.target_shadows() or self.target_p
            # transposed bf16 block weights: the input-gradient products read both operands K-contiguously
            self.actor.enable_transposed([f"encoder.{i}.w{j}.w.weight" for i in range(cfg.actor_num_blocks)
                                          for j in (1, 2)])
            self.critic.enable_transposed([f"encoder.{i}.w{j}.weight" for i in range(cfg.critic_num_blocks)
                                           for j in (1, 2)])
            self.actor.refresh_shadows()
            self.critic.refresh_shadows()
            # optimizers
            self.actor_optimizer = FusedOptimizer(self.actor, cfg)
            self.critic_optimizer = FusedOptimizer(self.critic, cfg, ema_tau=cfg.critic_target_update_tau)
            self.temperature_optimizer = FusedOptimizer(self.temperature, cfg, plain=True)
            # networks / activations
            self.actor_net = Trunk(ensemble=1, in_dim=Oa, hidden=ha, blocks=cfg.actor_num_blocks, max_rows=2 * B,
                                   device=dev, mode=self.mode, prefix_linear=".w.weight",
                                   bf16_activations=bf16_activations)
            self.critic_net = Trunk(ensemble=2, in_dim=I, hidden=hc, blocks=cfg.critic_num_blocks, max_rows=2 * B,
                                    device=dev, mode=self.mode, prefix_linear=".weight",
                                    bf16_activations=bf16_activations)
            self.bf16_activations = bf and bf16_activations
            self.workspace = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
            self.actor_net.workspace = self.critic_net.workspace = self.workspace
            z = lambda *s: torch.zeros(*s, device=dev)  # noqa: E731
            self.batch = {"observation": z(B, Oc), "action": z(B, A), "reward": z(B), "terminated": z(B),
                          "truncated": z(B), "next_observation": z(B, Oc), "discount": z(B)}
            self.indices = torch.zeros(B, dtype=torch.long, device=dev)
            self.reward_used = z(B)
            self.actor_in = z(2 * B, Oa)
            self.critic_in = z(2 * B, I)
            self.actor_head = z(2 * B, 2 * A)
            self.actor_dhead = z(2 * B, 2 * A)
            half = lambda *s: torch.zeros(*s, dtype=torch.bfloat16, device=dev) if bf else None  # noqa: E731
            self.actor_dhead_h = half(2 * B, 2 * A)
            self.actor_noise = z(2 * B, A)
            self.next_noise = z(B, A)
            self.actions_all = z(2 * B, A)
            self.log_probs_all = z(2 * B)
            self.dlog_probs = z(2 * B)
            self.next_log_probs = z(B)
            self.q = z(2, B)
            self.dq = z(2, B)
            self.dactions_bc = z(B, A)
            self.dactions_sum = z(B, A)
            self.critic_in_actor = z(B, I)
            self.critic_dx = z(2, B, I)
            self.logits = z(2, B, cfg.critic_num_bins)
            self.target_logits = z(2, B, cfg.critic_num_bins)
            self.dlogits = z(2, B, cfg.critic_num_bins)
            self.dlogits_h = half(2, B, cfg.critic_num_bins)
            self.loss_rows = z(2, B)
            self.entropy_rows = z(B)
            self.target_probabilities = z(B, cfg.critic_num_bins)
            self.q_next = z(2, B)
            self.alpha = z(1)
            self.temperature_grad_metrics = z(2)
            self.metrics_buffer = z(len(METRIC_KEYS))
            self.objective_partial = z(5 * ((2 * B + 255) // 256) + 1)
            self.bias_partial = z(2 * K.chunks(2 * B) * max(2 * A, cfg.critic_num_bins))
            self.support = torch.linspace(cfg.critic_min_v, cfg.critic_max_v, cfg.critic_num_bins,
                                          dtype=torch.float32).to(dev)
            self.update_counters = torch.zeros(3, dtype=torch.long, device=dev)
            # replay storage (device ring) and reward normalizer state
            self.capacity = cfg.buffer_max_length
            self.replay = None
            self.replay_counters = torch.zeros(3, dtype=torch.long, device=dev)  # additions, position, count
            self.pending = None
            self._host_additions = 0
            self._num_in_buffer_host = 0
            self._replay_position = 0
            # return statistics (reward_normalization.py:75-105): G_r per environment,
            # running max |G_r| and RunningMeanStd [mean, var, count]
            self.reward_returns = torch.zeros(num_envs, device=dev)
            self.reward_max = torch.zeros(1, device=dev)
            self.reward_running = torch.tensor([0.0, 1.0, 0.0], device=dev)
            self.gather_error = torch.zeros(1, dtype=torch.int32, device=dev)
            # exploration-noise repeats (agent.py:159-214): truncated zeta CDF, [count, length, refresh],
            # the held noise of the num_envs acting rows and the device draw counter
            lengths = torch.arange(1, cfg.actor_noise_zeta_max + 1, dtype=torch.float32)
            pmf = lengths ** (-cfg.actor_noise_zeta_mu)
            self.zeta_cdf = torch.cumsum(pmf / torch.sum(pmf), dim=0).to(dev)
            self.exploration_state = torch.tensor([0, 1, 0], dtype=torch.int32, device=dev)
            self.exploration_step = torch.zeros(1, dtype=torch.long, device=dev)
            self.exploration_noise = torch.zeros(num_envs, action_dim, device=dev)
            self._act_nets = {}
        self.metrics = {key: self.metrics_buffer[i: i + 1] for i, key in enumerate(METRIC_KEYS)}

    # ------------------------------------------------------------------
    # initialization and state
    # ------------------------------------------------------------------
    @torch.no_grad()
    def _init_parameters(self, seed: int):
        """Orthogonal unit-linear rows, identity BN/RMS, projection, target copy (agent.py:40-156)."""
        from .networks import projection_kind

        generator = torch.Generator().manual_seed(seed)
        for store in (self.actor, self.critic):
            host = {}
            for name, view in store.params().items():
                value = torch.zeros(view.shape)
                kind = projection_kind(name)
                if kind == 0:
                    for matrix in (value if value.dim() == 3 else [value]):
                        torch.nn.init.orthogonal_(matrix, gain=1, generator=generator)
                    value = torch.nn.functional.normalize(value, dim=-1, eps=1e-8)
                elif kind in (1, 2) and name.endswith("weight"):
                    value.fill_(1.0)
                host[name] = value
            for name, value in host.items():
                kind = projection_kind(name)
                if kind == 2 or (kind == 1 and name.endswith("weight")):
                    bias = host.get(name[: -len("weight")] + "bias") if kind == 1 else None
                    sq = value * value + (bias * bias if bias is not None else 0.0)
                    factor = math.sqrt(value.shape[-1]) * torch.rsqrt(sq.sum(-1, keepdim=True) + 1e-8)
                    value.mul_(factor)
                    if bias is not None:
                        bias.mul_(factor)
            for name, view in store.params().items():
                view.copy_(host[name])
        self.critic.target.copy_(self.critic.param)

    def parameters(self) -> list:
        """Learnable tensors (target critic excluded)."""
        return list(self.actor.params().values()) + list(self.critic.params().values()) + [self.log_temperature]

    def _state_arrays(self) -> dict:
        arrays = {}
        for name, view in self.actor.params().items():
            arrays[f"actor.{name}"] = view
        for name, view in self.actor_running.views.items():
            arrays[f"actor.{name}"] = view
        for name, view in self.critic.params().items():
            arrays[f"critic.{name}"] = view
        for name, view in self.critic_running.views.items():
            arrays[f"critic.{name}"] = view
        for name, view in self.critic.targets().items():
            arrays[f"target_critic.{name}"] = view
        for name, view in self.target_running.views.items():
            arrays[f"target_critic.{name}"] = view
        for label, store, optimizer in (("actor", self.actor, self.actor_optimizer),
                                        ("critic", self.critic, self.critic_optimizer),
                                        ("temperature", self.temperature, self.temperature_optimizer)):
            m1, m2 = store.moments()
            for i, name in enumerate(store.shapes):
                arrays[f"optimizer.{label}.m1.{i}"] = m1[name]
                arrays[f"optimizer.{label}.m2.{i}"] = m2[name]
            arrays[f"optimizer.{label}.timestep"] = optimizer.timestep
            arrays[f"optimizer.{label}.lr"] = optimizer.lr
        arrays["log_temperature"] = self.log_temperature
        arrays["update_counters"] = self.update_counters
        arrays["normalizer.maximum"] = self.reward_max
        arrays["normalizer.running"] = self.reward_running
        return arrays

    def state_dict(self, include_replay: bool = True) -> dict:
        """Snapshot weights, BN buffers, Adam, counters (and replay storage) as NumPy arrays."""
        torch.cuda.synchronize(self.device)
        state = {key: value.detach().cpu().numpy().copy() for key, value in self._state_arrays().items()}
        state["replay.num_in_buffer"] = np.array([self._num_in_buffer_host], dtype=np.int64)
        state["replay.position"] = np.array([self._replay_position], dtype=np.int64)
        state["replay.counters"] = self.replay_counters.cpu().numpy().copy()
        state["normalizer.returns"] = self.reward_returns.cpu().numpy().copy()
        if include_replay and self.replay is not None:
            n = self._num_in_buffer_host
            for key, value in self.replay.items():
                state[f"replay.{key}"] = value[:n].cpu().numpy()
            for key, value in self.pending.items():
                state[f"replay.pending.{key}"] = value.cpu().numpy()
        state["replay_storage_included"] = np.array([include_replay and self.replay is not None], dtype=np.bool_)
        return state

    @torch.no_grad()
    def load_state_dict(self, state: dict) -> None:
        """Restore arrays in place (captured graphs keep valid pointers)."""
        arrays = self._state_arrays()
        for key, array in arrays.items():
            if key not in state or tuple(np.asarray(state[key]).shape) != tuple(array.shape):
                raise ValueError(f"Checkpoint array {key} is missing or has the wrong shape.")
        for key, array in arrays.items():
            array.copy_(torch.as_tensor(np.asarray(state[key])).to(array.dtype))
        returns = state.get("normalizer.returns")
        if returns is not None and tuple(np.asarray(returns).shape) == tuple(self.reward_returns.shape):
            self.reward_returns.copy_(torch.as_tensor(np.asarray(returns)))
        else:
            self.reward_returns.zero_()
        self.actor.refresh_shadows()
        self.critic.refresh_shadows()
        if bool(np.asarray(state.get("replay_storage_included", [False]))[0]):
            n = int(np.asarray(state["replay.num_in_buffer"])[0])
            self.load_replay({key: state[f"replay.{key}"] for key in BATCH_KEYS}, count=n,
                             position=int(np.asarray(state["replay.position"])[0]))
            staged = [f"replay.pending.{key}" for key in self.pending]
            if all(key in state for key in staged):
                shapes_match = all(tuple(np.asarray(state[f"replay.pending.{key}"]).shape) == tuple(value.shape)
                                   for key, value in self.pending.items())
                if shapes_match:  # same environment count: continue the n-step staging exactly
                    for key, value in self.pending.items():
                        value.copy_(torch.as_tensor(np.asarray(state[f"replay.pending.{key}"])))
                    additions = int(np.asarray(state["replay.counters"])[0])
                    self.replay_counters[0] = additions
                    self._host_additions = additions
        self._update_step = int(np.asarray(state["update_counters"])[0])

    default_checkpoint_format = "native"

    def save(self, path, *, include_replay: bool = False, format: str | None = None) -> None:
        """Checkpoint directory: "native" (config.json + agent.npz, optional replay), "torch", the
        reference's Torch layout (robolearn/flashsac/agent.py:529-551), or "warp", the reference Warp
        learner's robolearn-warp-flashsac-v1 arrays (robolearn/warp/flashsac.py:1169-1195); each is
        readable by the matching reference load()."""
        format = format or self.default_checkpoint_format
        if format == "torch":
            from . import torch_checkpoint

            torch_checkpoint.save(self, path)
            if include_replay:
                torch_checkpoint.save_replay_buffer(self, path)
            return
        if format == "warp":
            from . import warp_checkpoint

            warp_checkpoint.save(self, path, include_replay=include_replay)
            return
        if format != "native":
            raise ValueError("format must be 'native', 'torch' or 'warp'.")
        directory = Path(path)
        directory.mkdir(parents=True, exist_ok=True)
        metadata = {
            "format": "robolearn-mi355x-flashsac-v1",
            "precision": self.compute_dtype,
            "observation_dim": self.observation_dim,
            "action_dim": self.action_dim,
            "critic_observation_dim": self.critic_observation_dim if self.cfg.asymmetric_observation else None,
            "num_envs": self.num_envs,
            "config": asdict(self.cfg),
            "replay_included": include_replay,
        }
        state = self.state_dict(include_replay=include_replay)
        (directory / "config.json").write_text(json.dumps(metadata, indent=2) + "\n")
        with (directory / "agent.npz").open("wb") as stream:
            np.savez(stream, **state)

    def load(self, path) -> None:
        """Load a native checkpoint, a Warp-format one (its config.json format tag) or a Torch-layout
        one (actor.pt beside config.json), in place: captured graphs keep their buffers."""
        directory = Path(path)
        if (directory / "actor.pt").exists():
            from . import torch_checkpoint

            torch_checkpoint.load(self, directory)
            return
        metadata = json.loads((directory / "config.json").read_text())
        if metadata.get("format") == "robolearn-warp-flashsac-v1":
            from . import warp_checkpoint

            warp_checkpoint.load(self, directory)
            return
        if metadata.get("format") != "robolearn-mi355x-flashsac-v1":
            raise ValueError("Unrecognized FlashSAC checkpoint format.")
        if metadata["observation_dim"] != self.observation_dim or metadata["action_dim"] != self.action_dim:
            raise ValueError("Checkpoint observation/action dimensions differ from this agent.")
        with np.load(directory / "agent.npz", allow_pickle=False) as archive:
            state = dict(archive)
        current = None
        if not self.cfg.load_optimizer or not self.cfg.load_reward_normalizer:
            current = self.state_dict(include_replay=False)
        if not self.cfg.load_optimizer:
            for key in current:
                if key.startswith("optimizer.") or key == "update_counters":
                    state[key] = current[key]
        if not self.cfg.load_reward_normalizer:
            for key in current:
                if key.startswith("normalizer."):
                    state[key] = current[key]
        elif self.cfg.normalize_reward:
            # a loaded normalizer restarts its per-environment returns (agent.py:570-572)
            state.pop("normalizer.returns", None)
        self.load_state_dict(state)

    def save_replay_buffer(self, path) -> None:
        """replay_buffer.pt in the reference layout (agent.py:553-554, replay.py:196-216)."""
        from . import torch_checkpoint

        torch_checkpoint.save_replay_buffer(self, path)

    def load_replay_buffer(self, path) -> None:
        """Restore replay_buffer.pt (agent.py:575-576, replay.py:218-240)."""
        from . import torch_checkpoint

        self._ensure_replay()
        torch_checkpoint.load_replay_buffer(self, path)

    # ------------------------------------------------------------------
    # replay
    # ------------------------------------------------------------------
    def _ensure_replay(self):
        if self.replay is None:
            c, dev = self.capacity, self.device
            o, a = self.critic_observation_dim, self.action_dim
            self.replay = {
                "observation": torch.zeros(c, o, device=dev),
                "action": torch.zeros(c, a, device=dev),
                "reward": torch.zeros(c, device=dev),
                "terminated": torch.zeros(c, device=dev),
                "truncated": torch.zeros(c, device=dev),
                "next_observation": torch.zeros(c, o, device=dev),
                "discount": torch.zeros(c, device=dev),
            }
            # n-step staging ring (robolearn/warp/_flash_replay.py:200-209): slot = additions % n_step
            n, e = self.cfg.n_step, self.num_envs
            self.pending = {
                "observation": torch.zeros(n, e, o, device=dev),
                "action": torch.zeros(n, e, a, device=dev),
                "next_observation": torch.zeros(n, e, o, device=dev),
                "scalars": torch.zeros(n, e, 3, device=dev),  # reward, terminated, truncated
            }

    @torch.no_grad()
    def load_replay(self, data: dict, *, count: int | None = None, position: int | None = None) -> None:
        """Fill replay storage directly (synthetic or restored contents; n-step already applied)."""
        self._ensure_replay()
        n = int(count if count is not None else len(data["reward"]))
        if n > self.capacity:
            raise ValueError("Replay contents exceed the configured capacity.")
        for key in BATCH_KEYS:
            value = data[key] if key in data else np.zeros((n,), dtype=np.float32)
            value = value if torch.is_tensor(value) else torch.as_tensor(np.asarray(value))
            self.replay[key][:n].copy_(value[:n].to(device=self.device, dtype=torch.float32).reshape(
                self.replay[key][:n].shape))
        self._num_in_buffer_host = n
        self._replay_position = (position if position is not None else n) % self.capacity
        # the n-step staging restarts empty, as after TorchUniformBuffer.load (replay.py:238-240)
        self._host_additions = 0
        self.replay_counters.copy_(torch.tensor([0, self._replay_position, n], dtype=torch.long))

    @torch.no_grad()
    def observe(self, observations, actions, rewards, terminated, truncated, next_observations) -> None:
        """Store one vector step of pre-reset transitions (agent.py:587-598 -> process_transition :457-468).

        The step is staged on the device and, once n_step steps are staged, the
        oldest is committed with its n-step return (replay.py:107-174); with
        reward normalization the return statistics advance too
        (reward_normalization.py:108-122).  Both run as HIP kernels on the
        current stream; no host read."""
        self._ensure_replay()
        e, o, a = self.num_envs, self.critic_observation_dim, self.action_dim
        fields = []
        for value, shape in ((observations, (e, o)), (actions, (e, a)), (rewards, (e,)), (terminated, (e,)),
                             (truncated, (e,)), (next_observations, (e, o))):
            tensor = torch.as_tensor(value, device=self.device)
            if tensor.numel() != math.prod(shape):
                raise ValueError(f"observe() expects {e} environments with fields shaped {shape}.")
            fields.append(tensor.to(torch.float32).reshape(shape).contiguous())
        obs, act, rew, term, trunc, next_obs = fields
        r, p = self.replay, self.pending
        _native.call("rl_replay_ingest", e, o, a, self.cfg.n_step, self.capacity, float(self.cfg.gamma),
                     obs.data_ptr(), act.data_ptr(), rew.data_ptr(), term.data_ptr(), trunc.data_ptr(),
                     next_obs.data_ptr(), p["observation"].data_ptr(), p["action"].data_ptr(),
                     p["next_observation"].data_ptr(), p["scalars"].data_ptr(), r["observation"].data_ptr(),
                     r["action"].data_ptr(), r["reward"].data_ptr(), r["terminated"].data_ptr(),
                     r["truncated"].data_ptr(), r["next_observation"].data_ptr(), r["discount"].data_ptr(),
                     self.replay_counters.data_ptr(), K.stream())
        if self.cfg.normalize_reward:
            _native.call("rl_reward_stats_update", e, float(self.cfg.gamma), rew.data_ptr(), term.data_ptr(),
                         trunc.data_ptr(), self.reward_returns.data_ptr(), self.reward_max.data_ptr(),
                         self.reward_running.data_ptr(), K.stream())
        if self._host_additions >= self.cfg.n_step - 1:
            self._replay_position = (self._replay_position + e) % self.capacity
            self._num_in_buffer_host = min(self._num_in_buffer_host + e, self.capacity)
        self._host_additions += 1

    def process_transition(self, transition: dict) -> None:
        """Reference-named entry (agent.py:457-468): a transition dict with the observe() fields."""
        self.observe(transition["observation"], transition["action"], transition["reward"],
                     transition["terminated"], transition["truncated"], transition["next_observation"])

    @property
    def ready(self) -> bool:
        return self.replay is not None and self._num_in_buffer_host >= self.cfg.buffer_min_length

    def can_start_training(self) -> bool:
        return self.ready

    # ------------------------------------------------------------------
    # inference
    # ------------------------------------------------------------------
    def _act_net(self, n: int):
        """fp32 eval-mode actor for n acting rows (the reference acts in fp32 under AMP too,
        robolearn/warp/flashsac.py:571-575), with its own activations and output buffers."""
        if n not in self._act_nets:
            cfg = self.cfg
            net = Trunk(ensemble=1, in_dim=self.observation_dim, hidden=cfg.actor_hidden_dim,
                        blocks=cfg.actor_num_blocks, max_rows=n, device=self.device, mode=K.FP32_SPLIT,
                        prefix_linear=".w.weight")
            head = torch.empty(n, 2 * self.action_dim, device=self.device)
            actions = torch.empty(n, self.action_dim, device=self.device)
            self._act_nets[n] = (net, head, actions)
        return self._act_nets[n]

    @torch.no_grad()
    def act(self, observations: torch.Tensor, training: bool = True) -> torch.Tensor:
        """Normalized actions from the eval-mode actor (agent.py:583-585 -> sample_actions :414-455).

        Deterministic inference returns tanh(mean) and leaves the exploration
        state alone.  Training acts over exactly num_envs rows and holds one
        Gaussian noise draw for a truncated-zeta number of calls
        (agent.py:180-214); the repeat state and the draws stay on the device."""
        obs = torch.as_tensor(observations, device=self.device, dtype=torch.float32)
        if obs.dim() != 2 or obs.shape[1] < self.observation_dim:
            raise ValueError("act() expects [rows, obs] observations with the actor's observation prefix.")
        obs = obs[:, : self.observation_dim].contiguous()
        n = obs.shape[0]
        if training and n != self.num_envs:
            raise ValueError("Training action batches must match num_envs.")
        A = self.action_dim
        net, head, actions = self._act_net(n)
        p = self.actor_p
        with torch.cuda.device(self.device):
            net.forward(p, p, self.actor_running, obs, rows=n, x_stride=0, training=False)
            net.post_norm(p, rows=n, row0=0, count=n)
            K.linear_forward(net.z, self.head_w, head, rows=n, in_dim=net.h, out_dim=2 * A, bias=self.head_b,
                             mode=K.FP32_SPLIT)
            noise = None
            if training:
                _native.call("rl_exploration_noise", self.cfg.seed * 7919 + 37, self.exploration_step.data_ptr(),
                             self.zeta_cdf.data_ptr(), self.cfg.actor_noise_zeta_max,
                             self.exploration_state.data_ptr(), self.exploration_noise.data_ptr(), n * A, None, None,
                             K.stream())
                noise = self.exploration_noise
            K.tanh_gaussian_forward(head, noise, actions, None, rows=n, action_dim=A, deterministic=not training)
            return actions.clone()

    def sample_actions(self, interaction_step: int, prev_transition: dict, training: bool) -> torch.Tensor:
        """Reference-named entry (agent.py:414-455): acts on prev_transition["next_observation"]."""
        return self.act(prev_transition["next_observation"], training=training)

    # ------------------------------------------------------------------
    # the update
    # ------------------------------------------------------------------
    def _pack_inputs(self):
        B, Oa, Oc, A, I = self.batch_size, self.observation_dim, self.critic_observation_dim, self.action_dim, \
            self.critic_in_dim
        b = self.batch
        K.concat_columns(self.actor_in, Oa, B, b["observation"], Oc, Oa)
        K.concat_columns(self.actor_in[B:], Oa, B, b["next_observation"], Oc, Oa)
        K.concat_columns(self.critic_in, I, B, b["observation"], Oc, Oc, b["action"], A, A)
        K.concat_columns(self.critic_in[B:], I, B, b["next_observation"], Oc, Oc)

    def _sample(self):
        B = self.batch_size
        K.sample_indices(self.indices, seed=self.cfg.seed * 7919 + 1, count=self.replay_counters[2:3],
                         counter=self.update_counters, stream_id=1)
        b, r = self.batch, self.replay
        _native.call("rl_replay_gather", self.indices.data_ptr(), B, self.capacity, self.critic_observation_dim,
                     self.action_dim, r["observation"].data_ptr(), r["next_observation"].data_ptr(),
                     r["action"].data_ptr(), r["reward"].data_ptr(), r["terminated"].data_ptr(),
                     r["truncated"].data_ptr(), r["discount"].data_ptr(), b["observation"].data_ptr(),
                     b["next_observation"].data_ptr(), b["action"].data_ptr(), b["reward"].data_ptr(),
                     b["terminated"].data_ptr(), b["truncated"].data_ptr(), b["discount"].data_ptr(),
                     self.gather_error.data_ptr(), K.stream())

    def _actor_phase(self, apply_optimizer: bool):
        cfg, B, A, I, Oc = self.cfg, self.batch_size, self.action_dim, self.critic_in_dim, self.critic_observation_dim
        bins = cfg.critic_num_bins
        net, p, g = self.actor_net, self.actor_p, self.actor_g
        cn, cp = self.critic_net, self.critic_p
        _native.call("rl_exp_scalar", self.log_temperature.data_ptr(), self.alpha.data_ptr(), K.stream())
        # actor forward on [obs; next_obs] in training mode (BN statistics over 2B rows)
        net.forward(p, self.actor_w, self.actor_running, self.actor_in, rows=2 * B, x_stride=0, training=True)
        net.post_norm(p, rows=2 * B, row0=0, count=2 * B)
        K.linear_forward(net.z_op, self.head_w_op, self.actor_head, rows=2 * B, in_dim=net.h, out_dim=2 * A,
                         bias=self.head_b, mode=self.mode, workspace=self.workspace)
        K.tanh_gaussian_forward(self.actor_head, self.actor_noise, self.actions_all, self.log_probs_all,
                                rows=2 * B, action_dim=A)
        # frozen critic in eval mode on (obs, first-half actions)
        K.concat_columns(self.critic_in_actor, I, B, self.batch["observation"], Oc, Oc, self.actions_all, A, A)
        cn.forward(cp, self.critic_w, self.critic_running, self.critic_in_actor, rows=B, x_stride=0, training=False)
        cn.post_norm(cp, rows=B, row0=0, count=B)
        K.linear_forward(cn.z_op, self.critic_w["predictor.w.weight"], self.logits, rows=B, in_dim=cn.h,
                         out_dim=bins, ensemble=2, x_stride=B * cn.h, bias=cp["predictor.bias"], mode=self.mode,
                         workspace=self.workspace)
        K.categorical_head_forward(self.logits, self.support, self.q, rows=B, bins=bins, ensemble=2)
        _native.call("rl_actor_objective", self.q.data_ptr(), self.q[1].data_ptr(), self.log_probs_all.data_ptr(),
                     self.actions_all.data_ptr(), A, self.batch["action"].data_ptr(), self.alpha.data_ptr(),
                     float(cfg.actor_bc_alpha), B, 2 * B, A, self.metrics_buffer.data_ptr(),
                     self.dlog_probs.data_ptr(), self.dq.data_ptr(), self.dq[1].data_ptr(),
                     self.dactions_bc.data_ptr() if cfg.actor_bc_alpha > 0 else None,
                     self.objective_partial.data_ptr(), K.stream())
        # critic backward to the action inputs (parameters frozen, BN in eval mode)
        bf = self.mode == K.BF16
        K.categorical_head_backward_q(self.logits, self.support, self.dq, None if bf else self.dlogits, rows=B,
                                      bins=bins, ensemble=2, dlogits_bf16=self.dlogits_h)
        K.linear_backward_input(self.dlogits_h if bf else self.dlogits, self.critic_w["predictor.w.weight"], cn.dz,
                                rows=B, in_dim=cn.h, out_dim=bins, ensemble=2, mode=self.mode)
        cn.post_norm_backward(cp, None, rows=B, row0=0, count=B)
        cn.backward(cp, self.critic_w, self.critic_running, None, self.critic_in_actor, rows=B, x_stride=0,
                    wt=self.critic.transposed,
                    training=False, workspace=self.workspace, input_grad=self.critic_dx)
        _native.call("rl_add", self.critic_dx[0].data_ptr(), self.critic_dx[1].data_ptr(), B * I, K.stream())
        if cfg.actor_bc_alpha > 0:
            K.concat_columns(self.dactions_sum, A, B, self.critic_dx[0].view(-1)[Oc:], I, A)
            _native.call("rl_add", self.dactions_sum.data_ptr(), self.dactions_bc.data_ptr(), B * A, K.stream())
            dact, ld = self.dactions_sum, A
        else:
            dact, ld = self.critic_dx[0].view(-1)[Oc:], I
        K.tanh_gaussian_backward(self.actor_head, self.actor_noise, dact, self.dlog_probs, self.actor_dhead,
                                 rows=2 * B, action_dim=A, grad_rows=B, ld_dactions=ld, dhead_bf16=self.actor_dhead_h)
        # actor backward
        dhead = self.actor_dhead_h if bf else self.actor_dhead
        K.linear_backward_weight(dhead, net.z_op, self.head_dw, rows=2 * B, in_dim=net.h, out_dim=2 * A,
                                 mode=self.mode, workspace=self.workspace)
        K.bias_grad(self.actor_dhead, self.head_db, self.bias_partial, rows=2 * B, channels=2 * A)
        K.linear_backward_input(dhead, self.head_w_op, net.dz, rows=2 * B, in_dim=net.h, out_dim=2 * A,
                                mode=self.mode)
        net.post_norm_backward(p, g, rows=2 * B, row0=0, count=2 * B)
        net.backward(p, self.actor_w, self.actor_running, g, self.actor_in, rows=2 * B, x_stride=0, training=True,
                     wt=self.actor.transposed,
                     workspace=self.workspace)
        if apply_optimizer:
            self.actor_optimizer.step()

    def _temperature_phase(self, apply_optimizer: bool):
        # temperature loss and d/dlog_temp (updates.py:297-326); metrics 5 (loss), 6 (value)
        _native.call("rl_temperature_objective", self.log_temperature.data_ptr(), self.metrics_buffer[1:].data_ptr(),
                     float(self.cfg.temp_target_entropy), self.temperature.grad.data_ptr(),
                     self.metrics_buffer[5:].data_ptr(), K.stream())
        if apply_optimizer:
            self.temperature_optimizer.step()

    def _critic_phase(self, apply_optimizer: bool):
        cfg, B, A, I, Oc = self.cfg, self.batch_size, self.action_dim, self.critic_in_dim, self.critic_observation_dim
        net, p = self.actor_net, self.actor_p
        cn, cp, cg = self.critic_net, self.critic_p, self.critic_g
        bins = cfg.critic_num_bins
        bf = self.mode == K.BF16
        # next actions from the updated actor in eval mode
        net.forward(p, self.actor_w, self.actor_running, self.actor_in[B:], rows=B, x_stride=0, training=False)
        net.post_norm(p, rows=B, row0=0, count=B)
        K.linear_forward(net.z_op, self.head_w_op, self.actor_head, rows=B, in_dim=net.h, out_dim=2 * A,
                         bias=self.head_b, mode=self.mode, workspace=self.workspace)
        K.tanh_gaussian_forward(self.actor_head, self.next_noise, self.critic_in[B:].view(-1)[Oc:],
                                self.next_log_probs, rows=B, action_dim=A, ld_actions=I)
        _native.call("rl_exp_scalar", self.log_temperature.data_ptr(), self.alpha.data_ptr(), K.stream())
        # target critic, training-mode BN over 2B rows; head only on the next-observation half
        cn.forward(self.target_p, self.target_w, self.target_running, self.critic_in, rows=2 * B, x_stride=0,
                   training=True)
        cn.post_norm(self.target_p, rows=2 * B, row0=B, count=B)
        K.linear_forward(cn.z_op.view(-1)[B * cn.h:], self.target_w["predictor.w.weight"], self.target_logits,
                         rows=B, in_dim=cn.h, out_dim=bins, ensemble=2, x_stride=2 * B * cn.h,
                         bias=self.target_p["predictor.bias"], mode=self.mode, workspace=self.workspace)
        # online critic, training mode; head on the current-observation half
        cn.forward(cp, self.critic_w, self.critic_running, self.critic_in, rows=2 * B, x_stride=0, training=True)
        cn.post_norm(cp, rows=2 * B, row0=0, count=B)
        K.linear_forward(cn.z_op, self.critic_w["predictor.w.weight"], self.logits, rows=B, in_dim=cn.h,
                         out_dim=bins, ensemble=2, x_stride=2 * B * cn.h, bias=cp["predictor.bias"], mode=self.mode,
                         workspace=self.workspace)
        K.td_cross_entropy(self.target_logits, None, B, self.logits, None, B, self.support, self.reward_used,
                           self.batch["terminated"], self.batch["discount"], self.next_log_probs, self.alpha,
                           min_v=cfg.critic_min_v, max_v=cfg.critic_max_v, batch=B, bins=bins, scale=1.0 / (2 * B),
                           dlogits=self.dlogits, loss_rows=self.loss_rows, entropy_rows=self.entropy_rows,
                           target_out=self.target_probabilities, q_next=self.q_next, dlogits_bf16=self.dlogits_h)
        K.reduce_sum(self.loss_rows, self.metrics_buffer[3:], scale=1.0 / (2 * B))
        K.reduce_max(self.entropy_rows, self.metrics_buffer[4:])
        # critic backward
        dlogits = self.dlogits_h if bf else self.dlogits
        K.linear_backward_weight(dlogits, cn.z_op, cg["predictor.w.weight"], rows=B, in_dim=cn.h, out_dim=bins,
                                 ensemble=2, x_stride=2 * B * cn.h, mode=self.mode, workspace=self.workspace)
        K.bias_grad(self.dlogits, cg["predictor.bias"], self.bias_partial, rows=B, channels=bins, ensemble=2)
        K.gemm(dlogits, self.critic_w["predictor.w.weight"], cn.dz, m=B, n=cn.h, k=bins, batch=2, a_kcontig=True,
               b_kcontig=False, lda=bins, ldb=cn.h, ldd=cn.h, stride_a=B * bins, stride_b=bins * cn.h,
               stride_d=2 * B * cn.h, mode=self.mode)
        cn.post_norm_backward(cp, cg, rows=2 * B, row0=0, count=B)
        cn.backward(cp, self.critic_w, self.critic_running, cg, self.critic_in, rows=2 * B, x_stride=0, training=True,
                    wt=self.critic.transposed,
                    workspace=self.workspace)
        if apply_optimizer:
            self.critic_optimizer.step()

    def launch_update(self, do_actor_update: bool = True, *, sample: bool = True, randomize_noise: bool = True,
                      apply_optimizer: bool = True, normalize_reward: bool = True) -> None:
        """Enqueue one static learning phase; no host reads, graph-capturable."""
        B, A = self.batch_size, self.action_dim
        seed = self.cfg.seed
        if sample:
            self._sample()
        self._pack_inputs()
        if normalize_reward and self.cfg.normalize_reward:
            self.reward_used.copy_(self.batch["reward"])
            _native.call("rl_scale_rewards", self.reward_used.data_ptr(), B, self.reward_running[1:2].data_ptr(),
                         self.reward_max.data_ptr(), float(self.cfg.normalized_G_max), 1e-8, K.stream())
        else:
            self.reward_used.copy_(self.batch["reward"])
        if do_actor_update:
            if randomize_noise:
                K.philox_normal(self.actor_noise, seed=seed * 7919 + 11, counter=self.update_counters, stream_id=11)
            self._actor_phase(apply_optimizer)
            self._temperature_phase(apply_optimizer)
        if randomize_noise:
            K.philox_normal(self.next_noise, seed=seed * 7919 + 23, counter=self.update_counters, stream_id=23)
        self._critic_phase(apply_optimizer)
        if apply_optimizer:
            _native.call("rl_advance_counters", self.update_counters.data_ptr(), int(do_actor_update), K.stream())

    def update_from_batch(self, batch: dict, *, actor_noise=None, next_noise=None, do_actor_update: bool | None = None,
                          apply_optimizer: bool = True, normalize_reward: bool = False,
                          tensor_metrics: bool = True) -> dict:
        """Run one update on an explicit batch and (optionally) prescribed noise."""
        with torch.cuda.device(self.device):
            for key, destination in self.batch.items():
                value = batch.get(key)
                if value is None:
                    if key == "truncated":
                        destination.zero_()
                        continue
                    raise ValueError(f"Batch field {key} is missing.")
                value = torch.as_tensor(np.asarray(value) if not torch.is_tensor(value) else value)
                if tuple(value.shape) != tuple(destination.shape):
                    raise ValueError(f"Shape of {key} differs from {tuple(destination.shape)}.")
                destination.copy_(value.to(torch.float32))
            prescribed = actor_noise is not None or next_noise is not None
            if prescribed and (actor_noise is None or next_noise is None):
                raise ValueError("Supply both actor_noise and next_noise for fixed-noise diagnostics.")
            if prescribed:
                self.actor_noise.copy_(torch.as_tensor(actor_noise).to(torch.float32))
                self.next_noise.copy_(torch.as_tensor(next_noise).to(torch.float32))
            actor_phase = (self._update_step % self.cfg.actor_update_period == 0
                           if do_actor_update is None else do_actor_update)
            self.launch_update(actor_phase, sample=False, randomize_noise=not prescribed,
                               apply_optimizer=apply_optimizer, normalize_reward=normalize_reward)
            if apply_optimizer:
                self._update_step += 1
            return self._metrics(actor_phase, tensor_metrics)

    def prepare(self, *, capture: bool = False) -> None:
        """Warm every kernel on both phases without changing training state."""
        if not self._prepared:
            if self.replay is None:
                raise RuntimeError("Fill the replay buffer (load_replay/observe) before preparing updates.")
            state = self.state_dict(include_replay=False)
            try:
                for phase in (True, False):
                    self.launch_update(phase)
                torch.cuda.synchronize(self.device)
            finally:
                self.load_state_dict(state)
            self._prepared = True
        if capture:
            self.capture_update()

    warmup = prepare

    def capture_update(self) -> None:
        """Capture the actor+critic and critic-only phases as HIP graphs."""
        self.prepare(capture=False)
        for phase in (True, False):
            if phase not in self._graphs:
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph):
                    self.launch_update(phase)
                self._graphs[phase] = graph

    def _pair_phases(self) -> tuple:
        period = self.cfg.actor_update_period
        return tuple((self._update_step + i) % period == 0 for i in range(2))

    def capture_pair(self) -> "torch.cuda.CUDAGraph":
        """One graph holding the next two updates (update-to-data 2), with the actor phases that the
        current update step gives them: an actor-phase update then a critic-only update when the step
        is even and actor_update_period is 2.  Replay it through ``update_pair``, which keeps the host
        update step in line with the device counters."""
        self.prepare(capture=False)
        phases = self._pair_phases()
        key = ("pair",) + phases
        if key not in self._graphs:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                for phase in phases:
                    self.launch_update(phase)
            self._graphs[key] = graph
        return self._graphs[key]

    def update_pair(self, *, tensor_metrics: bool = False) -> dict:
        """Two updates in one graph replay (the update-to-data-2 step of robolearn/warp/flashsac.py:1033-1048
        called twice).  The metrics are those of the second update plus, when only the first was an actor
        phase, the first update's actor and temperature metrics."""
        if not self.ready:
            raise RuntimeError("Replay has not reached buffer_min_length.")
        phases = self._pair_phases()
        with torch.cuda.device(self.device):
            self.capture_pair().replay()
        self._update_step += 2
        return self._metrics(any(phases), tensor_metrics)

    def update(self, *, tensor_metrics: bool = False, capture: bool = True) -> dict:
        if not self.ready:
            raise RuntimeError("Replay has not reached buffer_min_length.")
        actor_phase = self._update_step % self.cfg.actor_update_period == 0
        with torch.cuda.device(self.device):
            if capture:
                self.capture_update()
                self._graphs[actor_phase].replay()
            else:
                self.launch_update(actor_phase)
        self._update_step += 1
        return self._metrics(actor_phase, tensor_metrics)

    def _metrics(self, actor_phase: bool, tensor_metrics: bool) -> dict:
        values = {key: value for key, value in self.metrics.items() if actor_phase or key.startswith("critic/")}
        if tensor_metrics:
            return values
        host = self.metrics_buffer.cpu().numpy()
        return {key: float(host[METRIC_KEYS.index(key)]) for key in values}

    def get_metrics(self) -> dict:
        result = self._metrics(True, False)
        result.update(actor_optimizer_steps=float(self.actor_optimizer.timestep.item()),
                      critic_optimizer_steps=float(self.critic_optimizer.timestep.item()),
                      temperature_optimizer_steps=float(self.temperature_optimizer.timestep.item()))
        return result


class WarpFlashSAC(FlashSAC):
    """The reference's WarpFlashSAC entry point (robolearn/warp/flashsac.py:340-353): the same
    learner, whose save() writes the Warp learner's robolearn-warp-flashsac-v1 checkpoint."""

    default_checkpoint_format = "warp"
