"""CPU restatement of one FlashSAC gradient update (TEST INFRASTRUCTURE ONLY).

Follows the reference Torch learner file by file:
  networks         robolearn/flashsac/layers.py:15-303, networks.py:23-119
  update order     robolearn/flashsac/agent.py:217-281 (actor -> temperature ->
                   critic -> target EMA), agent.py:473-527 (phase from the
                   update counter, actor_update_period)
  losses           robolearn/flashsac/updates.py:19-326
  optimizer        torch.optim.Adam (agent.py:64-65, 92-96, 133-137) with
                   LambdaLR over warmup_cosine_decay_scheduler (scheduler.py:43-65)
  projection/EMA   robolearn/flashsac/_utils/network.py:55-90
  log-det term     robolearn/flashsac/_utils/distribution.py:12-19
  replay sample    robolearn/flashsac/replay.py:179-194 (indices injected)

Random draws (replay indices, the reparameterization noise of
``Normal.rsample``) are injected, as the reference's own parity tools do
(examples/diagnose_warp_flashsac.py:311-329).  Initial weights are injected or
produced by ``init_state`` (orthogonal + projection, layers.py:17-19, 178-179,
agent.py:151-154).

Parity pinning (see tests/test_oracle.py and tests/golden/):
  * actor/critic forward (train and eval BN, running statistics), head
    gradients, projection, EMA and the LR schedule are pinned against golden
    vectors written from the reference modules themselves
    (tests/golden/make_golden.py imports layers.py, networks.py and
    _utils/{network,scheduler,distribution}.py);
  * the categorical TD projection is pinned by closed forms (unit mass,
    non-negativity, exact grid points, clamping to the end bins);
  * the composite update is pinned by central finite differences of each
    phase loss and by the piecewise golden vectors.  updates.py itself is not
    importable here (it needs gymnasium, absent from the image), so the
    composite ordering rests on reading updates.py/agent.py.
"""

import math
from collections import OrderedDict
from dataclasses import dataclass

import torch
import torch.nn.functional as F

BN_EPS = 1e-5
BN_MOMENTUM = 0.01
RMS_EPS = 1e-6
LOG_STD_MIN = -10.0
LOG_STD_MAX = 2.0


@dataclass
class Dims:
    actor_obs: int
    critic_obs: int
    action: int
    actor_hidden: int
    actor_blocks: int
    critic_hidden: int
    critic_blocks: int
    bins: int
    min_v: float
    max_v: float

    @property
    def critic_in(self) -> int:
        return self.critic_obs + self.action


def dims_from_config(observation_dim, action_dim, cfg, critic_observation_dim=None) -> Dims:
    return Dims(
        actor_obs=observation_dim,
        critic_obs=critic_observation_dim or observation_dim,
        action=action_dim,
        actor_hidden=cfg.actor_hidden_dim,
        actor_blocks=cfg.actor_num_blocks,
        critic_hidden=cfg.critic_hidden_dim,
        critic_blocks=cfg.critic_num_blocks,
        bins=cfg.critic_num_bins,
        min_v=cfg.critic_min_v,
        max_v=cfg.critic_max_v,
    )


# ---------------------------------------------------------------------------
# Parameter inventories, in the reference's named_parameters() order.
# ---------------------------------------------------------------------------
def actor_parameter_shapes(d: Dims) -> "OrderedDict[str, tuple]":
    """FlashSACActor (networks.py:23-61); names match its state_dict."""
    h = d.actor_hidden
    shapes = OrderedDict()
    shapes["embedder.norm.weight"] = (d.actor_obs,)
    shapes["embedder.norm.bias"] = (d.actor_obs,)
    shapes["embedder.w.w.weight"] = (h, d.actor_obs)
    for i in range(d.actor_blocks):
        shapes[f"encoder.{i}.w1.w.weight"] = (4 * h, h)
        shapes[f"encoder.{i}.w2.w.weight"] = (h, 4 * h)
        shapes[f"encoder.{i}.norm1.weight"] = (4 * h,)
        shapes[f"encoder.{i}.norm1.bias"] = (4 * h,)
        shapes[f"encoder.{i}.norm2.weight"] = (h,)
        shapes[f"encoder.{i}.norm2.bias"] = (h,)
    shapes["post_norm.weight"] = (h,)
    shapes["predictor.mean_w.w.weight"] = (d.action, h)
    shapes["predictor.mean_bias"] = (d.action,)
    shapes["predictor.std_w.w.weight"] = (d.action, h)
    shapes["predictor.std_bias"] = (d.action,)
    return shapes


def actor_buffer_shapes(d: Dims) -> "OrderedDict[str, tuple]":
    h = d.actor_hidden
    shapes = OrderedDict()
    shapes["embedder.norm.running_mean"] = (d.actor_obs,)
    shapes["embedder.norm.running_var"] = (d.actor_obs,)
    for i in range(d.actor_blocks):
        for name, width in (("norm1", 4 * h), ("norm2", h)):
            shapes[f"encoder.{i}.{name}.running_mean"] = (width,)
            shapes[f"encoder.{i}.{name}.running_var"] = (width,)
    return shapes


def critic_parameter_shapes(d: Dims) -> "OrderedDict[str, tuple]":
    """FlashSACDoubleCritic with two stacked critics (networks.py:64-110)."""
    h, i = d.critic_hidden, d.critic_in
    shapes = OrderedDict()
    shapes["embedder.norm.weight"] = (2, i)
    shapes["embedder.norm.bias"] = (2, i)
    shapes["embedder.w.weight"] = (2, h, i)
    for b in range(d.critic_blocks):
        shapes[f"encoder.{b}.w1.weight"] = (2, 4 * h, h)
        shapes[f"encoder.{b}.w2.weight"] = (2, h, 4 * h)
        shapes[f"encoder.{b}.norm1.weight"] = (2, 4 * h)
        shapes[f"encoder.{b}.norm1.bias"] = (2, 4 * h)
        shapes[f"encoder.{b}.norm2.weight"] = (2, h)
        shapes[f"encoder.{b}.norm2.bias"] = (2, h)
    shapes["post_norm.weight"] = (2, h)
    shapes["predictor.w.weight"] = (2, d.bins, h)
    shapes["predictor.bias"] = (2, d.bins)
    return shapes


def critic_buffer_shapes(d: Dims) -> "OrderedDict[str, tuple]":
    h, i = d.critic_hidden, d.critic_in
    shapes = OrderedDict()
    shapes["embedder.norm.running_mean"] = (2, i)
    shapes["embedder.norm.running_var"] = (2, i)
    for b in range(d.critic_blocks):
        for name, width in (("norm1", 4 * h), ("norm2", h)):
            shapes[f"encoder.{b}.{name}.running_mean"] = (2, width)
            shapes[f"encoder.{b}.{name}.running_var"] = (2, width)
    return shapes


def projection_kind(name: str) -> str | None:
    """Which normalize_parameters rule applies (layers.py:24-29, 57-64, 76-81)."""
    if name.endswith("mean_bias") or name.endswith("std_bias") or name == "predictor.bias":
        return None
    if ".norm" in name or name.startswith("embedder.norm"):
        return "bn"
    if name.startswith("post_norm"):
        return "rms"
    if name.endswith("weight"):
        return "row"
    return None


# ---------------------------------------------------------------------------
# Projection, EMA and schedule
# ---------------------------------------------------------------------------
@torch.no_grad()
def normalize_parameters(params: "OrderedDict[str, torch.Tensor]") -> None:
    """Network.normalize_parameters (network.py:55-64, 82-85)."""
    for name, value in params.items():
        kind = projection_kind(name)
        if kind == "row":
            value.copy_(F.normalize(value, dim=-1, eps=1e-8))
        elif kind == "rms":
            ndim = value.shape[-1]
            sqsum = torch.sum(value * value, dim=-1, keepdim=True)
            value.copy_(value * (math.sqrt(ndim) * torch.rsqrt(sqsum + 1e-8)))
        elif kind == "bn" and name.endswith(".weight"):
            bias = params[name[: -len("weight")] + "bias"]
            ndim = value.shape[-1]
            sqsum = torch.sum(value * value + bias * bias, dim=-1, keepdim=True)
            factor = math.sqrt(ndim) * torch.rsqrt(sqsum + 1e-8)
            value.copy_(value * factor)
            bias.copy_(bias * factor)


@torch.no_grad()
def ema_update(target: "OrderedDict[str, torch.Tensor]", source: "OrderedDict[str, torch.Tensor]", tau: float):
    """torch._foreach_lerp_(target, online, tau) over parameters (network.py:66-80)."""
    torch._foreach_lerp_(list(target.values()), list(source.values()), tau)


def warmup_cosine(init_value, peak_value, end_value, warmup_steps, decay_steps):
    """scheduler.py:43-65 (optax-style cosine after linear warmup)."""

    def schedule(step: int) -> float:
        if step < warmup_steps:
            return init_value + (peak_value - init_value) * (step / warmup_steps)
        if step < decay_steps:
            progress = (step - warmup_steps) / (decay_steps - warmup_steps)
            return end_value + (peak_value - end_value) * 0.5 * (1 + math.cos(math.pi * progress))
        return end_value

    return schedule


def safe_tanh_log_det_jacobian(x: torch.Tensor) -> torch.Tensor:
    """distribution.py:12-19."""
    return 2.0 * (math.log(2.0) - x - F.softplus(-2.0 * x))


# ---------------------------------------------------------------------------
# Parity-test hooks (the comparison needs them; the reference has no counterpart)
# ---------------------------------------------------------------------------
def round_bf16(x: torch.Tensor) -> torch.Tensor:
    """Round to the nearest bfloat16 (ties to even), returned in x's dtype."""
    return x.to(torch.bfloat16).to(x.dtype)


class _Round(torch.autograd.Function):
    """Identity or bf16 rounding in the forward and, independently, in the backward."""

    @staticmethod
    def forward(ctx, x, forward_round, backward_round):
        ctx.backward_round = backward_round
        return round_bf16(x) if forward_round else x.clone()

    @staticmethod
    def backward(ctx, grad):
        return (round_bf16(grad) if ctx.backward_round else grad), None, None


class Emulation:
    """How one device update rounds, for parity tests of it.

    relu_masks: one 0/1 tensor per ReLU, in execution order (per block norm1 then norm2, per
        forward in update order: actor, eval critic, next-action actor, target critic, online
        critic), shaped like that ReLU's input.  Each replaces the ReLU's pass/block decision with
        the device's, so inputs within rounding of zero (passed on one side, blocked on the other)
        do not enter the comparison; the forward value x * mask differs from relu(x) only on such
        elements, by less than their rounding.
    bf16: the bf16-operand mode: every dense product reads its operands rounded to bf16 (RNE) and
        the gradient reaching its output rounded to bf16 (the device feeds both backward products
        from a bf16 copy of it; bias gradients read the unrounded one).
    bf16_activations: with bf16, the block products' outputs (the BatchNorm inputs) are stored in
        bf16, and so is the gradient reaching the second block product's input (the ReLU-BatchNorm
        gradient).
    after_actor_phase: optional callable(state), run after the actor and temperature steps, before
        the critic phase (a test loads the device's post-step actor, log-temperature and actor
        BatchNorm statistics there, so the critic phase is compared from the same start).
    """

    def __init__(self, relu_masks=None, bf16: bool = False, bf16_activations: bool = False,
                 after_actor_phase=None, record_masks: list | None = None,
                 record_products: list | None = None):
        self.relu_masks = list(relu_masks) if relu_masks is not None else None
        self.bf16 = bf16
        self.bf16_activations = bf16 and bf16_activations
        self.after_actor_phase = after_actor_phase
        self.record_masks = record_masks  # receives the natural decisions x > 0 when nothing is forced
        self.record_products = record_products  # receives the block products' outputs (BatchNorm inputs)
        self.used = 0

    def relu(self, x: torch.Tensor) -> torch.Tensor:
        if self.relu_masks is None:
            if self.record_masks is not None:
                self.record_masks.append((x.detach() > 0).clone())
            return F.relu(x)
        if self.used >= len(self.relu_masks):
            raise ValueError("More ReLUs than forced masks.")
        mask = torch.as_tensor(self.relu_masks[self.used])
        self.used += 1
        if tuple(mask.shape) != tuple(x.shape):
            raise ValueError(f"Forced ReLU mask {tuple(mask.shape)} does not fit its input {tuple(x.shape)}.")
        return x * mask.to(x.dtype)

    def product(self, x, w, ensemble: bool, *, output_bf16: bool = False, input_grad_bf16: bool = False):
        """x W^T (ensemble: per member), with the device's roundings in bf16 mode."""
        if self.bf16:
            x = _Round.apply(x, True, input_grad_bf16 and self.bf16_activations)
            w = _Round.apply(w, True, False)
        y = torch.einsum("nbi,noi->nbo", x, w) if ensemble else F.linear(x, w)
        if self.bf16:
            y = _Round.apply(y, output_bf16 and self.bf16_activations, True)
        if output_bf16 and self.record_products is not None:
            self.record_products.append(y.detach().clone())
        return y


def _emulation(emulation):
    return emulation if emulation is not None else Emulation()


# ---------------------------------------------------------------------------
# Forward passes
# ---------------------------------------------------------------------------
def actor_forward(p, s, observations, training: bool, noise: torch.Tensor | None, d: Dims,
                  emulation: Emulation | None = None):
    """FlashSACActor.forward (networks.py:50-61) with rsample noise injected.

    Returns (actions, log_prob, mean, std).  BN running statistics in ``s``
    are updated in place in training mode, as F.batch_norm does (layers.py:36-55).
    ``emulation`` (parity tests only) applies a device's roundings and ReLU decisions.
    """
    em = _emulation(emulation)
    x = F.batch_norm(observations, s["embedder.norm.running_mean"], s["embedder.norm.running_var"],
                     p["embedder.norm.weight"], p["embedder.norm.bias"], training=training, momentum=BN_MOMENTUM,
                     eps=BN_EPS)
    x = em.product(x, p["embedder.w.w.weight"], False)
    for i in range(d.actor_blocks):
        residual = x
        x = em.product(x, p[f"encoder.{i}.w1.w.weight"], False, output_bf16=True)
        x = F.batch_norm(x, s[f"encoder.{i}.norm1.running_mean"], s[f"encoder.{i}.norm1.running_var"],
                         p[f"encoder.{i}.norm1.weight"], p[f"encoder.{i}.norm1.bias"], training=training,
                         momentum=BN_MOMENTUM, eps=BN_EPS)
        x = em.relu(x)
        x = em.product(x, p[f"encoder.{i}.w2.w.weight"], False, output_bf16=True, input_grad_bf16=True)
        x = F.batch_norm(x, s[f"encoder.{i}.norm2.running_mean"], s[f"encoder.{i}.norm2.running_var"],
                         p[f"encoder.{i}.norm2.weight"], p[f"encoder.{i}.norm2.bias"], training=training,
                         momentum=BN_MOMENTUM, eps=BN_EPS)
        x = em.relu(x)
        x = x + residual
    x = F.rms_norm(x, (d.actor_hidden,), p["post_norm.weight"], eps=RMS_EPS)
    mean = em.product(x, p["predictor.mean_w.w.weight"], False) + p["predictor.mean_bias"]
    raw_log_std = em.product(x, p["predictor.std_w.w.weight"], False) + p["predictor.std_bias"]
    log_std = LOG_STD_MIN + (LOG_STD_MAX - LOG_STD_MIN) * 0.5 * (1 + torch.tanh(raw_log_std))
    std = torch.exp(log_std)
    if noise is None:
        return torch.tanh(mean), None, mean, std
    dist = torch.distributions.Normal(mean, std)
    raw_action = mean + noise * std  # Normal.rsample: loc + eps * scale
    actions = torch.tanh(raw_action)
    log_prob = dist.log_prob(raw_action) - safe_tanh_log_det_jacobian(raw_action)
    return actions, log_prob.sum(1), mean, std


def _ensemble_bn(x, p, s, prefix, training):
    """EnsembleUnitBatchNorm.forward (layers.py:202-214)."""
    weight, bias = p[prefix + ".weight"], p[prefix + ".bias"]
    running_mean, running_var = s[prefix + ".running_mean"], s[prefix + ".running_var"]
    if training:
        mean = x.mean(dim=1, keepdim=True)
        var = x.var(dim=1, correction=0, keepdim=True)
        with torch.no_grad():
            rows = x.shape[1]
            running_mean.lerp_(mean.squeeze(1).to(running_mean.dtype), BN_MOMENTUM)
            running_var.lerp_((var.squeeze(1) * (rows / (rows - 1))).to(running_var.dtype), BN_MOMENTUM)
        x = (x - mean) * torch.rsqrt(var + BN_EPS)
    else:
        x = (x - running_mean.unsqueeze(1)) * torch.rsqrt(running_var.unsqueeze(1) + BN_EPS)
    return x * weight.unsqueeze(1) + bias.unsqueeze(1)


def critic_support(d: Dims, dtype=torch.float32) -> torch.Tensor:
    return torch.linspace(d.min_v, d.max_v, d.bins, dtype=torch.float32).to(dtype)


def _relu_margin(x, margins):
    """Per row, the smallest |ReLU input| relative to the row's largest (how near a rounding flip is)."""
    if margins is not None:
        with torch.no_grad():
            scale = x.abs().amax(dim=-1, keepdim=True).clamp_min(1e-30)
            margins.append((x.abs() / scale).amin(dim=-1))


def critic_forward(p, s, observations, actions, training: bool, d: Dims, margins: list | None = None,
                   emulation: Emulation | None = None):
    """FlashSACDoubleCritic.forward (networks.py:97-110); returns (q [2, R], log_probs [2, R, K]).
    margins (optional): receives one [2, R] tensor per ReLU, see _relu_margin.
    ``emulation`` (parity tests only) applies a device's roundings and ReLU decisions."""
    em = _emulation(emulation)
    x = torch.cat((observations, actions), dim=-1)
    x = x.unsqueeze(0).expand(2, -1, -1)
    x = _ensemble_bn(x, p, s, "embedder.norm", training)
    x = em.product(x, p["embedder.w.weight"], True)
    for b in range(d.critic_blocks):
        residual = x
        x = em.product(x, p[f"encoder.{b}.w1.weight"], True, output_bf16=True)
        x = _ensemble_bn(x, p, s, f"encoder.{b}.norm1", training)
        _relu_margin(x, margins)
        x = em.relu(x)
        x = em.product(x, p[f"encoder.{b}.w2.weight"], True, output_bf16=True, input_grad_bf16=True)
        x = _ensemble_bn(x, p, s, f"encoder.{b}.norm2", training)
        _relu_margin(x, margins)
        x = em.relu(x)
        x = x + residual
    rms = torch.sqrt(torch.mean(x * x, dim=-1, keepdim=True) + RMS_EPS)
    x = (x / rms) * p["post_norm.weight"].unsqueeze(1)
    value = em.product(x, p["predictor.w.weight"], True) + p["predictor.bias"].unsqueeze(1)
    log_prob = F.log_softmax(value, dim=-1)
    q = torch.sum(torch.exp(log_prob) * critic_support(d, log_prob.dtype).reshape(1, 1, -1), dim=-1)
    return q, log_prob


# ---------------------------------------------------------------------------
# Categorical target (updates.py:19-80)
# ---------------------------------------------------------------------------
def select_min_q_log_probs(next_qs, next_q_log_probs):
    bins = next_q_log_probs.shape[-1]
    min_indices = next_qs.argmin(dim=0)
    return torch.gather(next_q_log_probs, 0, min_indices[None, :, None].expand(1, -1, bins))[0]


def categorical_td_target(target_log_probs, reward, done, actor_entropy, gamma, bins, min_v, max_v):
    batch = reward.shape[0]
    reward = reward.reshape(-1, 1)
    done = done.reshape(-1, 1)
    actor_entropy = actor_entropy.reshape(-1, 1)
    gamma = gamma.reshape(-1, 1)
    bin_width = (max_v - min_v) / (bins - 1)
    bin_values = torch.linspace(min_v, max_v, bins, dtype=torch.float32).to(target_log_probs.dtype).view(1, -1)
    values = reward + gamma * (bin_values - actor_entropy) * (1.0 - done)
    values = torch.clamp(values, min_v, max_v)
    b = (values - min_v) / bin_width
    lower = torch.floor(b).long()
    upper = torch.clamp(lower + 1, 0, bins - 1)
    frac = b - lower.to(b.dtype)
    probs = target_log_probs.exp()
    target = torch.zeros(batch, bins, dtype=probs.dtype)
    target.scatter_add_(1, lower, probs * (1.0 - frac))
    target.scatter_add_(1, upper, probs * frac)
    return target


# ---------------------------------------------------------------------------
# State and update
# ---------------------------------------------------------------------------
class OracleState:
    """Parameters, BN buffers, Adam optimizers/schedulers of the three networks."""

    def __init__(self, d: Dims, cfg, dtype=torch.float32):
        self.d = d
        self.cfg = cfg
        self.dtype = dtype
        self.actor = OrderedDict((k, torch.zeros(v, dtype=dtype)) for k, v in actor_parameter_shapes(d).items())
        self.actor_buffers = OrderedDict((k, torch.zeros(v, dtype=dtype)) for k, v in actor_buffer_shapes(d).items())
        self.critic = OrderedDict((k, torch.zeros(v, dtype=dtype)) for k, v in critic_parameter_shapes(d).items())
        self.critic_buffers = OrderedDict((k, torch.zeros(v, dtype=dtype)) for k, v in critic_buffer_shapes(d).items())
        self.target = OrderedDict((k, torch.zeros(v, dtype=dtype)) for k, v in critic_parameter_shapes(d).items())
        self.target_buffers = OrderedDict((k, torch.zeros(v, dtype=dtype)) for k, v in critic_buffer_shapes(d).items())
        self.log_temp = torch.zeros(1, dtype=dtype)
        for group in (self.actor_buffers, self.critic_buffers, self.target_buffers):
            for name, value in group.items():
                if name.endswith("running_var"):
                    value.fill_(1.0)
        for group in (self.actor, self.critic, self.target, self.log_temp):
            for value in (group.values() if isinstance(group, dict) else [group]):
                value.requires_grad_(True)
        self.update_step = 0
        self._make_optimizers()

    def _make_optimizers(self):
        cfg = self.cfg
        schedule = warmup_cosine(cfg.learning_rate_init, cfg.learning_rate_peak, cfg.learning_rate_end,
                                 cfg.learning_rate_warmup_step, cfg.learning_rate_decay_step)
        self.optimizers, self.schedulers = {}, {}
        for name, params in (("actor", list(self.actor.values())), ("critic", list(self.critic.values())),
                             ("temperature", [self.log_temp])):
            optimizer = torch.optim.Adam(params, lr=cfg.learning_rate_peak, fused=False, foreach=False)
            self.optimizers[name] = optimizer
            self.schedulers[name] = torch.optim.lr_scheduler.LambdaLR(
                optimizer, lr_lambda=lambda step, f=schedule: f(step) / cfg.learning_rate_peak)

    def load_flat(self, state: dict) -> None:
        """Load parameters / buffers from a flat dict keyed actor.*, critic.*, target_critic.*, log_temperature."""
        with torch.no_grad():
            for prefix, params, buffers in (("actor", self.actor, self.actor_buffers),
                                            ("critic", self.critic, self.critic_buffers),
                                            ("target_critic", self.target, self.target_buffers)):
                for name, value in list(params.items()) + list(buffers.items()):
                    value.copy_(torch.as_tensor(state[f"{prefix}.{name}"]).reshape(value.shape).to(self.dtype))
            self.log_temp.copy_(torch.as_tensor(state["log_temperature"]).reshape(1).to(self.dtype))

    def flat(self) -> dict:
        out = {}
        for prefix, params, buffers in (("actor", self.actor, self.actor_buffers),
                                        ("critic", self.critic, self.critic_buffers),
                                        ("target_critic", self.target, self.target_buffers)):
            for name, value in list(params.items()) + list(buffers.items()):
                out[f"{prefix}.{name}"] = value.detach().clone()
        out["log_temperature"] = self.log_temp.detach().clone()
        return out

    def moments(self) -> dict:
        out = {}
        for name, params in (("actor", self.actor), ("critic", self.critic)):
            optimizer = self.optimizers[name]
            for key, value in params.items():
                st = optimizer.state.get(value, {})
                if st:
                    out[f"{name}.{key}.m1"] = st["exp_avg"].detach().clone()
                    out[f"{name}.{key}.m2"] = st["exp_avg_sq"].detach().clone()
        st = self.optimizers["temperature"].state.get(self.log_temp, {})
        if st:
            out["temperature.m1"] = st["exp_avg"].detach().clone()
            out["temperature.m2"] = st["exp_avg_sq"].detach().clone()
        return out


@torch.no_grad()
def init_state(d: Dims, cfg, seed: int = 0, dtype=torch.float32) -> OracleState:
    """Orthogonal unit-linear init, identity BN / RMS, projection, target copy (agent.py:40-156)."""
    state = OracleState(d, cfg, dtype)
    g = torch.Generator().manual_seed(seed)
    for params in (state.actor, state.critic):
        for name, value in params.items():
            kind = projection_kind(name)
            if kind == "row":
                if value.dim() == 3:
                    for e in range(value.shape[0]):
                        torch.nn.init.orthogonal_(value[e], gain=1, generator=g)
                else:
                    torch.nn.init.orthogonal_(value, gain=1, generator=g)
            elif kind in ("bn", "rms"):
                value.fill_(1.0 if name.endswith("weight") else 0.0)
            else:
                value.zero_()
    normalize_parameters(state.actor)
    normalize_parameters(state.critic)
    for name, value in state.critic.items():
        state.target[name].copy_(value)
    normalize_parameters(state.target)
    state.log_temp.fill_(math.log(cfg.temp_initial_value))
    return state


def target_entropy(action_dim: int, sigma: float) -> float:
    """agent.py:329."""
    return 0.5 * action_dim * math.log(2 * math.pi * math.e * sigma**2)


def _adam_step(state: OracleState, name: str, params, grads):
    for value, grad in zip(params, grads):
        value.grad = grad.detach().clone()
    state.optimizers[name].step()
    state.schedulers[name].step()
    for value in params:
        value.grad = None


def update(state: OracleState, batch: dict, actor_noise: torch.Tensor, next_noise: torch.Tensor,
           do_actor_update: bool | None = None, record: dict | None = None,
           emulation: Emulation | None = None) -> dict:
    """One FlashSAC update (agent.py:217-281 over updates.py:83-326).

    ``batch`` holds observation, action, reward, terminated, next_observation,
    discount (fp tensors, B rows).  ``record`` (optional) receives gradients
    and intermediate tensors for parity tests; ``emulation`` (optional) applies
    a device's roundings and ReLU decisions (parity tests).  Returns the
    reference metric dictionary.
    """
    em = emulation
    d, cfg = state.d, state.cfg
    dt = state.dtype
    if do_actor_update is None:
        do_actor_update = state.update_step % cfg.actor_update_period == 0
    b = {k: torch.as_tensor(v).to(dt) for k, v in batch.items()}
    obs, next_obs = b["observation"], b["next_observation"]
    actor_obs, actor_next_obs = obs[:, : d.actor_obs], next_obs[:, : d.actor_obs]
    rows = obs.shape[0]
    info = {}
    record = record if record is not None else {}

    if do_actor_update:
        # update_actor (updates.py:83-166)
        actor_params = list(state.actor.values())
        actions_all, log_probs_all, _, _ = actor_forward(state.actor, state.actor_buffers,
                                                         torch.cat([actor_obs, actor_next_obs], 0), True,
                                                         actor_noise.to(dt), d, emulation=em)
        actions = actions_all[:rows]
        log_probs = log_probs_all[:rows]
        critic_frozen = OrderedDict((k, v.detach()) for k, v in state.critic.items())
        qs, _ = critic_forward(critic_frozen, state.critic_buffers, obs, actions, False, d, emulation=em)
        q = torch.minimum(qs[0], qs[1])
        temp_value = torch.exp(state.log_temp).detach()
        actor_loss = (log_probs * temp_value - q).mean()
        if cfg.actor_bc_alpha > 0:
            q_abs = torch.abs(q).mean().detach()
            actor_loss = actor_loss + cfg.actor_bc_alpha * q_abs * ((actions - b["action"]) ** 2).mean()
        entropy = -log_probs.mean()
        mean_action = actions.mean()
        grads = torch.autograd.grad(actor_loss, actor_params + [actions_all])
        record["actor_dactions"] = grads[-1].detach().clone()  # the loss's gradient at the tanh outputs
        grads = grads[:-1]
        record["actor_grads"] = OrderedDict((k, g.detach().clone()) for k, g in zip(state.actor.keys(), grads))
        record["actor_actions"] = actions_all.detach().clone()
        record["actor_log_probs"] = log_probs_all.detach().clone()
        record["actor_q"] = qs.detach().clone()
        _adam_step(state, "actor", actor_params, grads)
        normalize_parameters(state.actor)
        info.update({"actor/loss": actor_loss.detach(), "actor/entropy": entropy.detach(),
                     "actor/mean_action": mean_action.detach()})
        # update_temperature (updates.py:297-326)
        temperature_value = torch.exp(state.log_temp)
        temperature_loss = temperature_value * (entropy.detach() - cfg.temp_target_entropy).mean()
        (grad,) = torch.autograd.grad(temperature_loss, [state.log_temp])
        record["temperature_grad"] = grad.detach().clone()
        _adam_step(state, "temperature", [state.log_temp], [grad])
        info.update({"temperature/value": temperature_value.detach(), "temperature/loss": temperature_loss.detach()})
        if em is not None and em.after_actor_phase is not None:
            em.after_actor_phase(state)

    # update_critic (updates.py:169-284)
    with torch.no_grad():
        actor_eval = OrderedDict((k, v.detach()) for k, v in state.actor.items())
        next_actions, next_log_probs, _, _ = actor_forward(actor_eval, state.actor_buffers, actor_next_obs, False,
                                                           next_noise.to(dt), d, emulation=em)
        temp_value = torch.exp(state.log_temp.detach())
        next_entropy = temp_value * next_log_probs
        obs_all = torch.cat([obs, next_obs], 0)
        act_all = torch.cat([b["action"], next_actions], 0)
        target_frozen = OrderedDict((k, v.detach()) for k, v in state.target.items())
        qs_all, lp_all = critic_forward(target_frozen, state.target_buffers, obs_all, act_all, True, d, emulation=em)
        next_qs = qs_all[:, rows:]
        next_lp = select_min_q_log_probs(next_qs, lp_all[:, rows:])
        target_probs = categorical_td_target(next_lp, b["reward"], b["terminated"], next_entropy, b["discount"],
                                             d.bins, d.min_v, d.max_v)
        max_entropy_bonus = next_entropy.max()
    record["next_actions"] = next_actions.clone()
    record["next_log_probs"] = next_log_probs.clone()
    record["target_q"] = qs_all.clone()
    record["target_probs"] = target_probs.clone()
    critic_params = list(state.critic.values())
    _, pred_lp = critic_forward(state.critic, state.critic_buffers, obs_all, act_all, True, d, emulation=em)
    ce = -(target_probs.unsqueeze(0) * pred_lp[:, :rows]).sum(dim=-1)
    critic_loss = ce.mean()
    grads = torch.autograd.grad(critic_loss, critic_params)
    record["critic_grads"] = OrderedDict((k, g.detach().clone()) for k, g in zip(state.critic.keys(), grads))
    _adam_step(state, "critic", critic_params, grads)
    normalize_parameters(state.critic)
    info.update({"critic/loss": critic_loss.detach(), "critic/max_entropy_bonus": max_entropy_bonus.detach()})
    # update_target_network (updates.py:287-294)
    ema_update(state.target, OrderedDict((k, v.detach()) for k, v in state.critic.items()),
               cfg.critic_target_update_tau)
    state.update_step += 1
    return info


def synthetic_replay(capacity: int, obs_dim: int, action_dim: int, *, seed: int, gamma: float,
                     reward_std: float = 1.0, done_prob: float = 0.01) -> dict:
    """Seeded replay contents with the BASELINE distributions (n_step = 1 semantics)."""
    g = torch.Generator().manual_seed(seed)
    return {
        "observation": torch.randn(capacity, obs_dim, generator=g),
        "next_observation": torch.randn(capacity, obs_dim, generator=g),
        "action": torch.rand(capacity, action_dim, generator=g) * 2 - 1,
        "reward": torch.randn(capacity, generator=g) * reward_std,
        "terminated": (torch.rand(capacity, generator=g) < done_prob).float(),
        "truncated": torch.zeros(capacity),
        "discount": torch.full((capacity,), gamma),
    }


def sample(storage: dict, indices) -> dict:
    """TorchUniformBuffer.sample with injected indices (replay.py:179-194)."""
    idx = torch.as_tensor(indices, dtype=torch.long)
    return {k: v[idx] for k, v in storage.items()}
