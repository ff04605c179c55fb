"""Fixed-shape PPO update on MI355X: GAE, advantage normalization, one device
permutation reused across epochs, and per minibatch the KL-adaptive learning
rate, the clipped surrogate/value/entropy loss, backward through both MLPs,
gradient clipping and Adam, all enqueued on one stream and captured in one
HIP graph.

Interface mirrors robolearn/warp/ppo.py:353-778 (WarpPPO): constructor, act,
store, compute_returns, launch_update, warmup, update, health_metrics,
state_dict/load_state_dict/save/load, with the same checkpoint keys.
Rollout buffers are time-major (k = step * num_envs + env), as the reference's.
"""

import math
from pathlib import Path

import numpy as np
import torch

from . import _native
from . import kernels as K
from .config import PPOConfig
from .networks import FlatStore, _align


def _mlp_shapes(prefix, input_dim, output_dim, hidden_dims):
    widths = (input_dim, *hidden_dims, output_dim)
    shapes = []
    for i, (a, b) in enumerate(zip(widths[:-1], widths[1:])):
        shapes.append((f"{prefix}.{i}.weight", (b, a)))
        shapes.append((f"{prefix}.{i}.bias", (b,)))
    return shapes


class WarpPPO:
    """PPO learner with the reference's WarpPPO interface, backed by HIP kernels."""

    def __init__(self, observation_dim: int, action_dim: int, num_envs: int, horizon: int,
                 config: PPOConfig | None = None, device: str = "cuda", gemm_mode: int = K.FP32_SPLIT):
        """gemm_mode: K.FP32_SPLIT (default; fp32-accurate products on the bf16 matrix cores from
        exact three-piece splits) or K.FP32 (the fp32 matrix-core instruction)."""
        if gemm_mode not in (K.FP32, K.FP32_SPLIT):
            raise ValueError("gemm_mode must be K.FP32 or K.FP32_SPLIT.")
        self.gemm_mode = gemm_mode
        self.config = cfg = config or PPOConfig()
        if min(observation_dim, action_dim, num_envs, horizon, cfg.epochs, *cfg.hidden_dims) < 1:
            raise ValueError("Dimensions, horizon, and epochs must be positive.")
        if cfg.initial_std <= 0:
            raise ValueError("initial_std must be positive.")
        if cfg.activation not in ("tanh", "elu") or cfg.std_type not in ("log", "scalar"):
            raise ValueError("activation must be 'tanh' or 'elu', and std_type must be 'log' or 'scalar'.")
        if cfg.schedule not in ("fixed", "adaptive") or cfg.desired_kl <= 0:
            raise ValueError("schedule must be 'fixed' or 'adaptive', and desired_kl must be positive.")
        if cfg.timeout_bootstrap not in ("next", "current"):
            raise ValueError("timeout_bootstrap must be 'next' or 'current'.")
        if cfg.std_range[0] <= 0 or cfg.std_range[0] > cfg.std_range[1]:
            raise ValueError("std_range must contain positive increasing bounds.")
        if action_dim > 64:
            raise ValueError("The MI355X PPO loss kernels support at most 64 action dimensions.")
        if cfg.activation != "elu":
            raise NotImplementedError("The MI355X PPO path implements ELU activations (the G1 recipe).")
        if not torch.cuda.is_available():
            raise RuntimeError("WarpPPO on MI355X requires a visible GPU; there is no CPU fallback.")
        _native.load()
        self.device = torch.device(device if ":" in str(device) else "cuda:0")
        self.num_envs, self.horizon = num_envs, horizon
        self.observation_dim, self.action_dim = observation_dim, action_dim
        self.batch_size = N = num_envs * horizon
        if cfg.num_mini_batches < 1 or N % cfg.num_mini_batches:
            raise ValueError("num_mini_batches must be positive and divide the rollout batch size.")
        self.mini_batch_size = M = N // cfg.num_mini_batches
        O, A = observation_dim, action_dim
        self.layers = len(cfg.hidden_dims) + 1
        actor = _mlp_shapes("actor", O, A, cfg.hidden_dims)
        critic = _mlp_shapes("critic", O, 1, cfg.hidden_dims)
        # With hidden layers the two output layers run as one batch-2 product of A outputs: the
        # value head's weight and bias are followed in the flat store by A - 1 zero rows (never
        # optimized, never part of a named parameter), so member 1 of the batch is the value head
        # padded to A outputs whose extra outputs and gradients are exactly zero.
        last = self.layers - 1
        self.batched_heads = bool(cfg.hidden_dims)
        pads = {}
        if self.batched_heads and A > 1:
            pads = {f"critic.{last}.weight": (f"critic.{last}.weight_pad", (A - 1, cfg.hidden_dims[-1])),
                    f"critic.{last}.bias": (f"critic.{last}.bias_pad", (A - 1,))}
        shapes = dict(actor + critic + [("std", (A,))] + list(pads.values()))
        dev = self.device
        with torch.cuda.device(dev):
            # actor tensors + std parameter form clipping group 0, critic tensors group 1
            order = [[n for n, _ in actor] + ["std"], [n for n, _ in critic]]
            groups = [[n] for n in order[0]] + [[n] + ([pads[n][0]] if n in pads else []) for n in order[1]]
            self.flat = FlatStore(shapes, dev, groups=groups)
            self.names = [n for n, _ in actor] + [n for n, _ in critic] + ["std"]
            views = self.flat.params()
            self.parameters = [views[n] for n in self.names]
            self.grads = self.flat.grads()
            rng = np.random.default_rng(cfg.seed)
            for n, shape in actor + critic:
                bound = 1.0 / math.sqrt(shape[-1] if n.endswith("weight") else shapes[n[:-4] + "weight"][-1])
                views[n].copy_(torch.as_tensor(rng.uniform(-bound, bound, shape).astype(np.float32)))
            std0 = math.log(cfg.initial_std) if cfg.std_type == "log" else cfg.initial_std
            views["std"].fill_(std0)
            self.distribution_parameter = views["std"]
            if cfg.std_type == "log":
                self.log_std = self.distribution_parameter
            else:
                self.std_param = self.distribution_parameter
            first_critic = self.flat.offsets[critic[0][0]]
            self.group_ranges = [(0, first_critic), (first_critic, self.flat.size)]
            if not cfg.separate_grad_clipping:
                self.group_ranges = [(0, self.flat.size)]
            self.timestep = torch.zeros(1, device=dev)
            self.lr = torch.full((1,), float(cfg.learning_rate), device=dev)
            self._make_optimizer()
            z = lambda *s: torch.zeros(*s, device=dev)  # noqa: E731
            self.observations = z(N, O)
            self.actions = z(N, A)
            self.means = z(N, A)
            self.stds = z(N, A)
            for name in ("log_probs", "values", "rewards", "next_values", "advantages", "returns"):
                setattr(self, name, z(N))
            self.terminated = torch.zeros(N, dtype=torch.int32, device=dev)
            self.truncated = torch.zeros(N, dtype=torch.int32, device=dev)
            self._seed = torch.tensor([cfg.seed], dtype=torch.int32, device=dev)
            self._stats = z(2)
            self._perm = torch.zeros(N, dtype=torch.int32, device=dev)
            # minibatch observations with 16-byte aligned rows (zero pad columns) so the
            # first layer's products read them with vector loads
            self.obs_ld = (O + 3) // 4 * 4
            self.b_obs = z(M, self.obs_ld)
            self.b_actions, self.b_means, self.b_stds = z(M, A), z(M, A), z(M, A)
            self.b_log_probs, self.b_values, self.b_advantages, self.b_returns = z(M), z(M), z(M), z(M)
            widths = (O, *cfg.hidden_dims)
            # hidden activations and input gradients of both MLPs as [2, M, width] pairs (actor, critic), so
            # each hidden layer of the two networks runs as one batch-2 product
            self.h_pair = [z(2, M, w) for w in cfg.hidden_dims]
            self.d_pair = [z(2, M, w) for w in widths]
            self.actor_h = [h[0] for h in self.h_pair]
            self.critic_h = [h[1] for h in self.h_pair]
            # element offsets from each actor hidden-layer tensor to the critic's (batch strides of the pairs)
            offsets = self.flat.offsets
            self.w_stride = [offsets[f"critic.{i}.weight"] - offsets[f"actor.{i}.weight"]
                             for i in range(len(cfg.hidden_dims))]
            self.b_stride = [offsets[f"critic.{i}.bias"] - offsets[f"actor.{i}.bias"]
                             for i in range(len(cfg.hidden_dims))]
            if self.batched_heads:
                # [2, M, A]: member 0 the mean, member 1 column 0 the value (columns 1.. stay zero in
                # the gradient: the loss writes column 0 only)
                self.head_out, self.head_grad = z(2, M, A), z(2, M, A)
                self.mean, self.value = self.head_out[0], self.head_out[1]
                self.dmean, self.dvalue = self.head_grad[0], self.head_grad[1]
                self.value_ld = A
                self.head_w_stride = offsets[f"critic.{last}.weight"] - offsets[f"actor.{last}.weight"]
                self.head_b_stride = offsets[f"critic.{last}.bias"] - offsets[f"actor.{last}.bias"]
            else:
                self.mean, self.value = z(M, A), z(M, 1)
                self.dmean, self.dvalue = z(M, A), z(M, 1)
                self.value_ld = 1
            self.loss_partial = z((5 + A) * ((M + 15) // 16))  # per-16-row-workgroup loss, KL, std-gradient sums
            self.totals = z(4)
            self.metrics = self.totals[1:]  # policy loss, value loss, entropy of the last minibatch
            self.loss = self.totals[:1]
            self.kl = z(1)
            max_width = max(A, 1, *cfg.hidden_dims)
            self.partial = z(max(K.chunks(M) * max_width, (M + 15) // 16))  # column / KL partial sums
            self.norm_partial = z((self.flat.size + 4095) // 4096 + 1)
            self.group_norms = [z(1) for _ in self.group_ranges]
            self.workspace = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
            self._act_buffers = {}
            self._act_rows = 0
            self._act_counter = torch.zeros(1, dtype=torch.long, device=dev)  # Philox draw counter of act()
        self._update_graph = None

    def _make_optimizer(self):
        n = len(self.names)
        store = self.flat
        ptrs = lambda buf: _native.pointer_array([store.view(buf, name).data_ptr() for name in self.names])  # noqa
        rows = [1] * n
        cols = [int(np.prod(store.shapes[name])) for name in self.names]
        self.optimizer_handle = _native.create(
            "rl_fused_optimizer_create", n, _native.int_array([3] * n), _native.ll_array(rows),
            _native.ll_array(cols), ptrs(store.param), ptrs(store.grad), ptrs(store.m1), ptrs(store.m2), None, None,
            None, _native.int_array([-1] * n), self.timestep.data_ptr(), self.lr.data_ptr(), 0.9, 0.999, 1e-8, 0.0, 1,
            0, 0.0, 0.0, 0.0, 0, 1)

    def __del__(self):
        handle = getattr(self, "optimizer_handle", None)
        if handle:
            try:
                _native.load().rl_fused_optimizer_destroy(handle)
            except Exception:
                pass

    # ------------------------------------------------------------------
    def _layer(self, prefix, i):
        p = self.flat.params()
        return p[f"{prefix}.{i}.weight"], p[f"{prefix}.{i}.bias"]

    def _mlp_forward(self, prefix, x, rows, hidden, out, x_ld=None):
        """Linear + ELU hidden layers (ELU fused in the GEMM epilogue), linear output.
        x_ld: row pitch of x (default the observation width)."""
        widths = (self.observation_dim, *self.config.hidden_dims)
        inputs = x
        for i, width in enumerate(self.config.hidden_dims):
            w, b = self._layer(prefix, i)
            K.linear_forward(inputs, w, hidden[i], rows=rows, in_dim=widths[i], out_dim=width, bias=b,
                             epilogue="elu", mode=self.gemm_mode, x_ld=x_ld if i == 0 else None)
            inputs = hidden[i]
        w, b = self._layer(prefix, self.layers - 1)
        K.linear_forward(inputs, w, out, rows=rows, in_dim=widths[-1], out_dim=out.shape[1], bias=b, mode=self.gemm_mode)

    def _joint_forward(self, rows):
        """Both MLPs on the minibatch observations: each hidden layer is one batch-2 product over
        the actor and critic weights (Linear + bias + ELU in the GEMM epilogue), then the two
        output layers (mean, value)."""
        hidden = self.config.hidden_dims
        widths = (self.observation_dim, *hidden)
        for i, width in enumerate(hidden):
            w, b = self._layer("actor", i)
            first = i == 0
            K.gemm(self.b_obs if first else self.h_pair[i - 1], w, self.h_pair[i], m=rows, n=width, k=widths[i],
                   batch=2, a_kcontig=True, b_kcontig=True, lda=self.obs_ld if first else widths[i], ldb=widths[i],
                   ldd=width, stride_a=0 if first else rows * widths[i], stride_b=self.w_stride[i],
                   stride_d=rows * width, bias=b, stride_bias=self.b_stride[i], epilogue="elu", mode=self.gemm_mode)
        last = self.layers - 1
        if self.batched_heads:
            w, b = self._layer("actor", last)
            A, width = self.action_dim, widths[-1]
            K.gemm(self.h_pair[-1], w, self.head_out, m=rows, n=A, k=width, batch=2, a_kcontig=True, b_kcontig=True,
                   lda=width, ldb=width, ldd=A, stride_a=rows * width, stride_b=self.head_w_stride,
                   stride_d=rows * A, bias=b, stride_bias=self.head_b_stride, mode=self.gemm_mode)
            return
        for member, (prefix, out) in enumerate((("actor", self.mean), ("critic", self.value))):
            w, b = self._layer(prefix, last)
            K.linear_forward(self.b_obs, w, out, rows=rows, in_dim=widths[-1], out_dim=out.shape[1], bias=b,
                             mode=self.gemm_mode, x_ld=self.obs_ld)

    def _joint_backward(self, rows):
        """Weight, bias and input gradients of both MLPs: the output layers one network at a time,
        the hidden layers as batch-2 products (the ELU backward of the layer below fused into each
        input-gradient epilogue; bias gradients as row sums of the weight-gradient products)."""
        hidden = self.config.hidden_dims
        widths = (self.observation_dim, *hidden)
        g = self.grads
        last = self.layers - 1
        if self.batched_heads:
            # both output layers as batch-2 products of A outputs (the value head zero-padded)
            A, width = self.action_dim, widths[-1]
            w, _ = self._layer("actor", last)
            dw, db = g[f"actor.{last}.weight"], g[f"actor.{last}.bias"]
            h = self.h_pair[last - 1]
            splits = K.split_count(A, width, rows, 2, self.gemm_mode)
            if splits > 1 and _native.load().rl_gemm_workspace(self.gemm_mode, A, width, rows, 2, splits) > \
                    self.workspace.numel():
                splits = 1
            K.gemm(self.head_grad, h, dw, m=A, n=width, k=rows, batch=2, a_kcontig=False, b_kcontig=False, lda=A,
                   ldb=width, ldd=width, stride_a=rows * A, stride_b=rows * width, stride_d=self.head_w_stride,
                   mode=self.gemm_mode, splits=splits, workspace=self.workspace if splits > 1 else None, a_sums=db,
                   stride_bias=self.head_b_stride)
            K.gemm(self.head_grad, w, self.d_pair[last], m=rows, n=width, k=A, batch=2, a_kcontig=True,
                   b_kcontig=False, lda=A, ldb=width, ldd=width, stride_a=rows * A, stride_b=self.head_w_stride,
                   stride_d=rows * width, mode=self.gemm_mode, c=h, epilogue="elu_grad")
        else:
            for member, (prefix, dout) in enumerate((("actor", self.dmean), ("critic", self.dvalue))):
                K.linear_backward_weight(dout, self.b_obs, g[f"{prefix}.{last}.weight"], rows=rows, in_dim=widths[-1],
                                         out_dim=dout.shape[1], mode=self.gemm_mode, workspace=self.workspace,
                                         x_ld=self.obs_ld, bias_grad=g[f"{prefix}.{last}.bias"])
        for i in reversed(range(last)):
            out_dim, in_dim = hidden[i], widths[i]
            d = self.d_pair[i + 1]
            first = i == 0
            inputs = self.b_obs if first else self.h_pair[i - 1]
            splits = K.split_count(out_dim, in_dim, rows, 2, self.gemm_mode)
            if splits > 1 and _native.load().rl_gemm_workspace(self.gemm_mode, out_dim, in_dim, rows, 2, splits) > \
                    self.workspace.numel():
                splits = 1
            K.gemm(d, inputs, g[f"actor.{i}.weight"], m=out_dim, n=in_dim, k=rows, batch=2, a_kcontig=False,
                   b_kcontig=False, lda=out_dim, ldb=self.obs_ld if first else in_dim, ldd=in_dim,
                   stride_a=rows * out_dim, stride_b=0 if first else rows * in_dim, stride_d=self.w_stride[i],
                   mode=self.gemm_mode, splits=splits, workspace=self.workspace if splits > 1 else None,
                   a_sums=g[f"actor.{i}.bias"], stride_bias=self.b_stride[i])
            if not first:
                w, _ = self._layer("actor", i)
                K.gemm(d, w, self.d_pair[i], m=rows, n=in_dim, k=out_dim, batch=2, a_kcontig=True, b_kcontig=False,
                       lda=out_dim, ldb=in_dim, ldd=in_dim, stride_a=rows * out_dim, stride_b=self.w_stride[i],
                       stride_d=rows * in_dim, mode=self.gemm_mode, c=self.h_pair[i - 1], epilogue="elu_grad")

    # ------------------------------------------------------------------
    def compute_returns(self) -> None:
        cfg = self.config
        _native.call("rl_gae", self.horizon, self.num_envs, float(cfg.gamma), float(cfg.gae_lambda),
                     int(cfg.timeout_bootstrap == "current"), self.rewards.data_ptr(), self.values.data_ptr(),
                     self.next_values.data_ptr(), self.terminated.data_ptr(), self.truncated.data_ptr(),
                     self.advantages.data_ptr(), self.returns.data_ptr(), K.stream())
        if cfg.normalize_advantages:
            _native.call("rl_normalize_advantages", self.advantages.data_ptr(), self.batch_size,
                         int(cfg.advantage_sample_std), self._stats.data_ptr(), K.stream())

    def _minibatch(self, offset: int):
        cfg = self.config
        M, A, O = self.mini_batch_size, self.action_dim, self.observation_dim
        _native.call("rl_ppo_gather", self._perm.data_ptr(), offset, M, O, A, self.obs_ld, self.observations.data_ptr(),
                     self.actions.data_ptr(), self.log_probs.data_ptr(), self.values.data_ptr(),
                     self.advantages.data_ptr(), self.returns.data_ptr(), self.means.data_ptr(),
                     self.stds.data_ptr(), self.b_obs.data_ptr(), self.b_actions.data_ptr(),
                     self.b_log_probs.data_ptr(), self.b_values.data_ptr(), self.b_advantages.data_ptr(),
                     self.b_returns.data_ptr(), self.b_means.data_ptr(), self.b_stds.data_ptr(), K.stream())
        self._joint_forward(M)
        # loss, its gradients, the pre-step KL with the adaptive learning rate and the std-parameter
        # gradient: two launches (ppo.py:207-310)
        _native.call("rl_ppo_minibatch_loss", self.mean.data_ptr(), A, self.value.data_ptr(), self.value_ld,
                     self.distribution_parameter.data_ptr(), self.b_actions.data_ptr(), self.b_log_probs.data_ptr(),
                     self.b_values.data_ptr(), self.b_advantages.data_ptr(), self.b_returns.data_ptr(),
                     self.b_means.data_ptr(), self.b_stds.data_ptr(), M, A, int(cfg.std_type == "scalar"),
                     float(cfg.std_range[0]), float(cfg.std_range[1]), float(cfg.clip_ratio),
                     float(cfg.value_coefficient), float(cfg.entropy_coefficient), float(cfg.value_loss_scale),
                     int(cfg.clip_value), float(cfg.desired_kl), int(cfg.schedule == "adaptive"),
                     self.dmean.data_ptr(), self.dvalue.data_ptr(), self.value_ld, self.grads["std"].data_ptr(),
                     self.loss_partial.data_ptr(), self.totals.data_ptr(), self.kl.data_ptr(), self.lr.data_ptr(),
                     K.stream())
        self._joint_backward(M)
        if len(self.group_ranges) == 1:
            # combined clipping (Adam(max_norm), ppo.py:434): folded into the optimizer step's two launches
            (start, end), norm = self.group_ranges[0], self.group_norms[0]
            grad = self.flat.grad[start:end]
            _native.call("rl_fused_optimizer_step_clipped", self.optimizer_handle, 0, 0, grad.data_ptr(),
                         grad.numel(), self.norm_partial.data_ptr(), norm.data_ptr(), float(cfg.max_grad_norm),
                         K.stream())
            return
        for (start, end), norm in zip(self.group_ranges, self.group_norms):
            grad = self.flat.grad[start:end]
            _native.call("rl_clip_grad_norm", grad.data_ptr(), grad.numel(), self.norm_partial.data_ptr(),
                         norm.data_ptr(), float(cfg.max_grad_norm), K.stream())
        _native.call("rl_fused_optimizer_step", self.optimizer_handle, 1, 0, 0, None, K.stream())

    def launch_update(self) -> None:
        """Enqueue the entire PPO update (graph-capturable)."""
        cfg = self.config
        self.compute_returns()
        if cfg.num_mini_batches > 1:
            _native.call("rl_advance_int", self._seed.data_ptr(), K.stream())
            _native.call("rl_permutation", self.batch_size, int(cfg.seed) * 2654435761 + 1, self._seed.data_ptr(),
                         None, self._perm.data_ptr(), K.stream())
        else:
            self._perm.copy_(torch.arange(self.batch_size, dtype=torch.int32, device=self.device))
        for _ in range(cfg.epochs):
            for mb in range(cfg.num_mini_batches):
                self._minibatch(mb * self.mini_batch_size)

    def warmup(self) -> None:
        state = self.state_dict()
        self.launch_update()
        torch.cuda.synchronize(self.device)
        self.load_state_dict(state)

    def update(self, capture: bool = True) -> None:
        with torch.cuda.device(self.device):
            if not capture:
                self.launch_update()
                return
            if self._update_graph is None:
                self.warmup()
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph):
                    self.launch_update()
                self._update_graph = graph
            self._update_graph.replay()

    # ------------------------------------------------------------------
    def _act_state(self, n: int):
        """Per-row-count buffers of act(): MLP activations, mean, value, noise and the sampled outputs."""
        if n not in self._act_buffers:
            z = lambda *s: torch.zeros(*s, device=self.device)  # noqa: E731
            A = self.action_dim
            self._act_buffers[n] = dict(hidden=[z(n, w) for w in self.config.hidden_dims], mean=z(n, A),
                                        value=z(n, 1), noise=z(n, A), actions=z(n, A), log_probs=z(n), values=z(n),
                                        std=z(A), next_value=z(n, 1))
        return self._act_buffers[n]

    @torch.no_grad()
    def act(self, observations, deterministic: bool = False):
        """Gaussian actions from the actor mean and the distribution parameter (ppo.py:488-507).

        The MLPs run on the fp32 MFMA GEMMs; the noise is a Philox draw keyed by
        the seed and a device counter, and rl_ppo_sample forms the actions,
        log-probs, values and sampled std (ppo.py:26-58) for store()."""
        obs = torch.as_tensor(observations, device=self.device, dtype=torch.float32)
        if obs.dim() != 2 or obs.shape[1] != self.observation_dim:
            raise ValueError("act() expects [rows, observation_dim] observations.")
        obs = obs.contiguous()
        n = obs.shape[0]
        b = self._act_state(n)
        cfg = self.config
        with torch.cuda.device(self.device):
            self._mlp_forward("actor", obs, n, b["hidden"], b["mean"])
            self._mlp_forward("critic", obs, n, b["hidden"], b["value"])
            noise = None
            if not deterministic:
                K.philox_normal(b["noise"], seed=cfg.seed * 7919 + 53, counter=self._act_counter, stream_id=53)
                noise = b["noise"]
            _native.call("rl_ppo_sample", b["mean"].data_ptr(), self.action_dim, b["value"].data_ptr(), 1,
                         self.distribution_parameter.data_ptr(), int(cfg.std_type == "scalar"),
                         float(cfg.std_range[0]), float(cfg.std_range[1]),
                         noise.data_ptr() if noise is not None else None, n, self.action_dim,
                         b["actions"].data_ptr(), b["log_probs"].data_ptr(), b["values"].data_ptr(),
                         b["std"].data_ptr(), self._act_counter.data_ptr() if noise is not None else None, K.stream())
        self._act_rows = n
        return b["actions"].clone()

    @torch.no_grad()
    def store(self, step, observations, rewards, terminated, truncated, next_observations) -> None:
        """Store the last sampled action and bootstrap from the pre-reset next observation (ppo.py:509-550)."""
        if not 0 <= step < self.horizon:
            raise ValueError("step must be within the rollout horizon.")
        n = self.num_envs
        if self._act_rows != n:
            raise RuntimeError("store() needs a preceding act() over num_envs observations.")
        b = self._act_state(n)
        dev = self.device
        obs = torch.as_tensor(observations, device=dev, dtype=torch.float32).reshape(n, self.observation_dim)
        next_obs = torch.as_tensor(next_observations, device=dev, dtype=torch.float32).reshape(n, self.observation_dim)
        rewards = torch.as_tensor(rewards, device=dev, dtype=torch.float32).reshape(n).contiguous()
        terminated = torch.as_tensor(terminated, device=dev).reshape(n).to(torch.int32).contiguous()
        truncated = torch.as_tensor(truncated, device=dev).reshape(n).to(torch.int32).contiguous()
        obs, next_obs = obs.contiguous(), next_obs.contiguous()
        with torch.cuda.device(dev):
            self._mlp_forward("critic", next_obs, n, b["hidden"], b["next_value"])
            _native.call("rl_ppo_store", int(step), n, self.observation_dim, self.action_dim, obs.data_ptr(),
                         b["actions"].data_ptr(), b["log_probs"].data_ptr(), b["values"].data_ptr(),
                         rewards.data_ptr(), terminated.data_ptr(), truncated.data_ptr(), b["next_value"].data_ptr(),
                         1, b["mean"].data_ptr(), self.action_dim, b["std"].data_ptr(),
                         self.observations.data_ptr(), self.actions.data_ptr(), self.log_probs.data_ptr(),
                         self.values.data_ptr(), self.rewards.data_ptr(), self.terminated.data_ptr(),
                         self.truncated.data_ptr(), self.next_values.data_ptr(), self.means.data_ptr(),
                         self.stds.data_ptr(), K.stream())

    def health_metrics(self) -> dict:
        parameter = self.distribution_parameter.detach().cpu().numpy()
        std = np.clip(parameter, *self.config.std_range) if self.config.std_type == "scalar" else np.exp(parameter)
        totals = self.totals.cpu().numpy()
        result = {
            "std_min": float(std.min()), "std_mean": float(std.mean()), "std_max": float(std.max()),
            "std_parameter_min": float(parameter.min()), "std_parameter_max": float(parameter.max()),
            "learning_rate": float(self.lr.item()), "kl": float(self.kl.item()),
            "policy_loss": float(totals[1]), "value_loss": float(totals[2]), "entropy": float(totals[3]),
            "optimizer_updates": float(self.timestep.item()),
        }
        if self.config.separate_grad_clipping:
            result["actor_grad_norm"] = float(np.sqrt(self.group_norms[0].item()))
            result["critic_grad_norm"] = float(np.sqrt(self.group_norms[1].item()))
        return result

    def state_dict(self) -> dict:
        torch.cuda.synchronize(self.device)
        m1, m2 = self.flat.moments()
        state = {f"parameter_{i}": p.detach().cpu().numpy().copy() for i, p in enumerate(self.parameters)}
        state.update({f"adam_m1_{i}": m1[n].cpu().numpy().copy() for i, n in enumerate(self.names)})
        state.update({f"adam_m2_{i}": m2[n].cpu().numpy().copy() for i, n in enumerate(self.names)})
        state["adam_timestep"] = self.timestep.cpu().numpy().copy()
        state["adam_lr"] = self.lr.cpu().numpy().copy()
        state["seed"] = self._seed.cpu().numpy().copy()
        return state

    @torch.no_grad()
    def load_state_dict(self, state: dict) -> None:
        m1, m2 = self.flat.moments()
        arrays = {f"parameter_{i}": p for i, p in enumerate(self.parameters)}
        arrays.update({f"adam_m1_{i}": m1[n] for i, n in enumerate(self.names)})
        arrays.update({f"adam_m2_{i}": m2[n] for i, n in enumerate(self.names)})
        arrays.update(adam_timestep=self.timestep, adam_lr=self.lr, seed=self._seed)
        if set(state) != set(arrays):
            raise ValueError("Checkpoint parameter or optimizer keys do not match this model.")
        for name, array in arrays.items():
            if tuple(np.asarray(state[name]).shape) != tuple(array.shape):
                raise ValueError(f"Checkpoint shape for {name} does not match this model.")
        for name, array in arrays.items():
            array.copy_(torch.as_tensor(np.asarray(state[name])).to(array.dtype))

    def save(self, path) -> None:
        with Path(path).open("wb") as file:
            np.savez(file, **self.state_dict())

    def load(self, path) -> None:
        with np.load(path, allow_pickle=False) as state:
            self.load_state_dict(dict(state))
