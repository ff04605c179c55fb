"""FlashSAC networks on persistent GPU buffers, driven through the C ABI.

Structure follows robolearn/flashsac/layers.py and networks.py:
  embedder   BN(x) -> Linear (bias-free)                         layers.py:84-93
  block      Linear -> BN -> ReLU -> Linear -> BN -> ReLU -> +x    layers.py:96-113
  post norm  RMSNorm (eps 1e-6)                                   layers.py:67-74, 225-240
  heads      tanh-Gaussian policy (layers.py:116-166) or categorical value
             head (layers.py:275-303)
The twin critic is one ensemble of two members (layers.py:174-303); every
kernel takes the member count and strides, so both critics run in one launch.

Parameters of a network live in one flat fp32 buffer with named views that
match the reference state_dict keys; gradients, Adam moments and the EMA target
are parallel flat buffers with the same offsets.  Activations are laid out
[member, row, channel] for the largest row count the learner uses.  Every
backward writes each gradient element exactly once (first writer overwrites),
so no gradient clearing pass exists.
"""

import math
from collections import OrderedDict

import torch

from . import _native
from . import kernels as K

ALIGN = 64  # floats: 256-byte alignment of every tensor in a flat buffer


def _numel(shape) -> int:
    return int(math.prod(shape))


def _align(value: int) -> int:
    return (value + ALIGN - 1) // ALIGN * ALIGN


class FlatStore:
    """Named views into flat parameter / gradient / moment / target buffers."""

    def __init__(self, shapes: "OrderedDict[str, tuple]", device, *, groups=None, adam=True, target=False,
                 grads=True, shadows=False):
        self.shapes = OrderedDict(shapes)
        groups = groups or [[name] for name in shapes]
        grouped = {name for group in groups for name in group}
        groups = list(groups) + [[name] for name in shapes if name not in grouped]
        self.offsets = {}
        position = 0
        for group in groups:
            position = _align(position)
            for name in group:
                self.offsets[name] = position
                position += _numel(self.shapes[name])
        self.size = _align(position)
        self.param = torch.zeros(self.size, device=device)
        self.grad = torch.zeros(self.size, device=device) if grads else None
        self.m1 = torch.zeros(self.size, device=device) if adam else None
        self.m2 = torch.zeros(self.size, device=device) if adam else None
        self.target = torch.zeros(self.size, device=device) if target else None
        # bf16 operand copies of the parameters (and of the target), written by the optimizer
        self.shadow = torch.zeros(self.size, dtype=torch.bfloat16, device=device) if shadows else None
        self.target_shadow = (torch.zeros(self.size, dtype=torch.bfloat16, device=device)
                              if shadows and target else None)

        # transposed bf16 copies of selected [E, out, in] weights, [E, in, out]
        self.transposed = OrderedDict()

    def enable_transposed(self, names):
        """Keep [E, in, out] transposed bf16 copies of these weights (input-gradient operands)."""
        if self.shadow is None:
            return
        for name in names:
            e, o, i = self._matrix_dims(name)
            self.transposed[name] = torch.zeros(e, i, o, dtype=torch.bfloat16, device=self.param.device)

    def _matrix_dims(self, name):
        shape = self.shapes[name]
        o, i = shape[-2], shape[-1]
        return _numel(shape) // (o * i), o, i

    def refresh_transposed(self):
        jobs = []
        for name, dst in self.transposed.items():
            e, o, i = self._matrix_dims(name)
            jobs.append((self.view(self.shadow, name), dst, e, o, i))
        if not jobs:
            return
        # one launch for the whole store where the shapes allow it (hidden widths are multiples of 4)
        if len(jobs) <= 8 and all(o % 4 == 0 and i % 4 == 0 and src.data_ptr() % 8 == 0 and dst.data_ptr() % 8 == 0
                                  for src, dst, _, o, i in jobs):
            K.transpose16_many(jobs)
            return
        for src, dst, e, o, i in jobs:
            K.transpose16(src, dst, batch=e, rows=o, cols=i)

    def refresh_shadows(self):
        """Re-derive the bf16 copies from the fp32 masters (after init or a checkpoint load)."""
        if self.shadow is not None:
            K.cast_bf16(self.param, self.shadow)
        if self.target_shadow is not None:
            K.cast_bf16(self.target, self.target_shadow)
        self.refresh_transposed()

    def view(self, buffer, name):
        offset = self.offsets[name]
        return buffer[offset: offset + _numel(self.shapes[name])].view(self.shapes[name])

    def span(self, buffer, names, shape):
        """Contiguous view over consecutive tensors of one allocation group."""
        offset = self.offsets[names[0]]
        total = sum(_numel(self.shapes[n]) for n in names)
        for a, b in zip(names, names[1:]):
            if self.offsets[b] != self.offsets[a] + _numel(self.shapes[a]):
                raise ValueError(f"{a} and {b} are not adjacent")
        return buffer[offset: offset + total].view(shape)

    def params(self):
        return OrderedDict((n, self.view(self.param, n)) for n in self.shapes)

    def grads(self):
        return OrderedDict((n, self.view(self.grad, n)) for n in self.shapes)

    def targets(self):
        return OrderedDict((n, self.view(self.target, n)) for n in self.shapes)

    def shadows(self):
        return OrderedDict((n, self.view(self.shadow, n)) for n in self.shapes) if self.shadow is not None else None

    def target_shadows(self):
        if self.target_shadow is None:
            return None
        return OrderedDict((n, self.view(self.target_shadow, n)) for n in self.shapes)

    def moments(self):
        return (OrderedDict((n, self.view(self.m1, n)) for n in self.shapes),
                OrderedDict((n, self.view(self.m2, n)) for n in self.shapes))


def projection_kind(name: str) -> int:
    """0 unit row, 1 BN pair, 2 RMS scale, 3 plain (layers.py:24-29, 57-64, 76-81)."""
    if name.endswith("mean_bias") or name.endswith("std_bias") or name == "predictor.bias":
        return 3
    if ".norm" in name or name.startswith("embedder.norm"):
        return 1
    if name.startswith("post_norm"):
        return 2
    return 0


class FusedOptimizer:
    """Adam + projection (+ EMA into the target copy) in one pass per step.

    Per-network scalar state (timestep, lr) lives on the device, as in
    robolearn/cuda/kernels.cu:310-337; the LR schedule is evaluated on the device
    before each step (robolearn/warp/flashsac.py:242-259, 645-649).
    """

    def __init__(self, store: FlatStore, cfg, *, project=True, ema_tau=None, plain=False, form=0,
                 schedule=True, kinds=None):
        """`kinds` optionally maps tensor names to projection kinds, overriding the name rule."""
        self.store = store
        device = store.param.device
        self.timestep = torch.zeros(1, device=device)
        self.lr = torch.full((1,), float(cfg.learning_rate_init), device=device)
        names = list(store.shapes)
        overrides = dict(kinds or {})
        kinds, rows, cols, params, grads, m1, m2, targets, partner = [], [], [], [], [], [], [], [], []
        index = {n: i for i, n in enumerate(names)}
        for name in names:
            shape = store.shapes[name]
            kind = 3 if (plain or not project) else overrides.get(name, projection_kind(name))
            if kind == 0:
                r, c = _numel(shape[:-1]), shape[-1]
            elif kind in (1, 2):
                r, c = _numel(shape[:-1]) if len(shape) > 1 else 1, shape[-1]
            else:
                r, c = 1, _numel(shape)
            kinds.append(kind)
            rows.append(r)
            cols.append(c)
            params.append(store.view(store.param, name).data_ptr())
            grads.append(store.view(store.grad, name).data_ptr())
            m1.append(store.view(store.m1, name).data_ptr())
            m2.append(store.view(store.m2, name).data_ptr())
            targets.append(store.view(store.target, name).data_ptr() if ema_tau is not None else None)
            partner.append(-1)
        for i, name in enumerate(names):
            if kinds[i] == 1 and name.endswith(".weight"):
                partner[i] = index[name[: -len("weight")] + "bias"]
        warmup, decay = cfg.learning_rate_warmup_step, cfg.learning_rate_decay_step
        self.handle = _native.create(
            "rl_fused_optimizer_create", len(names), _native.int_array(kinds), _native.ll_array(rows),
            _native.ll_array(cols), _native.pointer_array(params), _native.pointer_array(grads),
            _native.pointer_array(m1), _native.pointer_array(m2),
            _native.pointer_array(targets) if ema_tau is not None else None,
            _native.pointer_array([store.view(store.shadow, n).data_ptr() for n in names])
            if store.shadow is not None else None,
            _native.pointer_array([store.view(store.target_shadow, n).data_ptr() for n in names])
            if (store.target_shadow is not None and ema_tau is not None) else None,
            _native.int_array(partner),
            self.timestep.data_ptr(), self.lr.data_ptr(), 0.9, 0.999, 1e-8,
            float(ema_tau if ema_tau is not None else 0.0), form, int(schedule), float(cfg.learning_rate_init),
            float(cfg.learning_rate_peak), float(cfg.learning_rate_end), int(warmup), int(decay),
        )
        self.project = project and not plain
        self.ema = ema_tau is not None

    def step(self, *, adam=True, project=None, ema=None):
        project = self.project if project is None else project
        ema = self.ema if ema is None else ema
        _native.call("rl_fused_optimizer_step", self.handle, int(adam), int(project), int(ema), None, K.stream())
        if adam or project:
            self.store.refresh_transposed()

    def close(self):
        if getattr(self, "handle", None):
            try:
                _native.load().rl_fused_optimizer_destroy(self.handle)
            except Exception:  # interpreter shutdown
                pass
            self.handle = None

    def __del__(self):
        self.close()


class Trunk:
    """BN -> Linear embedder, residual BN blocks and the post RMSNorm, batched over members.

    In bf16 mode every GEMM operand is a bf16 tensor written by its producer
    (BN apply, RMS, GEMM epilogues, BN backward), so the GEMMs never convert;
    fp32 copies exist only where an fp32 consumer needs them (BN statistics,
    the residual stream, the BN backward inputs).
    """

    def __init__(self, *, ensemble, in_dim, hidden, blocks, max_rows, device, mode, prefix_linear,
                 bf16_activations=True):
        self.E, self.in_dim, self.h, self.blocks, self.R = ensemble, in_dim, hidden, blocks, max_rows
        self.mode = mode
        self.bf = mode == K.BF16
        self.linear = prefix_linear  # name suffix of unit-linear weights (".w.weight" actor, ".weight" critic)
        E, R, h = ensemble, max_rows, hidden
        # split-K partial sums for fp32 block products whose tile grid cannot fill the GPU (set by the
        # owner; bf16 block products keep their fused BatchNorm moments instead)
        self.workspace = None

        def buf(*shape):
            return torch.zeros(*shape, device=device)

        def half(*shape):
            return torch.zeros(*shape, dtype=torch.bfloat16, device=device) if self.bf else None

        def full(*shape):
            return None if self.bf else buf(*shape)

        # BatchNorm inputs and their gradients: bf16 in bf16 mode, as the Linear
        # outputs an autocast forward feeds the BatchNorm (the BN kernels need
        # channels in multiples of 4 for bf16 rows); bf16_activations=False keeps
        # them fp32 (bf16 GEMM operands with fp32 activations)
        narrow = self.bf and bf16_activations and h % 4 == 0
        self.bf16_activations = narrow

        def pre_norm(*shape):
            return torch.zeros(*shape, dtype=torch.bfloat16, device=device) if narrow else buf(*shape)

        self.y0, self.y0_h = full(E, R, in_dim), half(E, R, in_dim)
        self.stream = [buf(E, R, h) for _ in range(blocks + 1)]
        self.stream_h = [half(E, R, h) for _ in range(blocks + 1)]
        self.u1 = [pre_norm(E, R, 4 * h) for _ in range(blocks)]
        self.r1 = [full(E, R, 4 * h) for _ in range(blocks)]
        self.r1_h = [half(E, R, 4 * h) for _ in range(blocks)]
        self.u2 = [pre_norm(E, R, h) for _ in range(blocks)]
        self.z, self.z_h = full(E, R, h), half(E, R, h)
        self.ms = buf(E * R)
        self.stats = {}
        for name, width in self.bn_layers():
            self.stats[name] = (buf(E, width), buf(E, width))
        self.d_stream, self.d_stream_h = buf(E, R, h), half(E, R, h)
        self.d_u2, self.d_u2_h = full(E, R, h), half(E, R, h)
        # in bf16 mode the product writes the ReLU-BN gradient in bf16 and the BN
        # backward turns it into the input gradient in place
        self.d_r1 = pre_norm(E, R, 4 * h)
        self.d_r1_h = self.d_r1 if narrow else half(E, R, 4 * h)
        self.dy0 = buf(E, R, in_dim)
        self.dz = buf(E, R, h)
        widest = max(4 * h, in_dim)
        self.partial = buf(E * 2 * K.chunks(R) * widest)
        self.sums = buf(2 * E * widest)

    # operand views: bf16 tensors in bf16 mode, fp32 otherwise
    def op(self, fp32, bf16):
        return bf16 if self.bf else fp32

    @property
    def z_op(self):
        return self.op(self.z, self.z_h)

    def bn_layers(self):
        yield "embedder.norm", self.in_dim
        for i in range(self.blocks):
            yield f"encoder.{i}.norm1", 4 * self.h
            yield f"encoder.{i}.norm2", self.h

    def _stats(self, name, running, training):
        if training:
            return self.stats[name]
        return running[name + ".running_mean"], running[name + ".running_var"]

    def forward(self, p, w, running, x, *, rows, x_stride, training, update_running=True):
        """Runs the trunk on `rows` rows of x; leaves the block outputs in self.stream.

        p: fp32 parameter views (BN, RMS); w: GEMM weight views (bf16 shadows in bf16 mode).
        """
        E, h, mode = self.E, self.h, self.mode
        name = "embedder.norm"
        mean, var = self.stats[name]
        K.bn_forward(x, p[name + ".weight"], p[name + ".bias"], running[name + ".running_mean"],
                     running[name + ".running_var"], mean, var, self.partial, self.y0, rows=rows,
                     channels=self.in_dim, ensemble=E, x_stride=x_stride, training=training,
                     update_running=update_running, y_bf16=self.y0_h)
        K.gemm(self.op(self.y0, self.y0_h), w["embedder.w" + self.linear], self.stream[0], m=rows, n=h,
               k=self.in_dim, batch=E, a_kcontig=True, b_kcontig=True, lda=self.in_dim, ldb=self.in_dim, ldd=h,
               stride_a=rows * self.in_dim, stride_b=h * self.in_dim, stride_d=rows * h, mode=mode,
               d_bf16=self.stream_h[0])
        for i in range(self.blocks):
            pre = f"encoder.{i}"
            # in training the GEMM also writes the BatchNorm's chunk moments of its output
            moments = self.partial if training else None
            K.linear_forward(self.op(self.stream[i], self.stream_h[i]), w[f"{pre}.w1{self.linear}"], self.u1[i],
                             rows=rows, in_dim=h, out_dim=4 * h, ensemble=E, mode=mode, moments=moments,
                             workspace=None if self.bf else self.workspace)
            mean, var = self.stats[pre + ".norm1"]
            K.bn_forward(self.u1[i], p[pre + ".norm1.weight"], p[pre + ".norm1.bias"],
                         running[pre + ".norm1.running_mean"], running[pre + ".norm1.running_var"], mean, var,
                         self.partial, self.r1[i], rows=rows, channels=4 * h, ensemble=E, training=training,
                         relu=True, update_running=update_running, y_bf16=self.r1_h[i], moments_ready=training)
            K.linear_forward(self.op(self.r1[i], self.r1_h[i]), w[f"{pre}.w2{self.linear}"], self.u2[i], rows=rows,
                             in_dim=4 * h, out_dim=h, ensemble=E, mode=mode, moments=moments,
                             workspace=None if self.bf else self.workspace)
            mean, var = self.stats[pre + ".norm2"]
            K.bn_forward(self.u2[i], p[pre + ".norm2.weight"], p[pre + ".norm2.bias"],
                         running[pre + ".norm2.running_mean"], running[pre + ".norm2.running_var"], mean, var,
                         self.partial, self.stream[i + 1], rows=rows, channels=h, ensemble=E, training=training,
                         relu=True, update_running=update_running, residual=self.stream[i],
                         y_bf16=self.stream_h[i + 1], moments_ready=training)

    def post_norm(self, p, *, rows, row0, count):
        """RMSNorm of rows [row0, row0 + count) of the last block output into z (same rows)."""
        offset = row0 * self.h
        K.rms_forward(self.stream[-1].view(-1)[offset:], p["post_norm.weight"], self.ms,
                      None if self.bf else self.z.view(-1)[offset:], rows=count, channels=self.h, ensemble=self.E,
                      member_stride=rows * self.h, y_bf16=self.z_h.view(-1)[offset:] if self.bf else None)

    def post_norm_backward(self, p, g, *, rows, row0, count):
        """dz rows [row0, row0+count) -> d_stream (same rows, overwrite), RMS weight grad."""
        offset = row0 * self.h
        K.rms_backward(self.stream[-1].view(-1)[offset:], self.dz.view(-1)[offset:], p["post_norm.weight"], self.ms,
                       self.partial, self.d_stream.view(-1)[offset:],
                       None if g is None else g["post_norm.weight"], rows=count, channels=self.h, ensemble=self.E,
                       member_stride=rows * self.h)
        if count < rows:
            # rows outside the head subset receive no gradient from the head
            for e in range(self.E):
                base = self.d_stream.view(-1)[e * rows * self.h: (e + 1) * rows * self.h].view(rows, self.h)
                if row0 > 0:
                    K.fill(base[:row0], 0.0)
                if row0 + count < rows:
                    K.fill(base[row0 + count: rows], 0.0)
        if self.bf and self.blocks == 0:
            K.cast_bf16(self.d_stream.view(-1)[: self.E * rows * self.h], self.d_stream_h)

    def backward(self, p, w, running, g, x, *, rows, x_stride, training, workspace, input_grad=None, wt=None):
        """Backward from self.d_stream (gradient of the last block output).

        g: gradient views (None for a frozen network: only input gradients).
        input_grad: optional [E, rows, in_dim] buffer receiving dL/dx per member.
        wt: optional transposed block weights ([E, in, out], bf16) for the input-gradient products.
        """
        wt = wt or {}
        E, h, mode = self.E, self.h, self.mode
        for i in reversed(range(self.blocks)):
            pre = f"encoder.{i}"
            mean, var = self._stats(pre + ".norm2", running, training)
            K.bn_backward(self.u2[i], self.d_stream, None, p[pre + ".norm2.weight"], mean, var, self.partial,
                          self.sums, self.d_u2, None if g is None else g[pre + ".norm2.weight"],
                          None if g is None else g[pre + ".norm2.bias"], rows=rows, channels=h, ensemble=E,
                          training=training, relu=True, b=p[pre + ".norm2.bias"], dx_bf16=self.d_u2_h)
            d_u2 = self.op(self.d_u2, self.d_u2_h)
            K.linear_backward_input(d_u2, w[f"{pre}.w2{self.linear}"], self.d_r1, rows=rows, in_dim=4 * h,
                                    out_dim=h, ensemble=E, mode=mode, wt=wt.get(f"{pre}.w2{self.linear}"),
                                    workspace=workspace)
            if g is not None:
                K.linear_backward_weight(d_u2, self.op(self.r1[i], self.r1_h[i]), g[f"{pre}.w2{self.linear}"],
                                         rows=rows, in_dim=4 * h, out_dim=h, ensemble=E, mode=mode,
                                         workspace=workspace)
            mean, var = self._stats(pre + ".norm1", running, training)
            K.bn_backward(self.u1[i], self.d_r1, None, p[pre + ".norm1.weight"], mean, var, self.partial,
                          self.sums, None if self.bf else self.d_r1, None if g is None else g[pre + ".norm1.weight"],
                          None if g is None else g[pre + ".norm1.bias"], rows=rows, channels=4 * h, ensemble=E,
                          training=training, relu=True, b=p[pre + ".norm1.bias"], dx_bf16=self.d_r1_h)
            d_r1 = self.op(self.d_r1, self.d_r1_h)
            # the bf16 copy of d_stream is read only after the first block (by the embedder's
            # products); the blocks above read the fp32 stream gradient
            K.linear_backward_input(d_r1, w[f"{pre}.w1{self.linear}"], self.d_stream, rows=rows, in_dim=h,
                                    out_dim=4 * h, ensemble=E, mode=mode, c=self.d_stream, beta=1.0,
                                    d_bf16=self.d_stream_h if i == 0 else None,
                                    wt=wt.get(f"{pre}.w1{self.linear}"), workspace=workspace)
            if g is not None:
                K.linear_backward_weight(d_r1, self.op(self.stream[i], self.stream_h[i]), g[f"{pre}.w1{self.linear}"],
                                         rows=rows, in_dim=h, out_dim=4 * h, ensemble=E, mode=mode,
                                         workspace=workspace)
        d_stream = self.op(self.d_stream, self.d_stream_h)
        if g is not None:
            K.linear_backward_weight(d_stream, self.op(self.y0, self.y0_h), g["embedder.w" + self.linear], rows=rows,
                                     in_dim=self.in_dim, out_dim=h, ensemble=E, mode=mode, workspace=workspace)
        if g is None and input_grad is None:
            return
        K.linear_backward_input(d_stream, w["embedder.w" + self.linear], self.dy0, rows=rows, in_dim=self.in_dim,
                                out_dim=h, ensemble=E, mode=mode, workspace=workspace)
        name = "embedder.norm"
        mean, var = self._stats(name, running, training)
        K.bn_backward(x, self.dy0, None, p[name + ".weight"], mean, var, self.partial, self.sums, input_grad,
                      None if g is None else g[name + ".weight"], None if g is None else g[name + ".bias"],
                      rows=rows, channels=self.in_dim, ensemble=E, x_stride=x_stride, training=training)
