"""Shared comparison rules of the GPU parity tests (imported by the test modules; collects nothing).

Reference-relative tolerance.  Two rounding-decided effects move a correct fp32 update away from the
float64 one by far more than 1e-4 on some tensors:

* Adam's first step maps a gradient g to -lr g / (|g| + eps), so elements with |g| near eps move by an
  amount their rounding decides (up to 2 lr);
* ReLU masks: a FlashSAC update at the README shape has about 35 ReLU inputs within 1e-7 and 300
  within 1e-6 of zero (relative to their row's largest input), each passed or blocked by rounding,
  and one flipped element changes its row's gradient.

The reference's own fp32 path, run as the oracle in float32, shows both: on the same update with
its batch rows permuted (mathematically the same update; the BatchNorm statistics, and with them
every ReLU input, round differently) its gradient error against float64 falls either near 1e-5 or
near 3e-4 .. 2e-3 per tensor, depending on which near-zero inputs flip.  A GPU result is therefore
held to 1e-4 relative L2 against float64 or, where the float32 oracle errs more, to 3x the largest
error over an ensemble of float32 oracle runs (the original row order and seeded permutations).
"""

import torch


def rel(actual, reference):
    """(max-norm, L2) errors of actual against reference, relative to the reference's max and L2 norms."""
    actual = torch.as_tensor(actual).double().reshape(-1)
    reference = torch.as_tensor(reference).double().reshape(-1)
    diff = actual - reference
    return (diff.abs().max().item() / max(reference.abs().max().item(), 1e-30),
            diff.norm().item() / max(reference.norm().item(), 1e-30))


def compare(label, gpu_values, cpu_values, reference, report, check=True):
    """Per tensor: the GPU's relative L2 error against `reference` (float64) may exceed 1e-4 only where
    the float32 oracle's does, and then by at most 3x the largest error over `cpu_values` (one dict or a
    list of dicts: float32 oracle runs).  Appends (label, name, GPU max, fp32 max, GPU L2, fp32 L2)
    rows to `report`; returns the worst error / allowance ratio (asserted <= 1 when `check`)."""
    runs = cpu_values if isinstance(cpu_values, (list, tuple)) else [cpu_values]
    worst = 0.0
    for name, ref in reference.items():
        gpu_max, gpu_l2 = rel(gpu_values[name], ref)
        errors = [rel(run[name], ref) for run in runs]
        cpu_max, cpu_l2 = max(e[0] for e in errors), max(e[1] for e in errors)
        report.append((label, name, gpu_max, cpu_max, gpu_l2, cpu_l2))
        allowed = max(1e-4, 3.0 * cpu_l2)
        worst = max(worst, gpu_l2 / allowed)
        assert not check or gpu_l2 <= allowed, (label, name, gpu_l2, cpu_l2)
    return worst


def permuted(batch, actor_noise, next_noise, seed):
    """The same update's inputs with the batch rows permuted (seeded): batch fields and next-action
    noise by row, the actor noise's two halves (current and next observations) by the same row map."""
    import numpy as np

    rows = next_noise.shape[0]
    perm = torch.as_tensor(np.random.default_rng(seed).permutation(rows))
    batch = {k: torch.as_tensor(v)[perm] for k, v in batch.items()}
    actor_noise = torch.cat([actor_noise[:rows][perm], actor_noise[rows:][perm]])
    return batch, actor_noise, next_noise[perm]


def delta_stats(before, after, reference):
    """The reference's delta policy (examples/diagnose_warp_flashsac.py:114-129) per parameter tensor:
    (max error of the change, bound 5e-7 + 0.02 max|reference change|, elements beyond it, L2 error)."""
    stats = {}
    for key, expected in reference.items():
        if "running" in key:
            continue
        actual = torch.as_tensor(after[key]).double()
        delta_ref = expected.double() - before[key].double()
        err = (actual - before[key].double() - delta_ref).abs()
        bound = 5e-7 + 0.02 * delta_ref.abs().max().item()
        stats[key] = (err.max().item(), bound, int((err > bound).sum()), err.norm().item())
    return stats


class DeviceReluRecorder:
    """Records, after every Trunk.forward of the learner, what its ReLU decisions depend on, so the
    oracle can be run with the same decisions (oracle.flashsac.Emulation(relu_masks=...)).

    Per block and BatchNorm (norm1, norm2): the BatchNorm input the device stored (u1, u2, fp32 or
    bf16), the statistics it normalized with (the batch's in training, the running ones in eval),
    the BN weight and bias, and (norm1) the post-ReLU output it stored.  ``masks()`` replays the
    device's decision bn_value(x) > 0 of csrc/norm.hip exactly: t = fp32((x - mean) * inv) with
    inv = 1 / sqrt(var + eps) in IEEE fp32, then the sign of the fused t * w + b, which float64
    evaluates exactly (the product is exact and rounding preserves the sign).  Each norm1 decision
    is checked against the sign of the stored post-ReLU output, so a replay that differs from the
    device fails loudly.  Use as a context manager around the device update."""

    def __init__(self, eps=1e-5):
        self.eps = eps
        self.records = []

    def __enter__(self):
        from robolearn_amd import networks

        self._networks = networks
        self._original = networks.Trunk.forward
        recorder = self

        def forward(trunk, p, w, running, x, *, rows, x_stride, training, update_running=True):
            recorder._original(trunk, p, w, running, x, rows=rows, x_stride=x_stride, training=training,
                               update_running=update_running)
            recorder._snapshot(trunk, p, running, rows, training)

        networks.Trunk.forward = forward
        return self

    def __exit__(self, *exc):
        self._networks.Trunk.forward = self._original
        return False

    def _snapshot(self, trunk, p, running, rows, training):
        E, h = trunk.E, trunk.h
        packed = lambda t, c: t.reshape(-1)[: E * rows * c].view(E, rows, c).clone()  # noqa: E731
        layers = []
        for i in range(trunk.blocks):
            pre = f"encoder.{i}"
            for j, (u, c) in enumerate(((trunk.u1[i], 4 * h), (trunk.u2[i], h))):
                name = f"{pre}.norm{j + 1}"
                mean, var = trunk._stats(name, running, training)
                post = None
                if j == 0:
                    post = packed(trunk.r1_h[i] if trunk.bf else trunk.r1[i], c)
                layers.append(dict(u=packed(u, c), mean=mean.reshape(E, c).clone(), var=var.reshape(E, c).clone(),
                                   w=p[name + ".weight"].reshape(E, c).clone(), b=p[name + ".bias"].reshape(E, c).clone(),
                                   post=post))
        self.records.append(dict(ensemble=E, layers=layers))

    def masks(self):
        """The recorded decisions in the oracle's ReLU order, shaped [R, C] (actor) or [2, R, C]."""
        import numpy as np

        out, mismatches = [], 0
        for record in self.records:
            for layer in record["layers"]:
                x = layer["u"].float().cpu().numpy()
                mean = layer["mean"].cpu().numpy().astype(np.float32)[:, None, :]
                var = layer["var"].cpu().numpy().astype(np.float32)[:, None, :]
                inv = np.float32(1.0) / np.sqrt(var + np.float32(self.eps))
                t = (x - mean) * inv
                y = t.astype(np.float64) * layer["w"].cpu().double().numpy()[:, None, :] + \
                    layer["b"].cpu().double().numpy()[:, None, :]
                mask = torch.as_tensor(y > 0)
                if layer["post"] is not None:
                    mismatches += int((mask != (layer["post"].float().cpu() > 0)).sum())
                out.append(mask[0] if record["ensemble"] == 1 else mask)
        assert mismatches == 0, f"{mismatches} replayed ReLU decisions differ from the device's stored outputs"
        return out


def load_device_optimizer(oracle, state):
    """Adam moments, step counts and learning rates of a device state_dict into the oracle's optimizers
    (same parameter order: the learner's stores follow the reference's named_parameters order), so an
    update after the first continues from the device's optimizer state."""
    for label, params in (("actor", list(oracle.actor.values())), ("critic", list(oracle.critic.values())),
                          ("temperature", [oracle.log_temp])):
        optimizer, scheduler = oracle.optimizers[label], oracle.schedulers[label]
        steps = float(torch.as_tensor(state[f"optimizer.{label}.timestep"]).reshape(-1)[0])
        for i, p in enumerate(params):
            optimizer.state[p] = {
                "step": torch.tensor(steps),
                "exp_avg": torch.as_tensor(state[f"optimizer.{label}.m1.{i}"]).reshape(p.shape).to(p.dtype).clone(),
                "exp_avg_sq": torch.as_tensor(state[f"optimizer.{label}.m2.{i}"]).reshape(p.shape).to(p.dtype).clone(),
            }
        scheduler.last_epoch = int(steps)
        for group in optimizer.param_groups:
            group["lr"] = float(torch.as_tensor(state[f"optimizer.{label}.lr"]).reshape(-1)[0])


def teacher_after_actor_phase(agent):
    """An oracle.flashsac.Emulation after_actor_phase hook that loads the device's post-step actor,
    its actor BatchNorm running statistics and its log-temperature into the oracle state, so the
    critic phase is compared from the device's own start (the steps themselves are checked apart)."""
    state = agent.state_dict(include_replay=False)

    def hook(oracle_state):
        with torch.no_grad():
            for name, value in list(oracle_state.actor.items()) + list(oracle_state.actor_buffers.items()):
                value.copy_(torch.as_tensor(state[f"actor.{name}"]).reshape(value.shape).to(value.dtype))
            oracle_state.log_temp.copy_(torch.as_tensor(state["log_temperature"]).reshape(1).to(oracle_state.dtype))

    return hook


def forced_update_check(agent, batch, actor_noise, next_noise, *, bound, label, actor_phase=True):
    """One device update (update_from_batch) against the float64 oracle run with the device's ReLU
    decisions (DeviceReluRecorder), the device's bf16 roundings when the agent runs bf16 operands
    (oracle.flashsac.Emulation), and the device's post-step actor and temperature loaded before the
    critic phase.  Asserts, per tensor, for the actor, critic and temperature gradients and every Adam
    moment, and for the metrics: relative L2 <= max(bound, 3 x the error of the same oracle run in
    float32).  The float32 run is the reference's own update at fp32 accumulation under the same
    decisions and roundings; it sits near 1e-5 in fp32 mode, so there the bound decides, and near 1e-2
    in bf16 mode, where each bf16 rounding of a value within fp32 accumulation error of a rounding
    midpoint goes either way and the training-mode BatchNorm backward amplifies the difference.
    Returns the worst error / allowance ratio, the float64 record and the pre-update state."""
    from oracle import flashsac as O

    state0 = agent.state_dict(include_replay=False)
    with DeviceReluRecorder() as recorder:
        metrics = agent.update_from_batch({k: torch.as_tensor(v).numpy() for k, v in batch.items()},
                                          actor_noise=torch.as_tensor(actor_noise).numpy(),
                                          next_noise=torch.as_tensor(next_noise).numpy(),
                                          do_actor_update=actor_phase, tensor_metrics=False)
        torch.cuda.synchronize()
    masks = recorder.masks()
    d = O.dims_from_config(agent.observation_dim, agent.action_dim, agent.cfg, agent.critic_observation_dim)
    runs, records = {}, {}
    for dtype in (torch.float64, torch.float32):
        oracle = O.OracleState(d, agent.cfg, dtype=dtype)
        oracle.load_flat(dict(state0))
        load_device_optimizer(oracle, state0)
        emulation = O.Emulation(relu_masks=masks, bf16=agent.cfg.use_amp, bf16_activations=agent.bf16_activations,
                                after_actor_phase=teacher_after_actor_phase(agent))
        record = {}
        info = O.update(oracle, batch, actor_noise, next_noise, do_actor_update=actor_phase, record=record,
                        emulation=emulation)
        assert emulation.used == len(masks), (emulation.used, len(masks))
        values = {f"metric {k}": torch.tensor([float(v)], dtype=torch.float64) for k, v in info.items()}
        if actor_phase:
            values.update({f"actor grad {k}": v for k, v in record["actor_grads"].items()})
            values["temperature grad"] = record["temperature_grad"]
        values.update({f"critic grad {k}": v for k, v in record["critic_grads"].items()})
        moments = oracle.moments()
        for key, value in moments.items():
            if key.startswith("actor.") and not actor_phase:
                continue
            values[key] = value
        runs[dtype], records[dtype] = values, record
    device = {f"metric {k}": torch.tensor([float(v)]) for k, v in metrics.items()}
    if actor_phase:
        device.update({f"actor grad {k}": v for k, v in agent.actor.grads().items()})
        device["temperature grad"] = agent.temperature.grad[:1]
    device.update({f"critic grad {k}": v for k, v in agent.critic.grads().items()})
    for net_label, store in (("actor", agent.actor), ("critic", agent.critic), ("temperature", agent.temperature)):
        m1, m2 = store.moments()
        for name in store.shapes:
            key = "temperature" if net_label == "temperature" else f"{net_label}.{name}"
            device[f"{key}.m1"], device[f"{key}.m2"] = m1[name], m2[name]
    reference, fp32 = runs[torch.float64], runs[torch.float32]
    rows = []
    for key, ref in reference.items():
        gpu_err = rel(device[key].detach().cpu(), ref)[1]
        cpu_err = rel(fp32[key], ref)[1]
        allowed = max(bound, 3.0 * cpu_err)
        rows.append((key, gpu_err, cpu_err, allowed))
    rows.sort(key=lambda r: -r[1] / r[3])
    print(f"{label}: {len(masks)} ReLU layers forced; relative L2 against float64 (allowed max({bound:g}, "
          f"3 x float32 oracle)):", flush=True)
    for key, gpu_err, cpu_err, allowed in rows[:8]:
        print(f"  {key:48s} device {gpu_err:.2e}  float32 oracle {cpu_err:.2e}  allowed {allowed:.2e}", flush=True)
    worst = max(r[1] / r[3] for r in rows)
    for key, gpu_err, cpu_err, allowed in rows:
        assert gpu_err <= allowed, (label, key, gpu_err, cpu_err)
    return worst, records[torch.float64], state0

