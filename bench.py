#!/usr/bin/env python3
"""Learner hot-path benchmark on one MI355X.

Default workload ("g1"): one captured HIP graph per
step holding two FlashSAC updates (update-to-data 2: an actor+critic update and
a critic-only update) at batch 8192, obs 123, act 37, actor 256x2, twin critics
1024x2, 101 bins on [-20, 20], bf16 dense operands with fp32 state; replay
4096 envs x 256 steps of seeded synthetic transitions resident in HBM.

Prints ONE JSON line: value = FlashSAC updates/sec on the GPU, with
  roofline      the dominant kernel (critic block-1 forward GEMM, bf16 MFMA)
                timed live with HIP events on the stream it runs on,
  update_roofline  two-term serial roofline of the whole update,
  cpu_baseline  the CPU oracle (PyTorch-CPU restatement of the reference update,
                fp32) timed on this host's cores on one update of the same shape,
  ppo           PPO update ms at configs[3] (one captured graph per update;
                fp32-accurate products on the bf16 matrix cores, roofline at
                the bf16 peak / 6; CPU oracle on one epoch scaled to five),
  kernel_sweep  configs[4]: fused categorical target + CE, fused optimizer and
                RMSNorm at their sweep shapes against the HBM roofline, plus the
                replay ingest (n-step commit), return statistics and act()
                (fp32 actor + exploration repeat) of one vector step at the G1
                collection shape.
"""

import argparse
import json
import math
import os
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
TRAFFIC_PROFILE = ROOT / "profiles" / "gemm_dma_critic_fwd_g1_traffic.md"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP32_PEAK_TFLOPS = 157.3

WORKLOADS = {
    "g1": dict(obs=123, act=37, batch=8192, envs=4096, horizon=256, actor_hidden=256, actor_blocks=2,
               critic_hidden=1024, critic_blocks=2, bins=101, min_v=-20.0, max_v=20.0, amp=True, utd=2,
               reward_std=0.5, done=0.005),
    "readme": dict(obs=31, act=8, batch=2048, envs=1024, horizon=1000, actor_hidden=256, actor_blocks=1,
                   critic_hidden=512, critic_blocks=2, bins=101, min_v=-10.0, max_v=10.0, amp=False, utd=2,
                   reward_std=1.0, done=0.01),
    "cartpole": dict(obs=4, act=1, batch=512, envs=64, horizon=500, actor_hidden=128, actor_blocks=1,
                     critic_hidden=256, critic_blocks=2, bins=101, min_v=-10.0, max_v=10.0, amp=False, utd=2,
                     reward_std=1.0, done=0.01),
}


def gemm_flops(w: dict) -> float:
    """Algorithmic GEMM FLOPs (2 M N K per product) of one actor-phase + one critic-only update.

    Counts forward, input-gradient and weight-gradient products actually needed:
    the actor embedder needs no input gradient; the frozen critic in the actor
    phase needs input gradients only; heads run on the rows whose outputs are used.
    """
    B, O, A = w["batch"], w["obs"], w["act"]
    I = O + A
    ha, hc, K = w["actor_hidden"], w["critic_hidden"], w["bins"]

    def trunk(rows, inp, h, blocks, members):
        embed = members * 2 * rows * inp * h
        body = members * 2 * rows * blocks * 2 * h * 4 * h
        return embed, body

    def actor(rows):
        e, b = trunk(rows, O, ha, w["actor_blocks"], 1)
        return e, b + 2 * rows * ha * 2 * A

    def critic_trunk(rows):
        return trunk(rows, I, hc, w["critic_blocks"], 2)

    def head(rows):
        return 2 * 2 * rows * hc * K

    ae, ab = actor(2 * B)
    ce_b, cb_b = critic_trunk(B)
    actor_phase = (ae + ab) + (ce_b + cb_b + head(B)) * 2 + (ae + ab) + ab
    ae1, ab1 = actor(B)
    ce, cb = critic_trunk(2 * B)
    critic_phase = (ae1 + ab1) + 2 * (ce + cb + head(B)) + (ce + cb + head(B)) + (cb + head(B))
    return actor_phase + 2 * critic_phase


def elementwise_bytes(w: dict, act_bytes: int = 4) -> float:
    """Approximate compulsory HBM bytes of the non-GEMM kernels for the same update pair.

    act_bytes: bytes per BatchNorm input / gradient element (2 when the bf16 path stores them
    in bf16; its producing GEMM also writes the statistics, so the forward has no stats read)."""
    B, hc, ha, K = w["batch"], w["critic_hidden"], w["actor_hidden"], w["bins"]
    per_block = 2 * 2 * B * (4 * hc + hc)  # members x rows x channels of one critic block
    stats_read = 0 if act_bytes == 2 else 1
    bn_fwd = (2 + stats_read) * act_bytes * per_block * w["critic_blocks"]  # (stats read +) apply read + write
    bn_bwd = 5 * act_bytes * per_block * w["critic_blocks"]  # partials read x, dy; apply read x, dy, write dx
    critic_pass = bn_fwd
    critic_total = 2 * critic_pass * 2 + bn_bwd * 2 + bn_bwd  # 2 updates x (target + online) fwd, bwd
    actor_bytes = 10 * 4 * 2 * B * 5 * ha * w["actor_blocks"]
    params = 2 * (w["critic_hidden"] * (w["obs"] + w["act"]) + w["critic_blocks"] * 8 * hc * hc + hc * K)
    optimizer = 36 * params * 2
    return critic_total + actor_bytes + optimizer + 3 * 2 * B * K * 4 * 4


def measured_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 --pmc summary, if it covers this kernel.

    The summary holds a `kernel:` line naming the launch and a
    `traffic_bytes_per_launch:` line (FETCH_SIZE + WRITE_SIZE, each scaled by a
    plain copy of known size); a summary for another kernel or shape is ignored.
    """
    try:
        text = TRAFFIC_PROFILE.read_text()
    except OSError:
        return None
    named = re.search(r"^kernel: (.+)$", text, flags=re.M)
    value = re.search(r"^traffic_bytes_per_launch: (\d+)$", text, flags=re.M)
    if named is None or value is None or named.group(1).strip() != kernel:
        return None
    return int(value.group(1))


def cpu_baseline(w: dict, cfg_kwargs: dict) -> dict:
    """Time the CPU oracle (fp32) on one actor-phase update at the workload shape."""
    import torch

    from oracle import flashsac as O
    from robolearn_amd.config import FlashSACConfig
    from dataclasses import replace

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    cfg = FlashSACConfig(**cfg_kwargs)
    cfg = replace(cfg, temp_target_entropy=O.target_entropy(w["act"], cfg.temp_target_sigma))
    d = O.dims_from_config(w["obs"], w["act"], cfg)
    state = O.init_state(d, cfg, seed=0, dtype=torch.float32)
    g = torch.Generator().manual_seed(5)
    B = w["batch"]
    batch = {
        "observation": torch.randn(B, w["obs"], generator=g), "next_observation": torch.randn(B, w["obs"], generator=g),
        "action": torch.rand(B, w["act"], generator=g) * 2 - 1, "reward": torch.randn(B, generator=g),
        "terminated": (torch.rand(B, generator=g) < w["done"]).float(), "discount": torch.full((B,), cfg.gamma),
    }
    noise = torch.randn(2 * B, w["act"], generator=g)
    next_noise = torch.randn(B, w["act"], generator=g)
    O.update(state, batch, noise, next_noise, do_actor_update=False)  # warm-up (critic-only)
    t0 = time.perf_counter()
    O.update(state, batch, noise, next_noise, do_actor_update=True)
    actor_seconds = time.perf_counter() - t0
    t0 = time.perf_counter()
    O.update(state, batch, noise, next_noise, do_actor_update=False)
    critic_seconds = time.perf_counter() - t0
    per_update = 0.5 * (actor_seconds + critic_seconds)
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as stream:
            for line in stream:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {
        "value": 1.0 / per_update,
        "unit": "updates/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"oracle.flashsac (PyTorch CPU fp32) at the same shape: 1 critic-only warm-up, then 1 actor-phase "
                   f"({actor_seconds:.2f} s) + 1 critic-only ({critic_seconds:.2f} s) update timed; {model}"),
    }


PPO_C3 = dict(envs=4096, horizon=24, obs=123, act=37, hidden=(512, 256, 128))


def ppo_config(**overrides):
    """The c3 PPO recipe (warp/config.py fields; ELU MLPs 512-256-128, adaptive KL)."""
    from robolearn_amd.config import PPOConfig

    fields = dict(hidden_dims=PPO_C3["hidden"], activation="elu", std_type="log", epochs=5, num_mini_batches=4,
                  clip_ratio=0.2, clip_value=True, entropy_coefficient=0.005, schedule="adaptive", desired_kl=0.01,
                  gamma=0.99, gae_lambda=0.95)
    fields.update(overrides)
    return PPOConfig(**fields)


def ppo_flops(cfg) -> float:
    """2 M N K summed over forward, weight- and input-gradient products of both MLPs, all epochs."""
    rows = PPO_C3["envs"] * PPO_C3["horizon"] * cfg.epochs
    total = 0
    for out in (PPO_C3["act"], 1):
        widths = [PPO_C3["obs"], *cfg.hidden_dims, out]
        layers = list(zip(widths[:-1], widths[1:]))
        total += 2 * sum(2 * i * o for i, o in layers) + sum(2 * i * o for i, o in layers[1:])
    return float(rows * total)


def ppo_rollout(agent, seed=0):
    """Synthetic c3 rollout on the device: obs, values ~ N(0,1); actions = mu(obs) + sigma*eps with their
    Gaussian log-probs; rewards ~ N(0,1); terminated ~ Bernoulli(1/1000); no truncations."""
    import torch

    n = agent.batch_size
    torch.manual_seed(seed)
    obs = torch.randn(n, agent.observation_dim, device=agent.device)
    actions = agent.act(obs)
    sampled = agent._act_state(n)
    agent.observations.copy_(obs)
    agent.actions.copy_(actions)
    agent.log_probs.copy_(sampled["log_probs"])
    agent.means.copy_(sampled["mean"])
    agent.stds.copy_(sampled["std"].expand(n, -1))
    agent.values.copy_(torch.randn(n, device=agent.device))
    agent.next_values.copy_(torch.randn(n, device=agent.device))
    agent.rewards.copy_(torch.randn(n, device=agent.device))
    agent.terminated.copy_((torch.rand(n, device=agent.device) < 1e-3).int())
    agent.truncated.zero_()


def bench_ppo(steps: int, warmup: int, with_cpu: bool) -> dict:
    """PPO update ms at c3: one captured graph (GAE, permutation, 5 epochs x 4 minibatches) per update."""
    import torch

    from robolearn_amd import kernels as K
    from robolearn_amd.ppo import WarpPPO

    cfg = ppo_config()
    agent = WarpPPO(PPO_C3["obs"], PPO_C3["act"], PPO_C3["envs"], PPO_C3["horizon"], cfg)
    ppo_rollout(agent)
    initial = agent.state_dict() if with_cpu else None
    agent.update()  # captures the graph (after an eager warm-up that restores the state)
    for _ in range(warmup):
        agent.update()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        agent.update()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    flops = ppo_flops(cfg)
    achieved = flops / (ms * 1e-3) / 1e12
    split = agent.gemm_mode == K.FP32_SPLIT
    # fp32-accurate products on the bf16 matrix cores cost six bf16 products per fp32 product
    peak = BF16_PEAK_TFLOPS / 6.0 if split else FP32_PEAK_TFLOPS
    result = {
        "metric": "PPO update ms", "value": round(ms, 4), "unit": "ms/update", "higher_is_better": False,
        "dtype": "fp32", "steps": steps, "warmup": warmup,
        "config": {"workload": "ppo_c3", "envs": PPO_C3["envs"], "horizon": PPO_C3["horizon"],
                   "obs_dim": PPO_C3["obs"], "act_dim": PPO_C3["act"], "hidden": list(cfg.hidden_dims),
                   "activation": cfg.activation, "epochs": cfg.epochs, "minibatches": cfg.num_mini_batches,
                   "schedule": cfg.schedule, "desired_kl": cfg.desired_kl},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": round(peak, 1), "unit": "TFLOP/s",
                     "frac": round(achieved / peak, 4), "flops_per_update": flops,
                     "products": ("fp32-accurate: three-piece bf16 splits, 6 bf16 MFMA products per fp32 product; "
                                  "peak = bf16 dense peak / 6") if split else "v_mfma_f32_32x32x2_f32"},
        "cpu_baseline": None,
    }
    if with_cpu:
        result["cpu_baseline"] = ppo_cpu_baseline(agent, initial)
    del agent
    return result


def ppo_cpu_baseline(agent, initial: dict) -> dict:
    """The CPU oracle (fp32) on one epoch of the same rollout (4 minibatch steps), scaled to 5 epochs."""
    import numpy as np
    import torch

    from oracle import ppo as OP

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    cfg = ppo_config(epochs=1)
    rollout = {name: getattr(agent, name).cpu().numpy() for name in
               ("observations", "actions", "means", "stds", "values", "log_probs", "rewards", "next_values",
                "terminated", "truncated")}
    layers = [initial[f"parameter_{i}"] for i in range(len(agent.parameters))]
    oracle = OP.PPOOracle(PPO_C3["obs"], PPO_C3["act"], PPO_C3["envs"], PPO_C3["horizon"], cfg, layers,
                          dtype=torch.float32)
    permutation = np.random.default_rng(0).permutation(agent.batch_size)
    t0 = time.perf_counter()
    oracle.update(rollout, permutation)
    seconds = time.perf_counter() - t0
    epochs = ppo_config().epochs
    return {"value": round(seconds * epochs * 1e3, 1), "unit": "ms/update", "cores": threads, "kind": "port",
            "sample": f"oracle.ppo (PyTorch CPU fp32): GAE + 1 epoch x 4 minibatches timed ({seconds:.2f} s), "
                      f"scaled x{epochs} epochs"}


def _time_launches(launch, reps: int = 20) -> float:
    import torch

    launch()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        launch()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / reps


def _hbm_line(name: str, ms: float, algorithmic_bytes: float, detail: str) -> dict:
    achieved = algorithmic_bytes / (ms * 1e-3) / 1e9
    return {"kernel": name, "ms": round(ms, 4), "algorithmic_bytes": int(algorithmic_bytes),
            "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "detail": detail}


def kernel_sweep() -> list:
    """c4: the HBM-bound kernels at their sweep shapes, each timed over 20 launches with HIP events."""
    from collections import OrderedDict

    import torch

    from robolearn_amd import kernels as K
    from robolearn_amd.config import FlashSACConfig
    from robolearn_amd.networks import FlatStore, FusedOptimizer

    device = torch.device("cuda:0")
    g = torch.Generator(device=device).manual_seed(11)
    lines = []

    # (a) fused categorical TD target + cross-entropy, 65536 rows x 101 bins, twin critics
    B, bins = 65536, 101
    target_logits = torch.randn(2, B, bins, generator=g, device=device)
    online_logits = torch.randn(2, B, bins, generator=g, device=device)
    support = torch.linspace(-10.0, 10.0, bins, device=device)
    reward = torch.randn(B, generator=g, device=device) * 5.0
    terminated = (torch.rand(B, generator=g, device=device) < 0.01).float()
    discount = torch.full((B,), 0.99, device=device)
    next_log_probs = torch.randn(B, generator=g, device=device)
    alpha = torch.full((1,), 0.01, device=device)
    dlogits = torch.empty(2, B, bins, device=device)
    loss_rows, entropy_rows = torch.empty(2, B, device=device), torch.empty(B, device=device)

    def categorical():
        K.td_cross_entropy(target_logits, None, B, online_logits, None, B, support, reward, terminated, discount,
                           next_log_probs, alpha, min_v=-10.0, max_v=10.0, batch=B, bins=bins, scale=1.0 / B,
                           dlogits=dlogits, loss_rows=loss_rows, entropy_rows=entropy_rows)

    ms = _time_launches(categorical)
    lines.append(_hbm_line("td_cross_entropy", ms, B * (6 * bins * 4 + 28),
                           "65536 rows x 101 bins, 2 critics: read target + online logits, write d-logits"))

    # (b) fused Adam + unit-row projection + EMA over 48 tensors (~25.2M fp32 parameters)
    shapes, kinds = OrderedDict(), {}
    for i in range(24):
        out, inp = ((1024, 1024), (4096, 256))[i % 2]
        shapes[f"layer{i}.weight"] = (out, inp)
        shapes[f"layer{i}.bias"] = (out,)
        kinds[f"layer{i}.weight"], kinds[f"layer{i}.bias"] = 0, 3
    store = FlatStore(shapes, device, target=True)
    count = sum(math.prod(s) for s in shapes.values())
    store.param.normal_(0.0, 0.05, generator=g)
    store.target.copy_(store.param)
    store.grad.normal_(0.0, 1e-3, generator=g)
    store.m1.normal_(0.0, 1e-4, generator=g)
    store.m2.copy_(store.m1 * store.m1)
    cfg = FlashSACConfig(learning_rate_init=3e-4, learning_rate_peak=3e-4, learning_rate_end=3e-4)
    optimizer = FusedOptimizer(store, cfg, ema_tau=0.005, kinds=kinds)
    ms = _time_launches(lambda: optimizer.step(adam=True, project=True, ema=True))
    lines.append(_hbm_line("fused_optimizer step_kernel", ms, 36 * count,
                           f"48 tensors, {count} params: read p, g, m1, m2, target; write p, m1, m2, target"))
    optimizer.close()
    del store, optimizer

    # (c) RMSNorm forward + backward, 65536 x 1024
    rows, channels = 65536, 1024
    x = torch.randn(rows, channels, generator=g, device=device)
    w = torch.rand(channels, generator=g, device=device) + 0.5
    dy = torch.randn(rows, channels, generator=g, device=device)
    y, dx = torch.empty_like(x), torch.empty_like(x)
    ms_buf = torch.empty(rows, device=device)
    dw = torch.empty(channels, device=device)
    partial = torch.empty(K.chunks(rows) * channels, device=device)
    ms = _time_launches(lambda: K.rms_forward(x, w, ms_buf, y, rows=rows, channels=channels))
    lines.append(_hbm_line("rms_forward", ms, 2 * rows * channels * 4 + rows * 4,
                           "65536 x 1024: read x, write y and the per-row mean square"))
    ms = _time_launches(lambda: K.rms_backward(x, dy, w, ms_buf, partial, dx, dw, rows=rows, channels=channels))
    lines.append(_hbm_line("rms_backward (rms_backward_fused + column_reduce)", ms,
                           3 * rows * channels * 4 + rows * 4,
                           "65536 x 1024: read x, dy (and ms), write dx; weight gradient reduced in fixed order"))
    del x, dy, y, dx, partial

    # (d) replay ingest of one vector step at the G1 collection shape: 4096 environments,
    # obs 123, action 37, n_step 3, into a 1,048,576-row ring; then the return statistics
    from robolearn_amd import _native

    envs, obs_dim, act_dim, n_step, capacity = 4096, 123, 37, 3, 1 << 20
    step_in = [torch.randn(envs, obs_dim, generator=g, device=device),
               torch.rand(envs, act_dim, generator=g, device=device) * 2 - 1,
               torch.randn(envs, generator=g, device=device),
               (torch.rand(envs, generator=g, device=device) < 0.005).float(),
               torch.zeros(envs, device=device),
               torch.randn(envs, obs_dim, generator=g, device=device)]
    pending = [torch.zeros(n_step, envs, obs_dim, device=device), torch.zeros(n_step, envs, act_dim, device=device),
               torch.zeros(n_step, envs, obs_dim, device=device), torch.zeros(n_step, envs, 3, device=device)]
    store = [torch.zeros(capacity, obs_dim, device=device), torch.zeros(capacity, act_dim, device=device),
             *[torch.zeros(capacity, device=device) for _ in range(3)],
             torch.zeros(capacity, obs_dim, device=device), torch.zeros(capacity, device=device)]
    counters = torch.zeros(3, dtype=torch.long, device=device)

    def ingest():
        _native.call("rl_replay_ingest", envs, obs_dim, act_dim, n_step, capacity, 0.99,
                     *[t.data_ptr() for t in step_in], *[t.data_ptr() for t in pending],
                     *[t.data_ptr() for t in store], counters.data_ptr(), K.stream())

    row = 2 * obs_dim + act_dim
    ingest_bytes = envs * 4 * ((row + 3) * 2 + (row + 3 * (n_step - 1)) + (row + 4))
    ms = _time_launches(ingest)
    lines.append(_hbm_line("replay_ingest (ingest_kernel + advance_kernel)", ms, ingest_bytes,
                           "4096 envs, obs 123, act 37, n_step 3: stage the step, commit the oldest n-step return; "
                           "two launches, latency-bound at this size"))
    returns, maximum = torch.zeros(envs, device=device), torch.zeros(1, device=device)
    running = torch.tensor([0.0, 1.0, 0.0], device=device)
    ms = _time_launches(lambda: _native.call("rl_reward_stats_update", envs, 0.99, step_in[2].data_ptr(),
                                             step_in[3].data_ptr(), step_in[4].data_ptr(), returns.data_ptr(),
                                             maximum.data_ptr(), running.data_ptr(), K.stream()))
    lines.append(_hbm_line("reward_stats_update", ms, envs * 4 * 5,
                           "4096 envs: per-environment returns, running max and RunningMeanStd merge; "
                           "one workgroup, latency-bound"))
    del store, pending

    # (e) act(training=True) at the G1 collection shape: fp32 eval-mode actor (256 x 2 blocks) over
    # 4096 environments plus the exploration-noise repeat; the critics are irrelevant here and kept small
    from robolearn_amd.flashsac import FlashSAC

    act_cfg = FlashSACConfig(actor_hidden_dim=256, actor_num_blocks=2, critic_hidden_dim=32, critic_num_blocks=1,
                             sample_batch_size=256, buffer_max_length=1024, buffer_min_length=256)
    actor_agent = FlashSAC(obs_dim, act_dim, num_envs=envs, cfg=act_cfg)
    observations = torch.randn(envs, obs_dim, generator=g, device=device)
    ms = _time_launches(lambda: actor_agent.act(observations, training=True))
    h = act_cfg.actor_hidden_dim
    flops = 2 * envs * (obs_dim * h + act_cfg.actor_num_blocks * 2 * h * 4 * h + h * 2 * act_dim)
    achieved = flops / (ms * 1e-3) / 1e12
    lines.append({"kernel": "act (fp32 actor forward + exploration repeat)", "ms": round(ms, 4),
                  "flops": int(flops), "bound": "mfma", "achieved": round(achieved, 2), "peak": FP32_PEAK_TFLOPS,
                  "unit": "TFLOP/s", "frac": round(achieved / FP32_PEAK_TFLOPS, 4),
                  "detail": "4096 envs, obs 123, act 37, actor 256 x 2 blocks, fp32 (the reference acts in fp32); "
                            "small products, launch-bound"})
    del actor_agent

    # (f) PPO rollout step at the c3 collection shape: act() (actor + critic MLPs, Philox noise, sampling)
    # then store() (critic MLP on the next observations, rollout row copies)
    from robolearn_amd.ppo import WarpPPO

    pcfg = ppo_config()
    ppo = WarpPPO(PPO_C3["obs"], PPO_C3["act"], PPO_C3["envs"], PPO_C3["horizon"], pcfg)
    n = PPO_C3["envs"]
    obs_now = torch.randn(n, PPO_C3["obs"], generator=g, device=device)
    obs_next = torch.randn(n, PPO_C3["obs"], generator=g, device=device)
    rewards = torch.randn(n, generator=g, device=device)
    flags = torch.zeros(n, dtype=torch.int32, device=device)

    def rollout_step():
        ppo.act(obs_now)
        ppo.store(0, obs_now, rewards, flags, flags, obs_next)

    ms = _time_launches(rollout_step)
    widths = (PPO_C3["obs"], *PPO_C3["hidden"])
    mlp = lambda out: sum(2 * n * a * b for a, b in zip(widths, widths[1:] + (out,)))  # noqa: E731
    flops = mlp(PPO_C3["act"]) + 2 * mlp(1)
    achieved = flops / (ms * 1e-3) / 1e12
    lines.append({"kernel": "ppo rollout step (act + store)", "ms": round(ms, 4), "flops": int(flops),
                  "bound": "mfma", "achieved": round(achieved, 2), "peak": FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
                  "frac": round(achieved / FP32_PEAK_TFLOPS, 4),
                  "detail": "4096 envs, obs 123, act 37, 512-256-128 ELU, fp32: three MLP forwards, sampling and "
                            "the rollout row copies; launch-bound"})
    return lines


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--workload", choices=sorted(WORKLOADS), default="g1")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-extras", action="store_true",
                        help="skip the PPO (c3) update timing and the HBM kernel sweep (c4)")
    parser.add_argument("--calibration-copy-mb", type=int, default=0,
                        help="after timing, run one plain device copy of this size (counter calibration)")
    parser.add_argument("--traffic", type=float, default=None,
                        help="HBM bytes per launch of the dominant kernel measured with rocprofv3 --pmc (reported)")
    args = parser.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the learner path is single-GPU (see DESIGN.md for sharding).",
              file=sys.stderr)
        return 2

    import torch

    from robolearn_amd import kernels as K
    from robolearn_amd.config import FlashSACConfig
    from robolearn_amd.flashsac import FlashSAC

    w = WORKLOADS[args.workload]
    B = w["batch"]
    capacity = w["envs"] * w["horizon"]
    cfg_kwargs = dict(seed=0, normalize_reward=False, n_step=1, sample_batch_size=B, buffer_max_length=capacity,
                      buffer_min_length=B, actor_hidden_dim=w["actor_hidden"], actor_num_blocks=w["actor_blocks"],
                      critic_hidden_dim=w["critic_hidden"], critic_num_blocks=w["critic_blocks"],
                      critic_num_bins=w["bins"], critic_min_v=w["min_v"], critic_max_v=w["max_v"],
                      critic_target_update_tau=0.005, learning_rate_init=3e-4, learning_rate_peak=3e-4,
                      learning_rate_end=3e-4, gamma=0.99, use_amp=w["amp"], actor_update_period=2)
    cfg = FlashSACConfig(**cfg_kwargs)
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    agent = FlashSAC(w["obs"], w["act"], num_envs=w["envs"], cfg=cfg)
    g = torch.Generator(device=device).manual_seed(0)
    data = {
        "observation": torch.randn(capacity, w["obs"], generator=g, device=device),
        "next_observation": torch.randn(capacity, w["obs"], generator=g, device=device),
        "action": torch.rand(capacity, w["act"], generator=g, device=device) * 2 - 1,
        "reward": torch.randn(capacity, generator=g, device=device) * w["reward_std"],
        "terminated": (torch.rand(capacity, generator=g, device=device) < w["done"]).float(),
        "truncated": torch.zeros(capacity, device=device),
        "discount": torch.full((capacity,), cfg.gamma, device=device),
    }
    agent.load_replay(data)
    del data
    graph = agent.capture_pair() if w["utd"] == 2 else None
    print(f"[bench] workload {args.workload}: captured update-to-data-{w['utd']} graph", file=sys.stderr, flush=True)

    def step():
        if graph is not None:
            graph.replay()
        else:
            agent.update()

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.steps):
        step()
    end.record()
    torch.cuda.synchronize()
    ms_per_step = start.elapsed_time(end) / args.steps
    updates_per_second = w["utd"] * 1000.0 / ms_per_step
    print(f"[bench] {ms_per_step:.3f} ms per step, {updates_per_second:.1f} updates/s", file=sys.stderr, flush=True)

    # Dominant kernel: critic block-1 forward GEMM [2 x 2B x h] . [4h x h]^T (bf16 MFMA), timed live on the
    # stream it is launched on, at the shape it runs with inside the update.
    net = agent.critic_net
    h = net.h
    rows = 2 * B
    reps = 20
    launch = lambda: K.linear_forward(net.op(net.stream[0], net.stream_h[0]),  # noqa: E731
                                      agent.critic_w["encoder.0.w1.weight"], net.u1[0], rows=rows, in_dim=h,
                                      out_dim=4 * h, ensemble=2, mode=agent.mode)
    launch()
    torch.cuda.synchronize()
    k0, k1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    k0.record()
    for _ in range(reps):
        launch()
    k1.record()
    torch.cuda.synchronize()
    kernel_ms = k0.elapsed_time(k1) / reps
    kernel_flops = 2.0 * 2 * rows * h * 4 * h
    peak = {K.BF16: BF16_PEAK_TFLOPS, K.FP32_SPLIT: BF16_PEAK_TFLOPS / 6.0}.get(agent.mode, FP32_PEAK_TFLOPS)
    achieved = kernel_flops / (kernel_ms * 1e-3) / 1e12
    operand = "unsigned short" if agent.mode == K.BF16 else "float"
    out_type = "bf16" if net.u1[0].dtype == torch.bfloat16 else "fp32"
    shape = f"critic block-1 forward [2 x {rows} x {h}] . [{4 * h} x {h}]^T -> {out_type}"
    if agent.mode == K.BF16 and rows % 256 == 0 and (4 * h) % 256 == 0 and h % 128 == 0:
        kernel_name = f"gemm_dma_kernel {shape}"  # 256x256 tiles, DMA-fed (both operands K-contiguous)
    elif agent.mode == K.BF16:
        kernel_name = f"gemm_bf16_kernel<{operand}, {operand}, true, true> {shape}"
    else:
        kernel_name = f"gemm_kernel<0, float, float, true, true> {shape}"
    traffic = args.traffic if args.traffic is not None else measured_traffic(kernel_name)
    operand_bytes = 2 if agent.mode == K.BF16 else 4
    # the output is the BatchNorm input: bf16 in bf16 mode
    algorithmic_bytes = 2 * (rows * h + 4 * h * h) * operand_bytes + 2 * rows * 4 * h * net.u1[0].element_size()
    roofline = {"bound": "mfma", "achieved": round(achieved, 2), "peak": peak, "unit": "TFLOP/s",
                "frac": round(achieved / peak, 4), "traffic": traffic, "kernel": kernel_name,
                "kernel_ms": round(kernel_ms, 4), "flops_per_launch": kernel_flops,
                "algorithmic_bytes_per_launch": algorithmic_bytes}
    if args.calibration_copy_mb:
        # plain device copy of known size, for scaling FETCH_SIZE / WRITE_SIZE counter readings
        n = args.calibration_copy_mb * (1 << 20) // 4
        src = torch.ones(n, device=device)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    flops = gemm_flops(w)
    hbm_bytes = elementwise_bytes(w, 2 if agent.mode == K.BF16 else 4)
    t_roof_ms = (flops / (peak * 1e12) + hbm_bytes / (HBM_PEAK_GBS * 1e9)) * 1e3
    update_roofline = {"gemm_tflop_per_step": round(flops / 1e12, 3),
                       "elementwise_gb_per_step": round(hbm_bytes / 1e9, 3),
                       "t_roof_ms_per_step": round(t_roof_ms, 3),
                       "frac": round(t_roof_ms / ms_per_step, 4)}

    ppo, sweep = None, None
    if not args.no_extras:
        print("[bench] PPO c3 update", file=sys.stderr, flush=True)
        ppo = bench_ppo(max(5, args.steps // 2), 2, not args.no_cpu_baseline)
        print("[bench] kernel sweep", file=sys.stderr, flush=True)
        sweep = kernel_sweep()

    baseline = None
    if not args.no_cpu_baseline:
        print("[bench] timing the CPU oracle baseline", file=sys.stderr, flush=True)
        baseline = cpu_baseline(w, cfg_kwargs)

    result = {
        "metric": "FlashSAC updates/sec at batch 8192 (1 GPU)" if args.workload == "g1"
        else f"FlashSAC updates/sec at batch {B} (1 GPU)",
        "value": round(updates_per_second, 3),
        "unit": "updates/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if w["amp"] else "fp32",
        "data": "synthetic",
        "config": {"workload": f"flashsac_{args.workload}", "batch": B, "obs_dim": w["obs"], "act_dim": w["act"],
                   "actor": f"{w['actor_hidden']}x{w['actor_blocks']}",
                   "critic": f"2x {w['critic_hidden']}x{w['critic_blocks']}", "bins": w["bins"],
                   "updates_per_step": w["utd"], "replay_rows": capacity, "parallelism": "single-gpu"},
        "roofline": roofline,
        "update_roofline": update_roofline,
        "cpu_baseline": baseline,
        "ppo": ppo,
        "kernel_sweep": sweep,
    }
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
