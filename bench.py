#!/usr/bin/env python3
"""Learner hot-path benchmark on one MI355X.

Headline ("g1"): one captured HIP graph per step
holding two FlashSAC updates (update-to-data 2: an actor+critic update and a
critic-only update) at batch 8192, obs 123, act 37, actor 256x2, twin critics
1024x2, 101 bins on [-20, 20], bf16 dense operands with fp32 state, BatchNorm
inputs and ReLU-BN gradients stored in bf16; replay 4096 envs x 256 steps of
seeded synthetic transitions resident in HBM.

Prints ONE JSON line: value = FlashSAC updates/sec on the GPU, with
  roofline        the dominant kernel (critic block-1 forward GEMM, bf16 MFMA)
                  timed live with HIP events on the stream it runs on; its HBM
                  traffic and MFMA-busy share come from the committed rocprofv3
                  summary only when that summary names the same kernel, shape and
                  kernel-source fingerprint as this build,
  update_roofline two-term serial roofline of the whole update,
  workloads       the other configurations at 1 GPU: G1 with fp32 BatchNorm
                  activations, configs[0] Cartpole (fp32) and configs[1] README in
                  both modes, each with updates/s and its update roofline,
  ppo             PPO update ms at configs[3] (one captured graph per update),
                  against the published fp32 matrix peak,
  kernel_sweep    configs[4]: the HBM-bound kernels at their sweep shapes,
  bf16_drift_100_updates
                  the bf16 learner against the fp32 learner over 100 G1 updates
                  from the same weights, replay and device draws (not timed),
  cpu_baseline    the CPU oracle (PyTorch-CPU restatement of the reference update,
                  fp32) at G1 on this host's cores; cpu_baselines holds c0, c1,
                  c2 and c3 at all cores and at 8 threads with the CPU model.
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
TRAFFIC_PROFILE = ROOT / "profiles" / "gemm_wide_critic_fwd_g1_counters.md"
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


BLOCK_STEPS = 20  # graph replays per timing block


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


# the sources the dominant kernel (gemm_wide_kernel) is compiled from
DOMINANT_SOURCES = ("common.hpp", "gemm.hpp", "gemm_bf16_big.hip")


def _code_of(text: str) -> str:
    """C++ source without its comments and blank lines (string literals kept as written)."""
    out, i, n = [], 0, len(text)
    while i < n:
        if text.startswith("//", i):
            i = text.find("\n", i)
            i = n if i < 0 else i
        elif text.startswith("/*", i):
            j = text.find("*/", i + 2)
            i = n if j < 0 else j + 2
        elif text[i] == '"':
            j = i + 1
            while j < n and text[j] != '"':
                j += 2 if text[j] == "\\" else 1
            out.append(text[i:j + 1])
            i = j + 1
        else:
            out.append(text[i])
            i += 1
    return "\n".join(line.rstrip() for line in "".join(out).splitlines() if line.strip())


def source_fingerprint() -> str:
    """First 16 hex digits of the SHA-256 of the dominant kernel's sources (names and code, in order;
    comments and blank lines do not count, so a comment edit does not orphan a measurement)."""
    import hashlib

    digest = hashlib.sha256()
    for name in DOMINANT_SOURCES:
        digest.update(name.encode())
        digest.update(_code_of((ROOT / "robolearn_amd" / "csrc" / name).read_text()).encode())
    return digest.hexdigest()[:16]


def measured_counters(kernel: str) -> dict:
    """HBM bytes per launch and MFMA-busy share of `kernel` from the committed rocprofv3 --pmc summary.

    The summary holds `kernel:`, `source:` (the kernel-source fingerprint of the build it
    measured), `traffic_bytes_per_launch:` (FETCH_SIZE + WRITE_SIZE, each scaled by a plain copy
    of known size) and `mfma_busy_percent:` lines; a summary of another kernel, shape or build
    is ignored, so the numbers cannot go stale silently."""
    try:
        text = TRAFFIC_PROFILE.read_text()
    except OSError:
        return {}
    fields = dict(re.findall(r"^([a-z_]+): (.+)$", text, flags=re.M))
    if fields.get("kernel", "").strip() != kernel or fields.get("source", "").strip() != source_fingerprint():
        return {}
    out = {}
    if "traffic_bytes_per_launch" in fields:
        out["traffic"] = int(fields["traffic_bytes_per_launch"])
    if "mfma_busy_percent" in fields:
        out["mfma_busy_percent"] = float(fields["mfma_busy_percent"])
    return out


def cpu_model() -> str:
    """The host CPU as lscpu names it (model name, family/model/stepping, the BIOS model name when
    present), falling back to /proc/cpuinfo."""
    import subprocess

    fields = {}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        for line in out.splitlines():
            key, _, value = line.partition(":")
            fields[key.strip()] = value.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    name = fields.get("Model name")
    if not name:
        try:
            with open("/proc/cpuinfo") as stream:
                for line in stream:
                    if line.startswith("model name"):
                        name = line.split(":", 1)[1].strip()
                        break
        except OSError:
            pass
    parts = [name or "unknown"]
    ids = [f"{k.lower()} {fields[k]}" for k in ("CPU family", "Model", "Stepping") if fields.get(k)]
    if ids:
        parts.append("(" + ", ".join(ids) + ")")
    if fields.get("BIOS Model name") and fields["BIOS Model name"] != name:
        parts.append(f"BIOS model name {fields['BIOS Model name']}")
    return " ".join(parts)


def _median(values):
    values = sorted(values)
    n = len(values)
    return values[n // 2] if n % 2 else 0.5 * (values[n // 2 - 1] + values[n // 2])


def cpu_flashsac(w: dict, cfg_kwargs: dict, threads: int, warmups: int, timed: int) -> dict:
    """The CPU oracle (fp32) at the workload shape: `warmups` untimed then `timed` timed updates,
    alternating actor-phase and critic-only updates as the UTD-2 step does; seconds per update is
    the mean of the two phases' medians."""
    import torch

    from dataclasses import replace

    from oracle import flashsac as O
    from robolearn_amd.config import FlashSACConfig

    torch.set_num_threads(threads)
    cfg = FlashSACConfig(**cfg_kwargs)
    cfg = replace(cfg, temp_target_entropy=O.target_entropy(w["act"], cfg.temp_target_sigma))
    d = O.dims_from_config(w["obs"], w["act"], cfg)
    state = O.init_state(d, cfg, seed=0, dtype=torch.float32)
    g = torch.Generator().manual_seed(5)
    B = w["batch"]
    batch = {
        "observation": torch.randn(B, w["obs"], generator=g), "next_observation": torch.randn(B, w["obs"], generator=g),
        "action": torch.rand(B, w["act"], generator=g) * 2 - 1,
        "reward": torch.randn(B, generator=g) * w["reward_std"],
        "terminated": (torch.rand(B, generator=g) < w["done"]).float(), "discount": torch.full((B,), cfg.gamma),
    }
    noise = torch.randn(2 * B, w["act"], generator=g)
    next_noise = torch.randn(B, w["act"], generator=g)
    times = {True: [], False: []}
    for i in range(warmups + timed):
        actor = i % 2 == 0
        t0 = time.perf_counter()
        O.update(state, batch, noise, next_noise, do_actor_update=actor)
        if i >= warmups:
            times[actor].append(time.perf_counter() - t0)
    medians = [_median(v) for v in times.values() if v]
    return {"seconds_per_update": sum(medians) / len(medians), "threads": threads, "warmups": warmups,
            "timed_updates": timed,
            "phases": {"actor_phase_s": _median(times[True]) if times[True] else None,
                       "critic_only_s": _median(times[False]) if times[False] else None}}


def cpu_ppo(threads: int, warmups: int, timed: int) -> dict:
    """The CPU oracle (fp32) on full c3 PPO updates (GAE, 5 epochs x 4 minibatches) of one rollout."""
    import numpy as np
    import torch

    from oracle import ppo as OP

    torch.set_num_threads(threads)
    cfg = ppo_config()
    E, T, O_, A = PPO_C3["envs"], PPO_C3["horizon"], PPO_C3["obs"], PPO_C3["act"]
    n = E * T
    rng = np.random.default_rng(0)
    rollout = dict(observations=rng.standard_normal((n, O_)).astype(np.float32),
                   actions=rng.standard_normal((n, A)).astype(np.float32),
                   means=rng.standard_normal((n, A)).astype(np.float32) * 0.1, stds=np.ones((n, A), np.float32),
                   values=rng.standard_normal(n).astype(np.float32),
                   log_probs=rng.standard_normal(n).astype(np.float32) - 40.0,
                   rewards=rng.standard_normal(n).astype(np.float32),
                   next_values=rng.standard_normal(n).astype(np.float32),
                   terminated=(rng.random(n) < 1e-3).astype(np.int32), truncated=np.zeros(n, np.int32))
    params = OP.init_parameters(O_, A, cfg)
    permutation = rng.permutation(n)
    times = []
    for i in range(warmups + timed):
        oracle = OP.PPOOracle(O_, A, E, T, cfg, params, dtype=torch.float32)
        t0 = time.perf_counter()
        oracle.update(rollout, permutation)
        if i >= warmups:
            times.append(time.perf_counter() - t0)
    return {"seconds_per_update": _median(times), "threads": threads, "warmups": warmups, "timed_updates": timed}


def cpu_baselines() -> dict:
    """c0, c1 (fp32), c2 and c3 on the CPU oracle at all host cores and at 8 threads (the reference
    harnesses pin 8: examples/benchmark_warp_flashsac.py:87, benchmark_official_flashsac.py:878).
    3 warm-ups and the median of 5 where the time allows; c2 (about 15-25 s per update on 8-16 cores)
    is capped at 1 warm-up + 2 timed updates (one of each phase) and c3 (about 5 s per update) at
    1 + 3 and 1 + 2; the counts are recorded in each entry."""
    all_cores = len(os.sched_getaffinity(0))
    out = {"cpu_model": cpu_model(), "all_cores": all_cores, "configs": {}}
    plans = {"c0_cartpole": ("cartpole", 3, 5, 3, 5), "c1_readme_fp32": ("readme", 3, 5, 2, 3),
             "c2_g1": ("g1", 1, 2, 1, 2)}
    for label, (name, warm_all, timed_all, warm_8, timed_8) in plans.items():
        w = dict(WORKLOADS[name], amp=False)
        kwargs = flashsac_config_kwargs(w)
        entry = {}
        for threads, warm, timed in ((all_cores, warm_all, timed_all), (min(8, all_cores), warm_8, timed_8)):
            print(f"[bench] CPU oracle {label} at {threads} threads", file=sys.stderr, flush=True)
            result = cpu_flashsac(w, kwargs, threads, warm, timed)
            entry[f"threads_{threads}"] = dict(result, updates_per_s=1.0 / result["seconds_per_update"])
        out["configs"][label] = entry
    entry = {}
    for threads, warm, timed in ((all_cores, 1, 3), (min(8, all_cores), 1, 2)):
        print(f"[bench] CPU oracle c3_ppo at {threads} threads", file=sys.stderr, flush=True)
        result = cpu_ppo(threads, warm, timed)
        entry[f"threads_{threads}"] = dict(result, ms_per_update=1e3 * result["seconds_per_update"])
    out["configs"]["c3_ppo"] = entry
    return out


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


def ppo_rollout(agent, seed=0, behaviour_shift=0.025):
    """Synthetic c3 rollout on the device: obs, next values ~ N(0,1); actions = mu(obs) + sigma*eps with
    their Gaussian log-probs and the critic's values from act(), the stored means and values shifted by
    N(0, behaviour_shift^2) as a rollout a few updates old holds; rewards ~ N(0,1); terminated ~
    Bernoulli(1/1000); no truncations."""
    import math

    import torch

    n = agent.batch_size
    g = torch.Generator(device=agent.device).manual_seed(seed)
    obs = torch.randn(n, agent.observation_dim, generator=g, device=agent.device)
    actions = agent.act(obs)
    sampled = agent._act_state(n)
    means = sampled["mean"] + behaviour_shift * torch.randn(n, agent.action_dim, generator=g, device=agent.device)
    std = sampled["std"].expand(n, -1)
    log_probs = (-0.5 * (((actions - means) / std) ** 2 + 2.0 * torch.log(std) + math.log(2 * math.pi))).sum(-1)
    agent.observations.copy_(obs)
    agent.actions.copy_(actions)
    agent.log_probs.copy_(log_probs)
    agent.means.copy_(means)
    agent.stds.copy_(std)
    agent.values.copy_(sampled["values"] + behaviour_shift * torch.randn(n, generator=g, device=agent.device))
    agent.next_values.copy_(torch.randn(n, generator=g, device=agent.device))
    agent.rewards.copy_(torch.randn(n, generator=g, device=agent.device))
    agent.terminated.copy_((torch.rand(n, generator=g, device=agent.device) < 1e-3).int())
    agent.truncated.zero_()


def bench_ppo(steps: int, warmup: int) -> dict:
    """PPO update ms at c3: one captured graph (GAE, permutation, 5 epochs x 4 minibatches) per update.
    The roofline prices the fp32 product FLOPs against the published fp32 matrix peak (157.3 TFLOP/s);
    the products run as fp32-accurate three-piece bf16 splits (6 bf16 MFMA products per fp32 product),
    whose issued bf16 rate is reported beside it."""
    import torch

    from robolearn_amd import kernels as K
    from robolearn_amd.ppo import WarpPPO

    cfg = ppo_config()
    agent = WarpPPO(PPO_C3["obs"], PPO_C3["act"], PPO_C3["envs"], PPO_C3["horizon"], cfg)
    ppo_rollout(agent)
    agent.update()  # captures the graph (after an eager warm-up that restores the state)
    for _ in range(warmup):
        agent.update()
    torch.cuda.synchronize()
    start, end = _events()
    start.record()
    for _ in range(steps):
        agent.update()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    flops = ppo_flops(cfg)
    achieved = flops / (ms * 1e-3) / 1e12
    split = agent.gemm_mode == K.FP32_SPLIT
    roofline = {"bound": "mfma", "achieved": round(achieved, 2), "peak": FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / FP32_PEAK_TFLOPS, 4), "flops_per_update": flops,
                "products": "fp32-accurate three-piece bf16 splits (6 bf16 MFMA products per fp32 product)"
                if split else "v_mfma_f32_32x32x2_f32"}
    if split:
        roofline["issued_bf16_tflops"] = round(6 * achieved, 2)
        roofline["issued_bf16_frac"] = round(6 * achieved / BF16_PEAK_TFLOPS, 4)
    result = {
        "metric": "PPO update ms", "value": round(ms, 4), "unit": "ms/update", "higher_is_better": False,
        "dtype": "fp32", "steps": steps, "warmup": warmup,
        "config": {"workload": "ppo_c3", "envs": PPO_C3["envs"], "horizon": PPO_C3["horizon"],
                   "obs_dim": PPO_C3["obs"], "act_dim": PPO_C3["act"], "hidden": list(cfg.hidden_dims),
                   "activation": cfg.activation, "epochs": cfg.epochs, "minibatches": cfg.num_mini_batches,
                   "schedule": cfg.schedule, "desired_kl": cfg.desired_kl,
                   "grad_clipping": "separate" if cfg.separate_grad_clipping else "combined"},
        "roofline": roofline,
        "cpu_baseline": None,
    }
    del agent
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return result


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


def flashsac_config_kwargs(w: dict) -> dict:
    B = w["batch"]
    capacity = w["envs"] * w["horizon"]
    return dict(seed=0, normalize_reward=False, n_step=1, sample_batch_size=B, buffer_max_length=capacity,
                buffer_min_length=B, actor_hidden_dim=w["actor_hidden"], actor_num_blocks=w["actor_blocks"],
                critic_hidden_dim=w["critic_hidden"], critic_num_blocks=w["critic_blocks"],
                critic_num_bins=w["bins"], critic_min_v=w["min_v"], critic_max_v=w["max_v"],
                critic_target_update_tau=0.005, learning_rate_init=3e-4, learning_rate_peak=3e-4,
                learning_rate_end=3e-4, gamma=0.99, use_amp=w["amp"], actor_update_period=2)


def _events():
    import torch

    return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


def dominant_kernel(agent, w: dict, reps: int = 20, calibration_copy_mb: int = 0) -> dict:
    """Critic block-1 forward GEMM [2 x 2B x h] . [4h x h]^T at the shape it runs with inside the
    update, timed over `reps` launches with HIP events recorded on the stream it is launched on."""
    import torch

    from robolearn_amd import kernels as K

    net = agent.critic_net
    h, rows = net.h, 2 * w["batch"]
    launch = lambda: K.linear_forward(net.op(net.stream[0], net.stream_h[0]),  # noqa: E731
                                      agent.critic_w["encoder.0.w1.weight"], net.u1[0], rows=rows, in_dim=h,
                                      out_dim=4 * h, ensemble=2, mode=agent.mode)
    launch()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()  # kernels.stream() launches on torch's current stream
    k0, k1 = _events()
    k0.record(stream)
    for _ in range(reps):
        launch()
    k1.record(stream)
    torch.cuda.synchronize()
    kernel_ms = k0.elapsed_time(k1) / reps
    if calibration_copy_mb:
        # one plain device copy of known size, for scaling FETCH_SIZE / WRITE_SIZE counter readings
        n = calibration_copy_mb * (1 << 20) // 4
        src = torch.ones(n, device=net.u1[0].device)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    flops = 2.0 * 2 * rows * h * 4 * h
    bf16 = agent.mode == K.BF16
    peak = BF16_PEAK_TFLOPS if bf16 else FP32_PEAK_TFLOPS
    achieved = flops / (kernel_ms * 1e-3) / 1e12
    out_type = "bf16" if net.u1[0].dtype == torch.bfloat16 else "fp32"
    shape = f"critic block-1 forward [2 x {rows} x {h}] . [{4 * h} x {h}]^T -> {out_type}"
    if bf16 and rows % 256 == 0 and (4 * h) % 256 == 0 and h % 128 == 0:
        kernel = f"rl::gemm::big::wide::gemm_wide_kernel {shape}"  # 8 waves, 256x256 tiles, DMA-fed
    elif bf16:
        kernel = f"rl::gemm::gemm_bf16_kernel {shape}"
    else:
        kernel = f"rl::gemm::gemm_kernel {shape}"
    operand_bytes = 2 if bf16 else 4
    algorithmic_bytes = 2 * (rows * h + 4 * h * h) * operand_bytes + 2 * rows * 4 * h * net.u1[0].element_size()
    counters = measured_counters(kernel)
    roofline = {"bound": "mfma", "achieved": round(achieved, 2), "peak": peak, "unit": "TFLOP/s",
                "frac": round(achieved / peak, 4), "traffic": counters.get("traffic"), "kernel": kernel,
                "kernel_ms": round(kernel_ms, 4), "flops_per_launch": flops,
                "algorithmic_bytes_per_launch": algorithmic_bytes, "source": source_fingerprint()}
    if "mfma_busy_percent" in counters:
        roofline["mfma_busy_percent"] = counters["mfma_busy_percent"]
    return roofline


def run_flashsac(name: str, steps: int, warmup: int, *, bf16_activations: bool = True, amp=None,
                 dominant: bool = False, calibration_copy_mb: int = 0) -> dict:
    """Updates/s of one workload: seeded synthetic replay resident in HBM, one captured graph per step
    (UTD 2: actor-phase + critic-only update, device-side replay sampling inside the graph)."""
    import torch

    from robolearn_amd import kernels as K
    from robolearn_amd.config import FlashSACConfig
    from robolearn_amd.flashsac import FlashSAC

    w = dict(WORKLOADS[name])
    if amp is not None:
        w["amp"] = amp
    cfg = FlashSACConfig(**flashsac_config_kwargs(w))
    device = torch.device("cuda:0")
    capacity = w["envs"] * w["horizon"]
    agent = FlashSAC(w["obs"], w["act"], num_envs=w["envs"], cfg=cfg, bf16_activations=bf16_activations)
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
    agent.capture_pair()
    for _ in range(warmup):
        agent.update_pair(tensor_metrics=True)
    torch.cuda.synchronize()
    # timed: exactly `steps` graph replays between two synchronizations, with an event at every block
    # boundary (blocks of `block` replays, no host wait inside the timed region); ms_per_step is the
    # whole region's mean, and the median of the block means is reported beside it (the reference
    # protocol, examples/benchmark_official_flashsac.py:422-429, 654-655)
    block = max(1, min(BLOCK_STEPS, steps))
    marks = [torch.cuda.Event(enable_timing=True) for _ in range((steps + block - 1) // block + 1)]
    marks[0].record()
    for i in range(steps):
        agent.update_pair(tensor_metrics=True)
        if (i + 1) % block == 0 or i + 1 == steps:
            marks[(i + block) // block].record()
    torch.cuda.synchronize()
    ms_per_step = marks[0].elapsed_time(marks[-1]) / steps
    sizes = [min(block, steps - j * block) for j in range(len(marks) - 1)]
    block_means = [marks[j].elapsed_time(marks[j + 1]) / sizes[j] for j in range(len(marks) - 1)]
    bf16 = agent.mode == K.BF16
    act_bytes = 2 if agent.bf16_activations else 4
    flops = gemm_flops(w)
    hbm_bytes = elementwise_bytes(w, act_bytes)
    peak = BF16_PEAK_TFLOPS if bf16 else FP32_PEAK_TFLOPS
    t_roof_ms = (flops / (peak * 1e12) + hbm_bytes / (HBM_PEAK_GBS * 1e9)) * 1e3
    result = {
        "workload": f"flashsac_{name}", "updates_per_s": round(2000.0 / ms_per_step, 3),
        "ms_per_step": round(ms_per_step, 4), "steps": steps, "warmup": warmup,
        "timing": {"block_steps": block, "blocks": len(block_means),
                   "median_block_ms_per_step": round(_median(block_means), 4),
                   "block_ms_per_step": [round(v, 4) for v in block_means]},
        "dtype": "bf16" if bf16 else "fp32",
        "batchnorm_activations": "bf16" if agent.bf16_activations else "fp32",
        "update_roofline": {"gemm_tflop_per_step": round(flops / 1e12, 4),
                            "elementwise_gb_per_step": round(hbm_bytes / 1e9, 4), "peak_tflops": peak,
                            "t_roof_ms_per_step": round(t_roof_ms, 4), "frac": round(t_roof_ms / ms_per_step, 4)},
    }
    if dominant:
        result["roofline"] = dominant_kernel(agent, w, calibration_copy_mb=calibration_copy_mb)
    del agent
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return result


def bf16_drift(name: str = "g1", pairs: int = 50) -> dict:
    """The 100-update drift of the bf16 learner against the fp32 learner at a workload shape: both start
    from the same weights and seeded synthetic replay and run `pairs` captured UTD-2 steps; with one seed
    their device samplers draw the same indices and noise.  Relative L2 parameter distance after the run
    (to the parameters and to the fp32 learner's own movement) and the largest relative difference of
    each loss over the run (absolute floor 1e-3).  Not timed."""
    import numpy as np
    import torch

    from robolearn_amd.config import FlashSACConfig
    from robolearn_amd.flashsac import FlashSAC

    w = dict(WORKLOADS[name])
    device = torch.device("cuda:0")
    capacity = w["envs"] * w["horizon"]
    agents = []
    for amp in (True, False):
        cfg = FlashSACConfig(**flashsac_config_kwargs(dict(w, amp=amp)))
        agents.append(FlashSAC(w["obs"], w["act"], num_envs=w["envs"], cfg=cfg))
    low, ref = agents
    ref.load_state_dict(low.state_dict(include_replay=False))
    g = torch.Generator(device=device).manual_seed(0)
    data = {
        "observation": torch.randn(capacity, w["obs"], generator=g, device=device),
        "next_observation": torch.randn(capacity, w["obs"], generator=g, device=device),
        "action": torch.rand(capacity, w["act"], generator=g, device=device) * 2 - 1,
        "reward": torch.randn(capacity, generator=g, device=device) * w["reward_std"],
        "terminated": (torch.rand(capacity, generator=g, device=device) < w["done"]).float(),
        "truncated": torch.zeros(capacity, device=device),
        "discount": torch.full((capacity,), low.cfg.gamma, device=device),
    }
    for agent in agents:
        agent.load_replay(data)
    del data
    start = {k: np.asarray(v, dtype=np.float64) for k, v in ref.state_dict(include_replay=False).items()}
    worst = {}
    for _ in range(pairs):
        m16, m32 = low.update_pair(tensor_metrics=False), ref.update_pair(tensor_metrics=False)
        for key, value in m32.items():
            worst[key] = max(worst.get(key, 0.0), abs(m16[key] - value) / max(abs(value), 1e-3))
    p16, p32 = low.state_dict(include_replay=False), ref.state_dict(include_replay=False)
    groups = {}
    for key, value in p32.items():
        value = np.asarray(value)
        if "running" in key or value.dtype.kind != "f":
            continue
        a, b = value.astype(np.float64), np.asarray(p16[key], dtype=np.float64)
        acc = groups.setdefault("actor" if key.startswith("actor") else "critic", [0.0, 0.0, 0.0])
        acc[0] += float(((b - a) ** 2).sum())
        acc[1] += float((a ** 2).sum())
        acc[2] += float(((a - start[key]) ** 2).sum())
    del agents, low, ref
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return {"workload": f"flashsac_{name}", "updates": 2 * pairs,
            "bf16": "bf16 operands, bf16 BatchNorm activations", "reference": "the fp32 learner",
            "parameter_drift_rel_l2": {k: round((v[0] / v[1]) ** 0.5, 6) for k, v in groups.items()},
            "drift_over_fp32_movement": {k: round((v[0] / max(v[2], 1e-30)) ** 0.5, 6) for k, v in groups.items()},
            "max_rel_loss_difference": {k: round(v, 6) for k, v in worst.items()}}


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=100)
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--workload", choices=sorted(WORKLOADS), default="g1")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-extras", action="store_true",
                        help="headline only: skip the other workloads, PPO (c3) and the kernel sweep (c4)")
    parser.add_argument("--sweep-only", action="store_true",
                        help="run only the configs[4] kernel sweep and print its lines as one JSON object "
                             "(for rocprofv3 counter passes over the sweep kernels)")
    parser.add_argument("--ppo-only", action="store_true",
                        help="run only the configs[3] PPO update and print its line as one JSON object")
    parser.add_argument("--bf16", action="store_true",
                        help="bf16 operands for the headline workload (configs[1] README runs fp32 by default)")
    parser.add_argument("--calibration-copy-mb", type=int, default=0,
                        help="after timing the dominant kernel, one plain device copy of this size "
                             "(scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    args = parser.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: every GPU box of this build has one GPU, and the learner "
              "update runs on one GPU.", file=sys.stderr)
        return 2

    import torch

    torch.cuda.set_device(0)
    if args.sweep_only:
        print(json.dumps({"kernel_sweep": kernel_sweep()}))
        return 0
    if args.ppo_only:
        print(json.dumps({"ppo": bench_ppo(max(5, min(20, args.steps // 5)), 2)}))
        return 0
    w = WORKLOADS[args.workload]
    head = run_flashsac(args.workload, args.steps, args.warmup, dominant=True,
                        calibration_copy_mb=args.calibration_copy_mb, amp=True if args.bf16 else None)
    print(f"[bench] {args.workload}: {head['ms_per_step']:.3f} ms per step, {head['updates_per_s']:.1f} updates/s",
          file=sys.stderr, flush=True)

    others, ppo, sweep, drift = None, None, None, None
    if not args.no_extras:
        few = max(10, min(50, args.steps // 2))
        others = []
        plans = [("g1", dict(bf16_activations=False)), ("cartpole", {}), ("readme", {}),
                 ("readme", dict(amp=True)), ("readme", dict(amp=True, bf16_activations=False))]
        for name, kwargs in plans:
            if name == args.workload and not kwargs:
                continue
            line = run_flashsac(name, few, 2, **kwargs)
            others.append(line)
            print(f"[bench] {line['workload']} {line['dtype']} (BatchNorm activations "
                  f"{line['batchnorm_activations']}): {line['updates_per_s']:.1f} updates/s",
                  file=sys.stderr, flush=True)
        print("[bench] PPO c3 update", file=sys.stderr, flush=True)
        ppo = bench_ppo(max(5, min(20, args.steps // 5)), 2)
        print("[bench] kernel sweep", file=sys.stderr, flush=True)
        sweep = kernel_sweep()
        print("[bench] 100-update bf16 drift at G1", file=sys.stderr, flush=True)
        drift = bf16_drift("g1")

    baselines, baseline = None, None
    if not args.no_cpu_baseline:
        print("[bench] timing the CPU oracle baselines", file=sys.stderr, flush=True)
        baselines = cpu_baselines()
        label = {"g1": "c2_g1", "readme": "c1_readme_fp32", "cartpole": "c0_cartpole"}[args.workload]
        entry = baselines["configs"][label][f"threads_{baselines['all_cores']}"]
        baseline = {"value": round(entry["updates_per_s"], 4), "unit": "updates/s", "cores": entry["threads"],
                    "kind": "port",
                    "sample": f"oracle.flashsac (PyTorch CPU, fp32) at the {args.workload} shape on "
                              f"{baselines['cpu_model']}: {entry['warmups']} warm-up + {entry['timed_updates']} "
                              f"timed updates alternating actor-phase and critic-only; mean of the two phases' "
                              f"medians"}
        if ppo is not None:
            c3 = baselines["configs"]["c3_ppo"][f"threads_{baselines['all_cores']}"]
            ppo["cpu_baseline"] = {"value": round(c3["ms_per_update"], 1), "unit": "ms/update",
                                   "cores": c3["threads"], "kind": "port",
                                   "sample": f"oracle.ppo (PyTorch CPU, fp32): full c3 updates, "
                                             f"{c3['warmups']} warm-up + median of {c3['timed_updates']}"}

    B = w["batch"]
    result = {
        "metric": "FlashSAC updates/sec at batch 8192 (1 GPU)" if args.workload == "g1"
        else f"FlashSAC updates/sec at batch {B} (1 GPU)",
        "value": head["updates_per_s"],
        "unit": "updates/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "timing": head["timing"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": head["dtype"],
        "data": "synthetic",
        "config": {"workload": f"flashsac_{args.workload}", "batch": B, "obs_dim": w["obs"], "act_dim": w["act"],
                   "actor": f"{w['actor_hidden']}x{w['actor_blocks']}",
                   "critic": f"2x {w['critic_hidden']}x{w['critic_blocks']}", "bins": w["bins"],
                   "updates_per_step": w["utd"], "replay_rows": w["envs"] * w["horizon"],
                   "batchnorm_activations": head["batchnorm_activations"], "parallelism": "single-gpu"},
        "roofline": head["roofline"],
        "update_roofline": head["update_roofline"],
        "cpu_baseline": baseline,
        "workloads": others,
        "ppo": ppo,
        "kernel_sweep": sweep,
        "bf16_drift_100_updates": drift,
        "cpu_baselines": baselines,
    }
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
