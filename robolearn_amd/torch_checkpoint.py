"""The reference's Torch FlashSAC checkpoint directory, read and written in place.

Layout (robolearn/flashsac/agent.py:529-576):
  config.json            observation_dim, critic_observation_dim, action_dim, config
  actor.pt, critic.pt, temperature.pt, target_critic.pt
                         Network.save dicts (robolearn/flashsac/_utils/network.py:115-127):
                         network_state_dict (module keys in registration order),
                         optimizer_state_dict (torch.optim.Adam), scheduler_state_dict
                         (LambdaLR), update_step; the target critic has no optimizer
  reward_normalizer.pt   G_r, G_r_max, G_rms_mean, G_rms_var, G_rms_count
                         (robolearn/flashsac/_utils/reward_normalization.py:136-163)
  agent_state.pt         update_step, grad_scaler_state_dict
  replay_buffer.pt       written by save_replay_buffer (robolearn/flashsac/replay.py:196-243)

Files are read with torch.load(weights_only=True) only.  Loading follows
agent.py:556-576: optimizer, scheduler and update step only with
cfg.load_optimizer; the reward normalizer only with cfg.load_reward_normalizer,
and then its per-environment returns restart at zero.  The module key order is
that of FlashSACActor / FlashSACDoubleCritic (robolearn/flashsac/networks.py,
layers.py): embedder (norm, w), encoder blocks (w1, w2, norm1, norm2),
post_norm, predictor; Adam's parameter indices follow the same order without
the buffers.
"""

import json
import math
import warnings
from dataclasses import asdict
from pathlib import Path

import numpy as np
import torch

def _bn(prefix):
    return [(f"{prefix}.weight", "param"), (f"{prefix}.bias", "param"),
            (f"{prefix}.running_mean", "buffer"), (f"{prefix}.running_var", "buffer")]


def actor_module_keys(blocks: int) -> list:
    """FlashSACActor state-dict keys in registration order, tagged param / buffer."""
    keys = _bn("embedder.norm") + [("embedder.w.w.weight", "param")]
    for i in range(blocks):
        keys += [(f"encoder.{i}.w1.w.weight", "param"), (f"encoder.{i}.w2.w.weight", "param")]
        keys += _bn(f"encoder.{i}.norm1") + _bn(f"encoder.{i}.norm2")
    keys += [("post_norm.weight", "param"), ("predictor.mean_bias", "param"), ("predictor.std_bias", "param"),
             ("predictor.mean_w.w.weight", "param"), ("predictor.std_w.w.weight", "param")]
    return keys


def critic_module_keys(blocks: int) -> list:
    """FlashSACDoubleCritic state-dict keys in registration order, tagged param / buffer / support."""
    keys = _bn("embedder.norm") + [("embedder.w.weight", "param")]
    for i in range(blocks):
        keys += [(f"encoder.{i}.w1.weight", "param"), (f"encoder.{i}.w2.weight", "param")]
        keys += _bn(f"encoder.{i}.norm1") + _bn(f"encoder.{i}.norm2")
    keys += [("post_norm.weight", "param"), ("predictor.bias", "param"), ("predictor.bin_values", "support"),
             ("predictor.w.weight", "param")]
    return keys


def _schedule(cfg):
    """warmup_cosine_decay_scheduler (robolearn/flashsac/_utils/scheduler.py:43-65) as a host function."""
    init, peak, end = cfg.learning_rate_init, cfg.learning_rate_peak, cfg.learning_rate_end
    warmup, decay = cfg.learning_rate_warmup_step, cfg.learning_rate_decay_step

    def lr(step):
        if step < warmup:
            return init + (peak - init) * (step / warmup)
        if step < decay:
            return end + (peak - end) * 0.5 * (1 + math.cos(math.pi * ((step - warmup) / (decay - warmup))))
        return end

    return lr


def _optimizer_dicts(cfg, params: list, m1: list, m2: list, timestep: float):
    """torch.optim.Adam and LambdaLR state dicts for `params` (CPU tensors) after `timestep` steps."""
    holders = [torch.nn.Parameter(p.clone()) for p in params]
    optimizer = torch.optim.Adam(holders, lr=cfg.learning_rate_peak)
    schedule = _schedule(cfg)
    scheduler = torch.optim.lr_scheduler.LambdaLR(optimizer, lr_lambda=lambda s: schedule(s) / cfg.learning_rate_peak)
    steps = int(round(timestep))
    if steps > 0:
        for holder, a, b in zip(holders, m1, m2):
            optimizer.state[holder] = {"step": torch.tensor(float(steps)), "exp_avg": a.clone(),
                                       "exp_avg_sq": b.clone()}
        scheduler.last_epoch = steps - 1
        scheduler._step_count = steps
        with warnings.catch_warnings():  # no optimizer.step() ran on these holders
            warnings.simplefilter("ignore")
            scheduler.step()  # lr = schedule(steps) and _last_lr, as after `steps` real steps
    return optimizer.state_dict(), scheduler.state_dict()


def save(agent, path) -> None:
    """Write the agent as the reference's Torch checkpoint directory (agent.py:529-551)."""
    directory = Path(path)
    directory.mkdir(parents=True, exist_ok=True)
    cfg = agent.cfg
    state = agent.state_dict(include_replay=False)
    t = lambda key: torch.as_tensor(np.asarray(state[key])).clone()  # noqa: E731
    metadata = {
        "observation_dim": agent.observation_dim,
        "critic_observation_dim": agent.critic_observation_dim if cfg.asymmetric_observation else None,
        "action_dim": agent.action_dim,
        "config": asdict(cfg),
    }
    with open(directory / "config.json", "w") as stream:
        json.dump(metadata, stream, indent=2)
        stream.write("\n")
    support = agent.support.detach().cpu().reshape(1, 1, -1)

    def network(prefix, keys):
        out = {}
        for key, kind in keys:
            out[key] = support.clone() if kind == "support" else t(f"{prefix}.{key}")
        return out

    def moments(label, store_names, param_names):
        index = {name: i for i, name in enumerate(store_names)}
        m1 = [t(f"optimizer.{label}.m1.{index[n]}") for n in param_names]
        m2 = [t(f"optimizer.{label}.m2.{index[n]}") for n in param_names]
        return m1, m2, float(np.asarray(state[f"optimizer.{label}.timestep"]).reshape(-1)[0])

    nets = (("actor", "actor", actor_module_keys(cfg.actor_num_blocks), agent.actor),
            ("critic", "critic", critic_module_keys(cfg.critic_num_blocks), agent.critic))
    for file_label, prefix, keys, store in nets:
        net = network(prefix, keys)
        names = [k for k, kind in keys if kind == "param"]
        m1, m2, steps = moments(file_label, list(store.shapes), names)
        opt, sched = _optimizer_dicts(cfg, [net[n] for n in names], m1, m2, steps)
        torch.save({"network_state_dict": net, "optimizer_state_dict": opt, "scheduler_state_dict": sched,
                    "update_step": 0}, directory / f"{file_label}.pt")
    target = network("target_critic", critic_module_keys(cfg.critic_num_blocks))
    torch.save({"network_state_dict": target, "optimizer_state_dict": None, "scheduler_state_dict": None,
                "update_step": 0}, directory / "target_critic.pt")
    log_temp = t("log_temperature").reshape(1)
    m1, m2, steps = moments("temperature", ["log_temp"], ["log_temp"])
    opt, sched = _optimizer_dicts(cfg, [log_temp], [m.reshape(1) for m in m1], [m.reshape(1) for m in m2], steps)
    torch.save({"network_state_dict": {"log_temp": log_temp}, "optimizer_state_dict": opt,
                "scheduler_state_dict": sched, "update_step": 0}, directory / "temperature.pt")
    if cfg.normalize_reward:
        running = t("normalizer.running")
        torch.save({"G_r": t("normalizer.returns"), "G_r_max": t("normalizer.maximum").reshape(1),
                    "G_rms_mean": running[0:1].clone(), "G_rms_var": running[1:2].clone(),
                    "G_rms_count": running[2].clone()}, directory / "reward_normalizer.pt")
    scaler = ({"scale": 65536.0, "growth_factor": 2.0, "backoff_factor": 0.5, "growth_interval": 2000,
               "_growth_tracker": 0} if cfg.use_amp else {})
    torch.save({"update_step": int(agent._update_step), "grad_scaler_state_dict": scaler},
               directory / "agent_state.pt")


def _load(path):
    return torch.load(path, map_location="cpu", weights_only=True)


def load(agent, path) -> None:
    """Load the reference's Torch checkpoint directory into the agent (agent.py:556-573)."""
    directory = Path(path)
    cfg = agent.cfg
    metadata = json.loads((directory / "config.json").read_text())
    if metadata["observation_dim"] != agent.observation_dim or metadata["action_dim"] != agent.action_dim:
        raise ValueError("Checkpoint observation/action dimensions differ from this agent.")
    # agent.py:532 records the critic width only for asymmetric observations; a mismatch
    # would surface in the reference as a shape error on the critic embedder
    saved_critic_dim = metadata.get("critic_observation_dim")
    expected_critic_dim = agent.critic_observation_dim if cfg.asymmetric_observation else None
    if saved_critic_dim != expected_critic_dim:
        raise ValueError(f"Checkpoint critic_observation_dim {saved_critic_dim} differs from this agent's "
                         f"{expected_critic_dim}.")
    state = agent.state_dict(include_replay=False)

    def put(key, value):
        current = np.asarray(state[key])
        value = torch.as_tensor(value).detach().cpu().to(torch.float32).numpy()
        if value.size != current.size:
            raise ValueError(f"Checkpoint tensor for {key} has {value.size} values, the agent expects {current.size}.")
        state[key] = value.reshape(current.shape).astype(current.dtype)

    def network(prefix, keys, saved):
        saved = {k.removeprefix("_orig_mod."): v for k, v in saved.items()}
        expected = {k for k, _ in keys}
        if set(saved) != expected:
            raise ValueError(f"{prefix} checkpoint keys differ from this agent's networks: "
                             f"{sorted(set(saved) ^ expected)}")
        for key, kind in keys:
            if kind == "support":
                if not torch.allclose(saved[key].reshape(-1).float().cpu(), agent.support.cpu(), atol=1e-6):
                    raise ValueError("Checkpoint critic support differs from this agent's configuration.")
                continue
            put(f"{prefix}.{key}", saved[key])

    def optimizer(label, store_names, param_names, ckpt):
        opt, sched = ckpt.get("optimizer_state_dict"), ckpt.get("scheduler_state_dict")
        if opt is None:
            return
        groups = opt["param_groups"]
        if len(groups) != 1 or len(groups[0]["params"]) != len(param_names):
            raise ValueError(f"{label} optimizer state does not match this agent's parameters.")
        index = {name: i for i, name in enumerate(store_names)}
        steps = 0.0
        for position, name in enumerate(param_names):
            entry = opt["state"].get(groups[0]["params"][position])
            i = index[name]
            if entry is None:  # no step taken yet
                put(f"optimizer.{label}.m1.{i}", torch.zeros(np.asarray(state[f"optimizer.{label}.m1.{i}"]).shape))
                put(f"optimizer.{label}.m2.{i}", torch.zeros(np.asarray(state[f"optimizer.{label}.m2.{i}"]).shape))
                continue
            put(f"optimizer.{label}.m1.{i}", entry["exp_avg"])
            put(f"optimizer.{label}.m2.{i}", entry["exp_avg_sq"])
            steps = float(entry["step"])
        put(f"optimizer.{label}.timestep", torch.tensor([steps]))
        lr = (sched or {}).get("_last_lr", [groups[0]["lr"]])[0]
        put(f"optimizer.{label}.lr", torch.tensor([float(lr)]))

    actor_keys = actor_module_keys(cfg.actor_num_blocks)
    critic_keys = critic_module_keys(cfg.critic_num_blocks)
    actor = _load(directory / "actor.pt")
    critic = _load(directory / "critic.pt")
    target = _load(directory / "target_critic.pt")
    temperature = _load(directory / "temperature.pt")
    network("actor", actor_keys, actor["network_state_dict"])
    network("critic", critic_keys, critic["network_state_dict"])
    network("target_critic", critic_keys, target["network_state_dict"])
    put("log_temperature", temperature["network_state_dict"]["log_temp"])
    if cfg.load_optimizer:
        optimizer("actor", list(agent.actor.shapes), [k for k, kind in actor_keys if kind == "param"], actor)
        optimizer("critic", list(agent.critic.shapes), [k for k, kind in critic_keys if kind == "param"], critic)
        optimizer("temperature", ["log_temp"], ["log_temp"], temperature)
        agent_state = _load(directory / "agent_state.pt")
        counters = np.asarray(state["update_counters"]).copy()
        counters[0] = int(agent_state["update_step"])
        state["update_counters"] = counters
    if cfg.normalize_reward and cfg.load_reward_normalizer:
        # the reference opens reward_normalizer.pt unconditionally here (agent.py:570-572)
        if not (directory / "reward_normalizer.pt").exists():
            raise FileNotFoundError(f"{directory / 'reward_normalizer.pt'} is missing; set load_reward_normalizer="
                                    "False to keep this agent's reward statistics.")
        normalizer = _load(directory / "reward_normalizer.pt")
        put("normalizer.maximum", torch.as_tensor(normalizer["G_r_max"]).reshape(1))
        put("normalizer.running", torch.stack([torch.as_tensor(normalizer[k]).reshape(()).float()
                                               for k in ("G_rms_mean", "G_rms_var", "G_rms_count")]))
        state.pop("normalizer.returns", None)  # returns restart at zero (agent.py:570-572)
    agent.load_state_dict(state)


def save_replay_buffer(agent, path) -> None:
    """replay_buffer.pt as TorchUniformBuffer.save writes it (replay.py:196-216)."""
    directory = Path(path)
    directory.mkdir(parents=True, exist_ok=True)
    if agent.replay is None:
        raise RuntimeError("The replay buffer is empty.")
    n = agent._num_in_buffer_host
    dataset = {key: agent.replay[key][:n].detach().cpu().clone() for key in
               ("observation", "action", "reward", "terminated", "truncated", "next_observation", "discount")}
    dataset["num_in_buffer"] = n
    dataset["current_idx"] = agent._replay_position
    torch.save(dataset, directory / "replay_buffer.pt")


def load_replay_buffer(agent, path) -> None:
    """Restore replay_buffer.pt (replay.py:218-240); in-flight n-step staging starts empty."""
    dataset = _load(Path(path) / "replay_buffer.pt")
    n = int(dataset["num_in_buffer"])
    if n > agent.capacity:
        raise ValueError("Saved replay buffer exceeds the configured capacity.")
    agent.load_replay({key: dataset[key] for key in
                       ("observation", "action", "reward", "terminated", "truncated", "next_observation", "discount")},
                      count=n, position=int(dataset["current_idx"]) % agent.capacity)
