"""The reference Warp learner's checkpoint format, robolearn-warp-flashsac-v1, read and written in place.

Layout (robolearn/warp/flashsac.py:1085-1239):
  config.json  format "robolearn-warp-flashsac-v1", precision, observation_dim, action_dim,
               critic_observation_dim (asymmetric only), num_envs, config, the Warp
               constructor flags, replay_included
  agent.npz    NumPy arrays (np.savez, no pickles):
    actor.<key>                      FlashActor.state_dict(): the Torch actor's module keys
                                     (weights, BN running statistics), same shapes
                                     (robolearn/warp/_flash_networks.py:483-528)
    critic.critics.<i>.<key>         FlashDoubleCritic: two separate critics i = 0, 1 whose keys
    target_critic.critics.<i>.<key>  are the Torch ensemble's with ".w.weight" spelled
                                     ".w.w.weight" (".w1"/".w2" likewise), each holding member i
                                     of the stacked [2, ...] tensor; predictor.bin_values is [K]
                                     (_flash_networks.py:583-708, load_author_state_dict)
    optimizer.<net>.m1.<j> / .m2.<j> Adam moments in the network's parameter order; the critic's
                                     run over critics.0 then critics.1
    optimizer.<net>.timestep / .lr   float32 [1] (robolearn/cuda/kernels.cu:44, 310-337)
    optimizer.<net>.amp.<key>        loss-scaler state of the AMP optimizers
                                     (robolearn/cuda/adam.py:64-80)
    log_temperature [1], update_counters int64 [3]
    rng.actor [2B], rng.next [B], rng.exploration [E], rng.repeat [1]   uint32 Warp RNG states
    exploration.repetition int32 [2], exploration.cached_noise [E, A]
    replay.counters int64 [3], replay.rng uint32 [B], replay.pending.<field> [n, E, ...],
    replay.storage.<field> [count, ...] (only with include_replay)
                                     (robolearn/warp/_flash_replay.py:183-344)
    normalizer.returns [E], .maximum [1], .running [3] (with normalize_reward,
                                     _flash_replay.py:446-457)
    replay_storage_included bool [1]

Where the two implementations draw random numbers differently, the arrays keep
their shapes: this backend draws from Philox streams keyed by the seed and its
device counters (the update counters and the exploration step) and ignores the
Warp RNG state arrays on load; the exploration step travels in an extra array
("mi355x.exploration_step") that the reference's loader skips (it reads only its
own keys, flashsac.py:1132-1138).  The Warp learner does read the RNG arrays and
draws row i's noise from state i (flashsac.py:44-50), so they are written as the
per-element states its constructor seeds (flashsac.py:495-501 with offsets 11,
23, 37, 41; _flash_replay.py:216 for replay.rng), see warp_rng_states: every
row and environment of a resumed Warp run gets its own stream.

The order of the Adam moments is the module order of the networks: a module's
own parameters in registration order, then its child modules in registration
order, as the reference's _named_parameters walks them (_flash_networks.py:
300-304); for the actor that is the Torch actor's parameter order.  Warp-NN's own
parameters() order (warp-nn 0.4.0, not in the reference tree) is assumed to walk
the same way: parity unpinned for that index order.
"""

import json
from collections import OrderedDict
from dataclasses import asdict
from pathlib import Path

import numpy as np
import torch

from .torch_checkpoint import actor_module_keys, critic_module_keys

FORMAT = "robolearn-warp-flashsac-v1"
REPLAY_FIELDS = ("observation", "action", "reward", "terminated", "truncated", "next_observation", "discount")
AMP_KEYS = (("loss_scale", np.float32), ("scale_growth_tracker", np.int32), ("found_inf", np.int32),
            ("step_skipped", np.int32), ("attempted_steps", np.int64), ("skipped_steps", np.int64))


def _pcg_hash(state: np.ndarray) -> np.ndarray:
    """The PCG-RXS-M-XS hash of Jarzynski and Olano, "Hash Functions for GPU Rendering", JCGT 9(3),
    2020, on uint32 arrays (wrapping arithmetic)."""
    state = state.astype(np.uint32)
    b = state * np.uint32(747796405) + np.uint32(2891336453)
    c = ((b >> ((b >> np.uint32(28)) + np.uint32(4))) ^ b) * np.uint32(277803737)
    return (c >> np.uint32(22)) ^ c


def warp_rng_states(seed: int, count: int) -> np.ndarray:
    """uint32 generator states for elements 0 .. count - 1 as warp-lang's rand_init(seed, i) builds
    them: the PCG hash of seed + hash(i), the composition warp-lang's open-source rand.h uses
    (warp-lang 1.18.0, not in the reference tree or this image: the exact values are parity
    unpinned; distinct per-element states are what the Warp learner's per-row draws need)."""
    index = np.arange(count, dtype=np.uint32)
    with np.errstate(over="ignore"):
        return _pcg_hash(np.uint32(seed & 0xFFFFFFFF) + _pcg_hash(index))


def warp_critic_name(torch_key: str) -> str:
    """Per-critic Warp key of a Torch ensemble-critic key (inverse of _flash_networks.py:690-694)."""
    for short, long in ((".w1.weight", ".w1.w.weight"), (".w2.weight", ".w2.w.weight"), (".w.weight", ".w.w.weight")):
        if torch_key.endswith(short):
            return torch_key[: -len(short)] + long
    return torch_key


def _network_arrays(agent):
    """(warp key, native key, member or None, is_support) for every network array."""
    cfg = agent.cfg
    rows = []
    for key, kind in actor_module_keys(cfg.actor_num_blocks):
        rows.append((f"actor.{key}", f"actor.{key}", None, False))
    for prefix in ("critic", "target_critic"):
        for member in range(2):
            for key, kind in critic_module_keys(cfg.critic_num_blocks):
                rows.append((f"{prefix}.critics.{member}.{warp_critic_name(key)}", f"{prefix}.{key}", member,
                             kind == "support"))
    return rows


def _optimizer_order(agent):
    """Per optimizer: the native flat-store tensor name and member (None = whole tensor) of moment j."""
    cfg = agent.cfg
    actor = [(k, None) for k, kind in actor_module_keys(cfg.actor_num_blocks) if kind == "param"]
    critic_params = [k for k, kind in critic_module_keys(cfg.critic_num_blocks) if kind == "param"]
    critic = [(k, member) for member in range(2) for k in critic_params]
    return {"actor": (agent.actor, actor), "critic": (agent.critic, critic),
            "temperature": (agent.temperature, [("log_temp", None)])}


def state_keys(agent, include_replay: bool = True) -> "OrderedDict[str, tuple]":
    """Every array the reference writes for this agent: key -> (shape, dtype)."""
    cfg = agent.cfg
    B, E, A, O = agent.batch_size, agent.num_envs, agent.action_dim, agent.critic_observation_dim
    native = agent.state_dict(include_replay=False)
    keys = OrderedDict()
    for warp_key, native_key, member, support in _network_arrays(agent):
        if support:
            shape = (cfg.critic_num_bins,)
        else:
            shape = np.asarray(native[native_key]).shape
            shape = shape[1:] if member is not None else shape
        keys[warp_key] = (tuple(shape), np.float32)
    for name, (store, order) in _optimizer_order(agent).items():
        for j, (tensor, member) in enumerate(order):
            shape = tuple(store.shapes[tensor])
            shape = shape[1:] if member is not None else shape
            keys[f"optimizer.{name}.m1.{j}"] = (shape, np.float32)
            keys[f"optimizer.{name}.m2.{j}"] = (shape, np.float32)
        keys[f"optimizer.{name}.timestep"] = ((1,), np.float32)
        keys[f"optimizer.{name}.lr"] = ((1,), np.float32)
        if cfg.use_amp and name != "temperature":  # robolearn/warp/flashsac.py:452-454: scaled=cfg.use_amp
            for amp_key, dtype in AMP_KEYS:
                keys[f"optimizer.{name}.amp.{amp_key}"] = ((1,), dtype)
    keys["log_temperature"] = ((1,), np.float32)
    keys["update_counters"] = ((3,), np.int64)
    keys["rng.actor"] = ((2 * B,), np.uint32)
    keys["rng.next"] = ((B,), np.uint32)
    keys["rng.exploration"] = ((E,), np.uint32)
    keys["rng.repeat"] = ((1,), np.uint32)
    keys["exploration.repetition"] = ((2,), np.int32)
    keys["exploration.cached_noise"] = ((E, A), np.float32)
    n = cfg.n_step
    keys["replay.counters"] = ((3,), np.int64)
    keys["replay.rng"] = ((B,), np.uint32)
    if include_replay:
        count = agent._num_in_buffer_host
        for field in REPLAY_FIELDS:
            width = O if field in ("observation", "next_observation") else A if field == "action" else None
            keys[f"replay.storage.{field}"] = ((count, width) if width else (count,), np.float32)
    for field, width in (("observation", O), ("action", A), ("next_observation", O)):
        keys[f"replay.pending.{field}"] = ((n, E, width), np.float32)
    for field in ("reward", "terminated", "truncated"):
        keys[f"replay.pending.{field}"] = ((n, E), np.float32)
    if cfg.normalize_reward:
        keys["normalizer.returns"] = ((E,), np.float32)
        keys["normalizer.maximum"] = ((1,), np.float32)
        keys["normalizer.running"] = ((3,), np.float32)
    keys["replay_storage_included"] = ((1,), np.bool_)
    return keys


def to_state(agent, include_replay: bool = True) -> dict:
    """The agent's state as the reference's WarpFlashSAC.state_dict() arrays (flashsac.py:1114-1130)."""
    cfg = agent.cfg
    native = agent.state_dict(include_replay=False)
    state = {}
    for warp_key, native_key, member, support in _network_arrays(agent):
        value = np.asarray(native[native_key]) if not support else agent.support.detach().cpu().numpy()
        if member is not None and not support:
            value = value[member]
        state[warp_key] = np.ascontiguousarray(value, dtype=np.float32)
    for name, (store, order) in _optimizer_order(agent).items():
        for j, (tensor, member) in enumerate(order):
            index = list(store.shapes).index(tensor)
            for moment in ("m1", "m2"):
                value = np.asarray(native[f"optimizer.{name}.{moment}.{index}"])
                state[f"optimizer.{name}.{moment}.{j}"] = np.ascontiguousarray(
                    value[member] if member is not None else value, dtype=np.float32)
        state[f"optimizer.{name}.timestep"] = np.asarray(native[f"optimizer.{name}.timestep"], np.float32)
        state[f"optimizer.{name}.lr"] = np.asarray(native[f"optimizer.{name}.lr"], np.float32)
        if cfg.use_amp and name != "temperature":
            # bf16 operands need no loss scaling: a neutral scaler that a float16 Warp agent can resume
            steps = int(np.asarray(native[f"optimizer.{name}.timestep"]).reshape(-1)[0])
            neutral = {"loss_scale": 65536.0, "scale_growth_tracker": 0, "found_inf": 0, "step_skipped": 0,
                       "attempted_steps": steps, "skipped_steps": 0}
            for amp_key, dtype in AMP_KEYS:
                state[f"optimizer.{name}.amp.{amp_key}"] = np.array([neutral[amp_key]], dtype=dtype)
    state["log_temperature"] = np.asarray(native["log_temperature"], np.float32).reshape(1)
    state["update_counters"] = np.asarray(native["update_counters"], np.int64)
    B, E = agent.batch_size, agent.num_envs
    for key, size, offset in (("rng.actor", 2 * B, 11), ("rng.next", B, 23), ("rng.exploration", E, 37),
                              ("rng.repeat", 1, 41)):
        state[key] = warp_rng_states(cfg.seed + offset, size)
    exploration = agent.exploration_state.cpu().numpy()
    state["exploration.repetition"] = exploration[:2].astype(np.int32)
    state["exploration.cached_noise"] = agent.exploration_noise.cpu().numpy().astype(np.float32)
    state["mi355x.exploration_step"] = agent.exploration_step.cpu().numpy().astype(np.int64)
    agent._ensure_replay()
    state["replay.counters"] = agent.replay_counters.cpu().numpy().astype(np.int64)
    state["replay.rng"] = warp_rng_states(cfg.seed, B)
    if include_replay:
        count = agent._num_in_buffer_host
        for field in REPLAY_FIELDS:
            state[f"replay.storage.{field}"] = agent.replay[field][:count].cpu().numpy()
    pending = agent.pending
    for field in ("observation", "action", "next_observation"):
        state[f"replay.pending.{field}"] = pending[field].cpu().numpy()
    scalars = pending["scalars"].cpu().numpy()
    for column, field in enumerate(("reward", "terminated", "truncated")):
        state[f"replay.pending.{field}"] = np.ascontiguousarray(scalars[..., column])
    if cfg.normalize_reward:
        state["normalizer.returns"] = agent.reward_returns.cpu().numpy().astype(np.float32)
        state["normalizer.maximum"] = agent.reward_max.cpu().numpy().astype(np.float32)
        state["normalizer.running"] = agent.reward_running.cpu().numpy().astype(np.float32)
    state["replay_storage_included"] = np.array([include_replay], dtype=np.bool_)
    return state


def load_state(agent, state: dict) -> None:
    """Restore WarpFlashSAC.state_dict() arrays into the agent in place (flashsac.py:1132-1156): every
    reference key must be present with its shape; captured graphs keep their buffers."""
    cfg = agent.cfg
    restore_storage = bool(np.asarray(state.get("replay_storage_included", [False])).reshape(-1)[0])
    expected = state_keys(agent, include_replay=False)
    for key, (shape, _) in expected.items():
        if key not in state or tuple(np.asarray(state[key]).shape) != tuple(shape):
            raise ValueError(f"Checkpoint array {key} is missing or has the wrong shape.")
    support = np.asarray(state["critic.critics.0.predictor.bin_values"], np.float32)
    if not np.allclose(support, agent.support.cpu().numpy(), atol=1e-6):
        raise ValueError("Checkpoint critic support differs from this agent's configuration.")
    native = agent.state_dict(include_replay=False)
    for warp_key, native_key, member, is_support in _network_arrays(agent):
        if is_support:
            continue
        value = np.asarray(state[warp_key], np.float32)
        if member is None:
            native[native_key] = value.reshape(np.asarray(native[native_key]).shape)
        else:
            target = np.array(native[native_key], copy=True)
            target[member] = value
            native[native_key] = target
    for name, (store, order) in _optimizer_order(agent).items():
        for j, (tensor, member) in enumerate(order):
            index = list(store.shapes).index(tensor)
            for moment in ("m1", "m2"):
                key = f"optimizer.{name}.{moment}.{index}"
                value = np.asarray(state[f"optimizer.{name}.{moment}.{j}"], np.float32)
                if member is None:
                    native[key] = value.reshape(np.asarray(native[key]).shape)
                else:
                    target = np.array(native[key], copy=True)
                    target[member] = value
                    native[key] = target
        native[f"optimizer.{name}.timestep"] = np.asarray(state[f"optimizer.{name}.timestep"], np.float32)
        native[f"optimizer.{name}.lr"] = np.asarray(state[f"optimizer.{name}.lr"], np.float32)
    native["log_temperature"] = np.asarray(state["log_temperature"], np.float32).reshape(1)
    native["update_counters"] = np.asarray(state["update_counters"], np.int64)
    if cfg.normalize_reward:
        native["normalizer.maximum"] = np.asarray(state["normalizer.maximum"], np.float32)
        native["normalizer.running"] = np.asarray(state["normalizer.running"], np.float32)
        native["normalizer.returns"] = np.asarray(state["normalizer.returns"], np.float32)
    agent.load_state_dict(native)
    with torch.no_grad():
        repetition = np.asarray(state["exploration.repetition"], np.int32)
        agent.exploration_state.copy_(torch.tensor([int(repetition[0]), int(repetition[1]), 0], dtype=torch.int32))
        agent.exploration_noise.copy_(torch.as_tensor(np.asarray(state["exploration.cached_noise"], np.float32)))
        if "mi355x.exploration_step" in state:
            agent.exploration_step.copy_(torch.as_tensor(np.asarray(state["mi355x.exploration_step"], np.int64)))
        counters = np.asarray(state["replay.counters"], np.int64)
        if counters.shape != (3,) or counters[0] < 0 or not 0 <= counters[1] < agent.capacity \
                or not 0 <= counters[2] <= agent.capacity:
            raise ValueError("Saved replay counters are incompatible with this buffer.")
        agent._ensure_replay()
        count = int(counters[2])
        if restore_storage and count:
            data = {}
            for field in REPLAY_FIELDS:
                name = f"replay.storage.{field}"
                if name not in state:
                    raise ValueError("A nonempty replay checkpoint must include storage.")
                data[field] = np.asarray(state[name], np.float32)
            agent.load_replay(data, count=count, position=int(counters[1]))
        elif not restore_storage and count and agent._num_in_buffer_host != count:
            raise ValueError("This checkpoint omits replay storage; restore it into an agent holding the same rows.")
        pending = agent.pending
        for field in ("observation", "action", "next_observation"):
            pending[field].copy_(torch.as_tensor(np.asarray(state[f"replay.pending.{field}"], np.float32)))
        for column, field in enumerate(("reward", "terminated", "truncated")):
            pending["scalars"][..., column].copy_(
                torch.as_tensor(np.asarray(state[f"replay.pending.{field}"], np.float32)))
        agent.replay_counters.copy_(torch.as_tensor(counters))
        agent._host_additions = int(counters[0])
        agent._replay_position = int(counters[1])
        agent._num_in_buffer_host = count


def save(agent, path, *, include_replay: bool = False) -> None:
    """WarpFlashSAC.save (flashsac.py:1169-1195)."""
    directory = Path(path)
    directory.mkdir(parents=True, exist_ok=True)
    metadata = {
        "format": FORMAT,
        "precision": agent.compute_dtype,
        "observation_dim": agent.observation_dim,
        "action_dim": agent.action_dim,
        "critic_observation_dim": agent.critic_observation_dim if agent.cfg.asymmetric_observation else None,
        "num_envs": agent.num_envs,
        "config": asdict(agent.cfg),
        "optimized_linear_backward": True,
        # the reference's name for its native dense backend, which this library stands in for: its
        # constructor accepts only "warp" or "cuda" (warp/flashsac.py:354-358), and fused updates
        # and mixed precision need "cuda"
        "dense_backend": "cuda",
        "fused_updates": agent.fused_updates,
        "cuda_autotune": False,
        "fresh_training_gradients": False,
        "replay_included": include_replay,
    }
    torch.cuda.synchronize(agent.device)
    state = to_state(agent, include_replay=include_replay)
    if not include_replay:
        state = {key: value for key, value in state.items() if not key.startswith("replay.")}
    with (directory / "config.json").open("w") as stream:
        json.dump(metadata, stream, indent=2)
        stream.write("\n")
    with (directory / "agent.npz").open("wb") as stream:
        np.savez(stream, **state)


def load(agent, path) -> None:
    """WarpFlashSAC.load (flashsac.py:1197-1239): dimension and precision checks, then an in-place
    restore; without saved replay the replay is reset, as the reference does."""
    directory = Path(path)
    metadata = json.loads((directory / "config.json").read_text())
    if metadata.get("format") != FORMAT:
        raise ValueError("Unrecognized WarpFlashSAC checkpoint format.")
    if metadata["observation_dim"] != agent.observation_dim or metadata["action_dim"] != agent.action_dim:
        raise ValueError("Checkpoint observation/action dimensions differ from this agent.")
    saved_critic_dim = metadata["critic_observation_dim"] or metadata["observation_dim"]
    if saved_critic_dim != agent.critic_observation_dim:
        raise ValueError("Checkpoint critic observation dimension differs from this agent.")
    saved_precision = metadata.get("precision", "float32")
    if saved_precision != agent.compute_dtype and agent.cfg.load_optimizer:
        raise ValueError("Switching checkpoint dense precision requires load_optimizer=False.")
    with np.load(directory / "agent.npz", allow_pickle=False) as archive:
        state = dict(archive)
    if metadata["replay_included"] and metadata["num_envs"] != agent.num_envs:
        raise ValueError("Exact replay continuation requires the original num_envs.")
    current = to_state(agent, include_replay=False)
    if not metadata["replay_included"]:
        agent._ensure_replay()
        agent.load_replay({field: np.zeros((0,), np.float32) for field in REPLAY_FIELDS}, count=0, position=0)
        current = to_state(agent, include_replay=False)
        state.update({key: value for key, value in current.items() if key.startswith("replay.")})
        if metadata["num_envs"] != agent.num_envs:
            for key in ("rng.exploration", "rng.repeat", "exploration.repetition", "exploration.cached_noise",
                        "mi355x.exploration_step"):
                state[key] = current[key]
        if agent.cfg.normalize_reward:
            state["normalizer.returns"] = np.zeros(agent.num_envs, dtype=np.float32)
    if not agent.cfg.load_optimizer:
        state.update({key: value for key, value in current.items() if key.startswith("optimizer.")})
        state["update_counters"] = current["update_counters"]
    if agent.cfg.normalize_reward and not agent.cfg.load_reward_normalizer:
        state.update({key: value for key, value in current.items() if key.startswith("normalizer.")})
    load_state(agent, state)
