"""The reference Warp learner's checkpoint format, robolearn-warp-flashsac-v1, on the GPU agent.

* Key and shape definition (robolearn/warp/flashsac.py:1085-1239): the saved
  arrays are checked against keys built here from the reference's own Torch
  checkpoint fixture (tests/golden/torch_checkpoint, written by the reference's
  Network.save) through the reference's Warp <-> Torch name mapping
  (robolearn/warp/_flash_networks.py:685-708: the two critics are separate
  networks "critics.<i>", ".w.weight" of a unit linear is ".w.w.weight"), plus
  the optimizer, RNG, exploration, replay and normalizer arrays with the
  reference's shapes and dtypes.
* The stacked [2, ...] critic tensors map member i onto critics.<i>, both ways:
  a Warp-layout archive assembled from the fixture's tensors loads into the
  agent exactly.
* save -> load round trip in place with the captured graph alive: the restored
  state equals the saved one bit for bit and the next update (graph replay)
  equals an update of a fresh agent loaded from the same files.
* Loading without replay resets the replay, as the reference does.
"""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import flashsac as O
from robolearn_amd import warp_checkpoint as WC

pytestmark = pytest.mark.gpu

FIXTURE = Path(__file__).resolve().parent / "golden" / "torch_checkpoint"
OBS, ACT, ENVS = 4, 2, 3


def _reference_to_torch_name(warp_name):
    """The reference's own mapping from a Warp critic key to the Torch key (_flash_networks.py:690-694)."""
    return warp_name.replace(".w.w.weight", ".w.weight").replace(".w1.w.weight", ".w1.weight").replace(
        ".w2.w.weight", ".w2.weight")


def _fixture(name):
    return torch.load(FIXTURE / name, map_location="cpu", weights_only=True)


def _agent(cls_name="WarpFlashSAC", **overrides):
    from robolearn_amd import flashsac
    from robolearn_amd.config import FlashSACConfig

    meta = json.loads((FIXTURE / "config.json").read_text())
    config = {k: v for k, v in meta["config"].items() if k in FlashSACConfig.__dataclass_fields__}
    config.update(buffer_max_length=256, buffer_min_length=32, sample_batch_size=16)
    config.update(overrides)
    return getattr(flashsac, cls_name)(OBS, ACT, num_envs=ENVS, cfg=FlashSACConfig(**config))


def _fill(agent, seed=3):
    store = O.synthetic_replay(200, OBS, ACT, seed=seed, gamma=agent.cfg.gamma, done_prob=0.1)
    agent.load_replay({k: v.numpy() for k, v in store.items()})


def test_warp_arrays_follow_the_reference_definition(gpu, tmp_path):
    print("case warp checkpoint key/shape definition", flush=True)
    agent = _agent()
    agent.save(tmp_path / "ckpt")  # WarpFlashSAC's default format
    meta = json.loads((tmp_path / "ckpt" / "config.json").read_text())
    assert meta["format"] == "robolearn-warp-flashsac-v1" and meta["replay_included"] is False
    assert meta["observation_dim"] == OBS and meta["action_dim"] == ACT and meta["num_envs"] == ENVS
    # a backend the reference's WarpFlashSAC constructor accepts with fused updates (flashsac.py:354-358)
    assert meta["dense_backend"] == "cuda" and meta["fused_updates"] is True
    with np.load(tmp_path / "ckpt" / "agent.npz", allow_pickle=False) as archive:
        saved = {k: archive[k] for k in archive.files}
    actor_keys = list(_fixture("actor.pt")["network_state_dict"])
    critic_state = _fixture("critic.pt")["network_state_dict"]
    expected = {}
    for key in actor_keys:
        expected[f"actor.{key}"] = (tuple(_fixture("actor.pt")["network_state_dict"][key].shape), np.float32)
    for prefix in ("critic", "target_critic"):
        for member in range(2):
            names = [k for k in saved if k.startswith(f"{prefix}.critics.{member}.")]
            mapped = {_reference_to_torch_name(k.split(".", 3)[3]): k for k in names}
            assert set(mapped) == set(critic_state), (prefix, member)
            for torch_key, warp_key in mapped.items():
                shape = tuple(critic_state[torch_key].shape)
                shape = (shape[-1],) if torch_key == "predictor.bin_values" else shape[1:]
                expected[warp_key] = (shape, np.float32)
    actor_params = [k for k in actor_keys if "running" not in k]
    critic_params = [k for k in critic_state if "running" not in k and k != "predictor.bin_values"]
    B, E = agent.batch_size, ENVS
    for name, params, store in (("actor", [(k, None) for k in actor_params], agent.actor),
                                ("critic", [(k, i) for i in range(2) for k in critic_params], agent.critic),
                                ("temperature", [("log_temp", None)], agent.temperature)):
        for j, (key, member) in enumerate(params):
            shape = tuple(store.shapes[key]) if member is None else tuple(store.shapes[key])[1:]
            expected[f"optimizer.{name}.m1.{j}"] = (shape, np.float32)
            expected[f"optimizer.{name}.m2.{j}"] = (shape, np.float32)
        expected[f"optimizer.{name}.timestep"] = ((1,), np.float32)
        expected[f"optimizer.{name}.lr"] = ((1,), np.float32)
    expected.update({
        "log_temperature": ((1,), np.float32), "update_counters": ((3,), np.int64),
        "rng.actor": ((2 * B,), np.uint32), "rng.next": ((B,), np.uint32), "rng.exploration": ((E,), np.uint32),
        "rng.repeat": ((1,), np.uint32), "exploration.repetition": ((2,), np.int32),
        "exploration.cached_noise": ((E, ACT), np.float32), "normalizer.returns": ((E,), np.float32),
        "normalizer.maximum": ((1,), np.float32), "normalizer.running": ((3,), np.float32),
        "replay_storage_included": ((1,), np.bool_),
    })
    extra = set(saved) - set(expected)
    assert extra == {"mi355x.exploration_step"}, extra
    for key, (shape, dtype) in expected.items():
        assert key in saved, key
        assert saved[key].shape == shape and saved[key].dtype == dtype, (key, saved[key].shape, saved[key].dtype)
    # the Warp learner draws row i from state i (robolearn/warp/flashsac.py:44-50): distinct states
    for key in ("rng.actor", "rng.next", "rng.exploration"):
        assert len(np.unique(saved[key])) == saved[key].size, key
    np.testing.assert_array_equal(saved["rng.actor"], WC.warp_rng_states(agent.cfg.seed + 11, 2 * B))
    # the module definition agrees with the one the loader validates against
    assert {k: v[0] for k, v in WC.state_keys(agent, include_replay=False).items()
            if not k.startswith("replay.")} == {k: v[0] for k, v in expected.items()}
    # member i of every stacked tensor is critics.<i>
    state = agent.state_dict(include_replay=False)
    for member in range(2):
        for torch_key in critic_params + ["embedder.norm.running_mean", "encoder.1.norm2.running_var"]:
            warp_key = f"critic.critics.{member}.{WC.warp_critic_name(torch_key)}"
            np.testing.assert_array_equal(saved[warp_key], state[f"critic.{torch_key}"][member], err_msg=warp_key)


def test_fixture_tensors_load_through_the_warp_layout(gpu, tmp_path):
    """A Warp-layout archive assembled from the reference-written Torch fixture loads member by member."""
    print("case warp checkpoint from the reference fixture's tensors", flush=True)
    agent = _agent(load_optimizer=False)
    WC.save(agent, tmp_path / "ckpt")
    archive = dict(np.load(tmp_path / "ckpt" / "agent.npz", allow_pickle=False))
    fixtures = {"actor": _fixture("actor.pt"), "critic": _fixture("critic.pt"),
                "target_critic": _fixture("target_critic.pt")}
    for key, value in fixtures["actor"]["network_state_dict"].items():
        archive[f"actor.{key}"] = value.numpy()
    for prefix in ("critic", "target_critic"):
        for key, value in fixtures[prefix]["network_state_dict"].items():
            for member in range(2):
                warp_key = f"{prefix}.critics.{member}.{WC.warp_critic_name(key)}"
                archive[warp_key] = value.numpy().reshape(-1) if key == "predictor.bin_values" else value[member].numpy()
    with (tmp_path / "ckpt" / "agent.npz").open("wb") as stream:
        np.savez(stream, **archive)
    agent.load(tmp_path / "ckpt")
    state = agent.state_dict(include_replay=False)
    for prefix in ("actor", "critic", "target_critic"):
        for key, value in fixtures[prefix]["network_state_dict"].items():
            if key == "predictor.bin_values":
                continue
            np.testing.assert_array_equal(state[f"{prefix}.{key}"].reshape(value.shape), value.numpy(),
                                          err_msg=f"{prefix}.{key}")


def test_warp_checkpoint_round_trip_under_live_graph(gpu, tmp_path):
    print("case warp checkpoint round trip with captured graphs", flush=True)
    agent = _agent()
    _fill(agent)
    agent.update()  # captures both phase graphs
    agent.update()
    agent.act(torch.randn(ENVS, OBS, device=gpu))
    agent.save(tmp_path / "ckpt", include_replay=True)
    saved = agent.state_dict(include_replay=True)
    # exploration_state = (repetition count, repetition length, refreshed-this-call flag): the flag is
    # written and read within one act() call, so only the first two travel (as the reference's
    # exploration.repetition)
    saved_exploration = (agent.exploration_state[:2].clone(), agent.exploration_noise.clone(),
                         agent.exploration_step.clone())
    agent.update()
    agent.update()
    agent.load(tmp_path / "ckpt")
    restored = agent.state_dict(include_replay=True)
    assert saved.keys() == restored.keys()
    for key in saved:
        np.testing.assert_array_equal(saved[key], restored[key], err_msg=key)
    for before, after in zip(saved_exploration, (agent.exploration_state[:2], agent.exploration_noise,
                                                 agent.exploration_step)):
        assert torch.equal(before, after)
    other = _agent()
    other.load(tmp_path / "ckpt")
    a = agent.update()  # graph replay on the restored buffers
    b = other.update(capture=False)
    torch.cuda.synchronize()
    assert a == b
    s1, s2 = agent.state_dict(include_replay=False), other.state_dict(include_replay=False)
    for key in s1:
        np.testing.assert_array_equal(s1[key], s2[key], err_msg=key)


def test_loading_without_replay_resets_it(gpu, tmp_path):
    print("case warp checkpoint without replay", flush=True)
    agent = _agent()
    _fill(agent)
    agent.update()
    agent.save(tmp_path / "ckpt")  # include_replay=False
    agent.load(tmp_path / "ckpt")
    assert not agent.ready and agent.replay_counters.tolist() == [0, 0, 0]
    _fill(agent)
    agent.update()  # the captured graph still runs after the reset and refill
    torch.cuda.synchronize()


def test_precision_switch_needs_load_optimizer_false(gpu, tmp_path):
    print("case warp checkpoint precision switch", flush=True)
    fp32 = _agent()
    fp32.save(tmp_path / "ckpt")
    bf16 = _agent(use_amp=True)
    with pytest.raises(ValueError, match="precision"):
        bf16.load(tmp_path / "ckpt")
    _agent(use_amp=True, load_optimizer=False).load(tmp_path / "ckpt")
