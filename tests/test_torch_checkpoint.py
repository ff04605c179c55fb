"""The reference Torch checkpoint layout, checked on the CPU against the fixture
written by the reference's own Network.save (tests/golden/make_torch_checkpoint.py)."""

import json
from pathlib import Path

import pytest
import torch

from robolearn_amd import torch_checkpoint as TC

FIXTURE = Path(__file__).resolve().parent / "golden" / "torch_checkpoint"


def _load(name):
    return torch.load(FIXTURE / name, map_location="cpu", weights_only=True)


@pytest.mark.parametrize("name,keys", [("actor.pt", TC.actor_module_keys(1)), ("critic.pt", TC.critic_module_keys(2)),
                                       ("target_critic.pt", TC.critic_module_keys(2))])
def test_module_key_order_matches_reference_files(name, keys):
    ckpt = _load(name)
    assert list(ckpt["network_state_dict"]) == [k for k, _ in keys]
    params = [k for k, kind in keys if kind == "param"]
    if ckpt["optimizer_state_dict"] is not None:
        group = ckpt["optimizer_state_dict"]["param_groups"][0]
        assert group["params"] == list(range(len(params)))
        state = ckpt["optimizer_state_dict"]["state"]
        for i, key in enumerate(params):  # Adam index i belongs to the i-th parameter of the module
            assert state[i]["exp_avg"].shape == ckpt["network_state_dict"][key].shape, key


def test_schedule_matches_reference_scheduler_state():
    from robolearn_amd.config import FlashSACConfig

    meta = json.loads((FIXTURE / "config.json").read_text())
    config = {k: v for k, v in meta["config"].items() if k in FlashSACConfig.__dataclass_fields__}
    cfg = FlashSACConfig(**config)
    sched = _load("actor.pt")["scheduler_state_dict"]
    lr = TC._schedule(cfg)
    assert sched["_last_lr"][0] == pytest.approx(lr(sched["last_epoch"]), rel=1e-12)
    # the dicts written for the same step count have the reference's structure
    params = [torch.zeros(3)]
    opt, written = TC._optimizer_dicts(cfg, params, [torch.ones(3)], [torch.ones(3)], sched["last_epoch"])
    assert set(written) == set(sched) and written["last_epoch"] == sched["last_epoch"]
    assert written["_step_count"] == sched["_step_count"]
    assert written["_last_lr"][0] == pytest.approx(sched["_last_lr"][0], rel=1e-12)
    reference_group = _load("actor.pt")["optimizer_state_dict"]["param_groups"][0]
    assert set(opt["param_groups"][0]) == set(reference_group)
    assert opt["param_groups"][0]["lr"] == pytest.approx(reference_group["lr"], rel=1e-12)
    assert set(opt["state"][0]) == {"step", "exp_avg", "exp_avg_sq"}
