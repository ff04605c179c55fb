"""Warp <-> Torch critic key names of the robolearn-warp-flashsac-v1 format, on the CPU.

warp_critic_name must be the inverse of the reference's mapping from a Warp
critic key to the Torch ensemble key (robolearn/warp/_flash_networks.py:690-694)
on every key of the reference-written critic fixture, and injective.
"""

from pathlib import Path

import torch

from robolearn_amd.warp_checkpoint import warp_critic_name

FIXTURE = Path(__file__).resolve().parent / "golden" / "torch_checkpoint"


def _reference_to_torch_name(warp_name):
    return warp_name.replace(".w.w.weight", ".w.weight").replace(".w1.w.weight", ".w1.weight").replace(
        ".w2.w.weight", ".w2.weight")


def test_critic_names_invert_the_reference_mapping():
    keys = list(torch.load(FIXTURE / "critic.pt", map_location="cpu", weights_only=True)["network_state_dict"])
    warp = [warp_critic_name(k) for k in keys]
    assert len(set(warp)) == len(keys)
    for torch_key, warp_key in zip(keys, warp):
        assert _reference_to_torch_name(warp_key) == torch_key
    # unit linears carry the Warp Linear's own ".w" level
    assert warp_critic_name("embedder.w.weight") == "embedder.w.w.weight"
    assert warp_critic_name("encoder.1.w2.weight") == "encoder.1.w2.w.weight"
    assert warp_critic_name("predictor.w.weight") == "predictor.w.w.weight"
    assert warp_critic_name("encoder.0.norm1.running_var") == "encoder.0.norm1.running_var"
