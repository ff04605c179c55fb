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


def _pcg_scalar(v):
    """The published PCG-RXS-M-XS hash (Jarzynski and Olano 2020) on one Python integer mod 2^32."""
    b = (v * 747796405 + 2891336453) & 0xFFFFFFFF
    c = (((b >> ((b >> 28) + 4)) ^ b) * 277803737) & 0xFFFFFFFF
    return (c >> 22) ^ c


def test_warp_rng_states_are_distinct_per_element():
    """The Warp learner draws row i's noise from state i (robolearn/warp/flashsac.py:44-50), so the
    checkpoint's RNG arrays must hold a distinct state per element, seeded per stream as the Warp
    constructor does (seed + 11, 23, 37, 41; the replay's own seed)."""
    import numpy as np

    from robolearn_amd.warp_checkpoint import warp_rng_states

    seed = 5
    arrays = {offset: warp_rng_states(seed + offset, 4096) for offset in (0, 11, 23, 37, 41)}
    for offset, states in arrays.items():
        assert states.dtype == np.uint32 and states.shape == (4096,)
        assert len(np.unique(states)) == states.size, offset
        # the vectorized wrap-around arithmetic equals the scalar hash composition
        for i in (0, 1, 2, 4095):
            assert int(states[i]) == _pcg_scalar((seed + offset + _pcg_scalar(i)) & 0xFFFFFFFF)
    assert len(np.unique(np.concatenate(list(arrays.values())))) == 5 * 4096
    np.testing.assert_array_equal(warp_rng_states(seed, 16), warp_rng_states(seed, 16))
