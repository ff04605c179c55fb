"""The oracle's parity-test hooks (oracle.flashsac.Emulation) on the CPU.

The GPU parity tests compare a device update with the oracle under two hooks: the device's ReLU
decisions forced into the oracle, and the device's bf16 roundings.  These tests pin the hooks
themselves, so that a hook that silently changed the update (or did nothing) would be caught:

* forcing the oracle's own natural decisions reproduces the unforced update bit for bit, and
  flipping one forced decision changes the gradients;
* the bf16 product equals the textbook product of the rounded operands, its backward feeds both
  backward products from the rounded output gradient, and with bf16 activations the stored output
  and the gradient at the second block product's input are rounded too;
* the after-actor-phase hook runs once, between the temperature step and the critic phase.
"""


import pytest
import torch

from oracle import flashsac as O
from robolearn_amd.config import FlashSACConfig


def _setup(seed=4):
    from dataclasses import replace

    cfg = FlashSACConfig(seed=0, normalize_reward=False, n_step=1, sample_batch_size=8, buffer_max_length=32,
                         buffer_min_length=8, actor_hidden_dim=8, actor_num_blocks=1, critic_hidden_dim=8,
                         critic_num_blocks=2, critic_num_bins=7, critic_min_v=-4.0, critic_max_v=4.0)
    cfg = replace(cfg, temp_target_entropy=O.target_entropy(2, cfg.temp_target_sigma))
    d = O.dims_from_config(3, 2, cfg)
    state = O.init_state(d, cfg, seed=seed, dtype=torch.float64)
    store = O.synthetic_replay(32, 3, 2, seed=1, gamma=0.99, done_prob=0.2)
    batch = {k: v.double() for k, v in O.sample(store, torch.arange(8)).items()}
    g = torch.Generator().manual_seed(3)
    return cfg, d, state, batch, torch.randn(16, 2, generator=g, dtype=torch.float64), \
        torch.randn(8, 2, generator=g, dtype=torch.float64)


def _fresh(cfg, d, state):
    copy = O.OracleState(d, cfg, dtype=torch.float64)
    copy.load_flat(state.flat())
    return copy


def test_forcing_the_natural_decisions_reproduces_the_update_exactly():
    cfg, d, state, batch, an, nn = _setup()
    recorded, plain, forced = [], {}, {}
    a = _fresh(cfg, d, state)
    info_a = O.update(a, batch, an, nn, record=plain, emulation=O.Emulation(record_masks=recorded))
    # actor (1 block) + eval critic (2) + next-action actor (1) + target critic (2) + online critic (2),
    # two ReLUs per block
    assert len(recorded) == 2 * (1 + 2 + 1 + 2 + 2)
    b = _fresh(cfg, d, state)
    em = O.Emulation(relu_masks=recorded)
    info_b = O.update(b, batch, an, nn, record=forced, emulation=em)
    assert em.used == len(recorded)
    for key in info_a:
        assert info_a[key].item() == info_b[key].item(), key
    for group in ("actor_grads", "critic_grads"):
        for name, value in plain[group].items():
            assert torch.equal(value, forced[group][name]), (group, name)
    # and the hooks with nothing forced equal no emulation at all
    c, none = _fresh(cfg, d, state), {}
    O.update(c, batch, an, nn, record=none)
    for name, value in none["critic_grads"].items():
        assert torch.equal(value, plain["critic_grads"][name]), name


def test_a_flipped_forced_decision_changes_the_gradients():
    cfg, d, state, batch, an, nn = _setup()
    recorded = []
    O.update(_fresh(cfg, d, state), batch, an, nn, emulation=O.Emulation(record_masks=recorded))
    flipped = [m.clone() for m in recorded]
    # the online critic's last ReLU: flip one passed element
    mask = flipped[-1]
    index = tuple(int(i) for i in torch.nonzero(mask)[0])
    mask[index] = False
    base, changed = {}, {}
    O.update(_fresh(cfg, d, state), batch, an, nn, record=base, emulation=O.Emulation(relu_masks=recorded))
    O.update(_fresh(cfg, d, state), batch, an, nn, record=changed, emulation=O.Emulation(relu_masks=flipped))
    differs = [name for name, value in base["critic_grads"].items()
               if not torch.equal(value, changed["critic_grads"][name])]
    assert differs
    with pytest.raises(ValueError):
        O.update(_fresh(cfg, d, state), batch, an, nn, emulation=O.Emulation(relu_masks=recorded[:-1]))


def test_bf16_product_rounds_operands_and_output_gradient():
    g = torch.Generator().manual_seed(7)
    x = torch.randn(2, 5, 6, generator=g, dtype=torch.float64, requires_grad=True)
    w = torch.randn(2, 4, 6, generator=g, dtype=torch.float64, requires_grad=True)
    dy = torch.randn(2, 5, 4, generator=g, dtype=torch.float64)
    r = O.round_bf16
    for activations in (False, True):
        em = O.Emulation(bf16=True, bf16_activations=activations)
        y = em.product(x, w, True, output_bf16=True, input_grad_bf16=True)
        exact = torch.einsum("nbi,noi->nbo", r(x.detach()), r(w.detach()))
        assert torch.equal(y.detach(), r(exact) if activations else exact)
        gx, gw = torch.autograd.grad(y, [x, w], dy)
        gx_ref = torch.einsum("nbo,noi->nbi", r(dy), r(w.detach()))
        gw_ref = torch.einsum("nbo,nbi->noi", r(dy), r(x.detach()))
        assert torch.allclose(gw, gw_ref, rtol=1e-14, atol=0)
        assert torch.allclose(gx, r(gx_ref) if activations else gx_ref, rtol=1e-14, atol=0)
    # rounding really happens: bf16 keeps 8 significant bits
    assert O.round_bf16(torch.tensor([1.0 + 2.0 ** -9], dtype=torch.float64)).item() == 1.0
    assert O.round_bf16(torch.tensor([1.0 + 3 * 2.0 ** -9], dtype=torch.float64)).item() == 1.0 + 2.0 ** -7


def test_bf16_emulated_update_stays_near_the_plain_one():
    cfg, d, state, batch, an, nn = _setup()
    plain, low = {}, {}
    O.update(_fresh(cfg, d, state), batch, an, nn, record=plain)
    O.update(_fresh(cfg, d, state), batch, an, nn, record=low,
             emulation=O.Emulation(bf16=True, bf16_activations=True))
    for name, value in plain["critic_grads"].items():
        diff = (low["critic_grads"][name] - value).norm() / value.norm().clamp_min(1e-30)
        assert 0 < diff < 0.5, (name, diff)  # a perturbation of the update, not another algorithm


def test_after_actor_phase_hook_runs_before_the_critic_phase():
    cfg, d, state, batch, an, nn = _setup()
    seen = []

    def hook(s):
        seen.append((s.optimizers["actor"].state[s.actor["embedder.w.w.weight"]]["step"].item(),
                     len(s.optimizers["critic"].state)))
        with torch.no_grad():
            s.log_temp.fill_(-50.0)  # alpha ~ 0: the target's entropy term vanishes

    record = {}
    O.update(_fresh(cfg, d, state), batch, an, nn, record=record, emulation=O.Emulation(after_actor_phase=hook))
    assert seen == [(1.0, 0)]
    assert O.update(_fresh(cfg, d, state), batch, an, nn, do_actor_update=False,
                    emulation=O.Emulation(after_actor_phase=hook)) and len(seen) == 1
    # the critic phase saw the hook's temperature: next-observation entropies are ~0
    reference = {}
    O.update(_fresh(cfg, d, state), batch, an, nn, record=reference)
    assert not torch.equal(record["target_probs"], reference["target_probs"])
