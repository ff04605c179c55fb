"""The bandwidth-bound kernels at the BASELINE.json configs[4] sweep shapes (the
shapes bench.py times), checked against float64 references.

(a) fused min-Q target + two-hot projection + cross-entropy + d-logits, 65536
    rows x 101 bins, twin critics, against oracle.flashsac's
    categorical_td_target (robolearn/flashsac/updates.py:19-80, 248-257);
(b) the fused Adam + unit-row projection + EMA step over 48 tensors (~25.2 M
    parameters, 1024 x 1024 and 4096 x 256 weights with their biases) against
    torch.optim.Adam in float64 (robolearn/flashsac/agent.py:64-65), F.normalize
    rows with eps 1e-8 (layers.py:24-29) and lerp by tau (network.py:66-80);
(c) RMSNorm forward and backward on 65536 x 1024 against float64 autograd of
    x / sqrt(mean(x^2) + 1e-6) * w (layers.py:67-74).
"""

import math
from collections import OrderedDict

import pytest
import torch
import torch.nn.functional as F

from oracle import flashsac as O
from robolearn_amd import kernels as K

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("B, bins", [(65536, 101), (2048, 513), (1024, 1024), (256, 4096)])
def test_td_cross_entropy_at_sweep_shape(gpu, B, bins):
    """configs[4](a) at 65536 x 101, and the one-workgroup-per-row path for wider heads (up to the
    reference's 4096-bin limit, robolearn/cuda/categorical_kernels.cuh:164-166)."""
    print(f"case td_cross_entropy {B} x {bins}", flush=True)
    min_v, max_v = -10.0, 10.0
    g = torch.Generator().manual_seed(41 + bins)
    target_logits = torch.randn(2, B, bins, generator=g)
    online_logits = torch.randn(2, B, bins, generator=g)
    # returns r + gamma (z - alpha logpi) spread like N(0, 5) and clipped at the support ends
    reward = torch.randn(B, generator=g) * 5.0
    terminated = (torch.rand(B, generator=g) < 0.01).float()
    discount = torch.full((B,), 0.99)
    next_log_probs = torch.randn(B, generator=g)
    alpha = torch.tensor([0.01])
    support = torch.linspace(min_v, max_v, bins)
    d = {k: v.to(gpu).contiguous() for k, v in dict(tl=target_logits, ol=online_logits, r=reward, t=terminated,
                                                     disc=discount, nlp=next_log_probs, a=alpha, z=support).items()}
    dlogits = torch.empty(2, B, bins, device=gpu)
    loss_rows, entropy_rows = torch.empty(2, B, device=gpu), torch.empty(B, device=gpu)
    target_out, q_next = torch.empty(B, bins, device=gpu), torch.empty(2, B, device=gpu)
    scale = 1.0 / B
    K.td_cross_entropy(d["tl"], None, B, d["ol"], None, B, d["z"], d["r"], d["t"], d["disc"], d["nlp"], d["a"],
                       min_v=min_v, max_v=max_v, batch=B, bins=bins, scale=scale, dlogits=dlogits,
                       loss_rows=loss_rows, entropy_rows=entropy_rows, target_out=target_out, q_next=q_next)
    torch.cuda.synchronize()
    lp_target = torch.log_softmax(target_logits.double(), -1)
    z = support.double()
    q = (lp_target.exp() * z).sum(-1)
    selected = O.select_min_q_log_probs(q, lp_target)
    entropy = alpha.double() * next_log_probs.double()
    expected = O.categorical_td_target(selected, reward.double(), terminated.double(), entropy, discount.double(),
                                       bins, min_v, max_v)
    torch.testing.assert_close(q_next.cpu().double(), q, rtol=1e-5, atol=1e-5)
    # The kernel forms the return v = r + gamma (z - alpha logpi)(1 - d) in fp32 (as the reference does):
    # with |r| up to ~25 here, v carries a few ulps of 2^-24 * 32, so each source bin's split fraction
    # b = (v - min_v) / width may differ from float64 by db.  Source j splits its mass p_j over bins
    # l_j and l_j + 1, so the mass moved into or out of bin k is at most db times the mass of the
    # sources landing on bins k - 1 .. k + 1: |dt_k| <= 2 db (t_{k-1} + t_k + t_{k+1}).
    bin_width = (max_v - min_v) / (bins - 1)
    db = 4 * 2.0 ** -24 * 32.0 / bin_width
    padded = torch.nn.functional.pad(expected, (1, 1))
    local = padded[:, :-2] + padded[:, 1:-1] + padded[:, 2:]
    mass_tol = 2 * db * local + 1e-7
    got = target_out.cpu().double()
    assert bool(((got - expected).abs() <= mass_tol).all()), ((got - expected).abs() / mass_tol).max().item()
    torch.testing.assert_close(got.sum(-1), torch.ones(B, dtype=torch.float64), rtol=0, atol=1e-5)
    lp_online = torch.log_softmax(online_logits.double(), -1)
    # the loss rows inherit the mass error times |log p|
    loss_tol = (mass_tol[None] * lp_online.abs()).sum(-1) + 1e-5 * (expected[None] * lp_online).sum(-1).abs()
    loss_ref = -(expected[None] * lp_online).sum(-1)
    assert bool(((loss_rows.cpu().double() - loss_ref).abs() <= loss_tol).all())
    grad = scale * (lp_online.exp() * expected.sum(-1, keepdim=True)[None] - expected[None])
    grad_tol = scale * (mass_tol[None] + lp_online.exp() * mass_tol.sum(-1, keepdim=True)[None]) + 1e-4 * grad.abs()
    assert bool(((dlogits.cpu().double() - grad).abs() <= grad_tol + 1e-9).all())
    torch.testing.assert_close(entropy_rows.cpu().double(), entropy, rtol=1e-6, atol=0)


def test_fused_optimizer_at_sweep_shape(gpu):
    print("case c4b fused Adam + projection + EMA, 48 tensors", flush=True)
    from robolearn_amd.config import FlashSACConfig
    from robolearn_amd.networks import FlatStore, FusedOptimizer

    shapes, kinds = OrderedDict(), {}
    for i in range(24):
        out, inp = ((1024, 1024), (4096, 256))[i % 2]
        shapes[f"layer{i}.weight"] = (out, inp)
        shapes[f"layer{i}.bias"] = (out,)
        kinds[f"layer{i}.weight"], kinds[f"layer{i}.bias"] = 0, 3
    count = sum(math.prod(s) for s in shapes.values())
    assert len(shapes) == 48 and 25_000_000 < count < 25_500_000
    g = torch.Generator(device=gpu).manual_seed(11)
    store = FlatStore(shapes, gpu, target=True)
    store.param.normal_(0.0, 0.05, generator=g)
    store.target.copy_(store.param)
    store.target.add_(torch.randn(store.target.shape, generator=g, device=gpu), alpha=1e-3)
    store.grad.normal_(0.0, 1e-3, generator=g)
    store.m1.normal_(0.0, 1e-4, generator=g)
    store.m2.copy_(store.m1 * store.m1)
    host = {name: {k: store.view(getattr(store, k), name).cpu().double() for k in ("param", "grad", "m1", "m2",
                                                                                  "target")} for name in shapes}
    lr, tau = 3e-4, 0.005
    cfg = FlashSACConfig(learning_rate_init=lr, learning_rate_peak=lr, learning_rate_end=lr)
    optimizer = FusedOptimizer(store, cfg, ema_tau=tau, kinds=kinds)
    optimizer.step(adam=True, project=True, ema=True)
    torch.cuda.synchronize()
    params = [torch.nn.Parameter(host[name]["param"].clone()) for name in shapes]
    adam = torch.optim.Adam(params, lr=lr, betas=(0.9, 0.999), eps=1e-8, foreach=False, fused=False)
    for p, name in zip(params, shapes):
        p.grad = host[name]["grad"].clone()
        adam.state[p] = {"step": torch.tensor(0.0), "exp_avg": host[name]["m1"].clone(),
                         "exp_avg_sq": host[name]["m2"].clone()}
    adam.step()
    worst = {}
    for p, name in zip(params, shapes):
        with torch.no_grad():
            expected = F.normalize(p, dim=-1, eps=1e-8) if kinds[name] == 0 else p.detach().clone()
        target = host[name]["target"] + tau * (expected - host[name]["target"])
        st = adam.state[p]
        for label, got, ref in (("param", store.view(store.param, name), expected),
                                ("m1", store.view(store.m1, name), st["exp_avg"]),
                                ("m2", store.view(store.m2, name), st["exp_avg_sq"]),
                                ("target", store.view(store.target, name), target)):
            err = (got.cpu().double() - ref).abs().max().item() / max(ref.abs().max().item(), 1e-30)
            worst[label] = max(worst.get(label, 0.0), err)
            assert err < 1e-5, (name, label, err)
    assert optimizer.timestep.item() == 1.0
    print(f"c4b worst relative error per field: {worst}", flush=True)
    optimizer.close()


def test_rmsnorm_at_sweep_shape(gpu):
    print("case c4c RMSNorm 65536 x 1024", flush=True)
    rows, channels = 65536, 1024
    g = torch.Generator().manual_seed(12)
    x = torch.randn(rows, channels, generator=g)
    w = torch.rand(channels, generator=g) + 0.5
    dy = torch.randn(rows, channels, generator=g)
    xd, wd, dyd = x.to(gpu), w.to(gpu), dy.to(gpu)
    y, dx = torch.empty_like(xd), torch.empty_like(xd)
    ms = torch.empty(rows, device=gpu)
    dw = torch.empty(channels, device=gpu)
    partial = torch.empty(K.chunks(rows) * channels, device=gpu)
    K.rms_forward(xd, wd, ms, y, rows=rows, channels=channels)
    K.rms_backward(xd, dyd, wd, ms, partial, dx, dw, rows=rows, channels=channels)
    torch.cuda.synchronize()
    xr = x.double().requires_grad_(True)
    wr = w.double().requires_grad_(True)
    out = xr / torch.sqrt((xr * xr).mean(-1, keepdim=True) + 1e-6) * wr
    torch.testing.assert_close(y.cpu().double(), out.detach(), rtol=1e-5, atol=1e-5)
    out.backward(dy.double())
    torch.testing.assert_close(dx.cpu().double(), xr.grad, rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(dw.cpu().double(), wr.grad, rtol=1e-4, atol=1e-3)
