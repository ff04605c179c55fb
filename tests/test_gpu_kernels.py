"""HIP primitive kernels against plain PyTorch fp32/fp64 references of the same op."""

import math

import pytest
import torch

from robolearn_amd import kernels as K

pytestmark = pytest.mark.gpu


def _rand(*shape, seed=0, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).float()


def _bf16_round(x):
    return x.to(torch.bfloat16).to(torch.float32)


GEMM_SHAPES = [(1, 5, 7, 3), (2, 130, 129, 40), (2, 257, 96, 160), (1, 64, 101, 256), (2, 300, 37, 123)]


@pytest.mark.parametrize("mode", [K.FP32, K.BF16])
@pytest.mark.parametrize("batch,rows,out_dim,in_dim", GEMM_SHAPES)
def test_linear_products_match_torch(gpu, mode, batch, rows, out_dim, in_dim):
    print(f"case mode={mode} batch={batch} rows={rows} out={out_dim} in={in_dim}", flush=True)
    x = _rand(batch, rows, in_dim, seed=1)
    w = _rand(batch, out_dim, in_dim, seed=2, scale=0.2)
    dy = _rand(batch, rows, out_dim, seed=3)
    bias = _rand(batch, out_dim, seed=4)
    rnd = _bf16_round if mode == K.BF16 else (lambda t: t)
    xd, wd, dyd, bd = (t.to(gpu) for t in (x, w, dy, bias))
    y = torch.empty(batch, rows, out_dim, device=gpu)
    K.linear_forward(xd, wd, y, rows=rows, in_dim=in_dim, out_dim=out_dim, ensemble=batch, bias=bd, mode=mode)
    ref = torch.einsum("bri,boi->bro", rnd(x).double(), rnd(w).double()) + bias.double()[:, None, :]
    tol = 1e-5 if mode == K.FP32 else 1e-5
    torch.testing.assert_close(y.cpu().double(), ref, rtol=tol, atol=tol * math.sqrt(in_dim))

    dx = torch.empty(batch, rows, in_dim, device=gpu)
    K.linear_backward_input(dyd, wd, dx, rows=rows, in_dim=in_dim, out_dim=out_dim, ensemble=batch, mode=mode)
    ref_dx = torch.einsum("bro,boi->bri", rnd(dy).double(), rnd(w).double())
    torch.testing.assert_close(dx.cpu().double(), ref_dx, rtol=tol, atol=tol * math.sqrt(out_dim))

    workspace = torch.empty(64 << 20, device=gpu, dtype=torch.uint8)
    for ws in (None, workspace):
        dw = torch.empty(batch, out_dim, in_dim, device=gpu)
        K.linear_backward_weight(dyd, xd, dw, rows=rows, in_dim=in_dim, out_dim=out_dim, ensemble=batch, mode=mode,
                                 workspace=ws)
        ref_dw = torch.einsum("bro,bri->boi", rnd(dy).double(), rnd(x).double())
        torch.testing.assert_close(dw.cpu().double(), ref_dw, rtol=tol, atol=tol * math.sqrt(rows))


def test_gemm_epilogues_beta_and_broadcast(gpu):
    rows, k, n = 200, 64, 72
    x = _rand(rows, k, seed=5)
    w = _rand(2, n, k, seed=6, scale=0.3)
    c = _rand(2, rows, n, seed=7)
    xd, wd, cd = x.to(gpu), w.to(gpu), c.to(gpu)
    for epilogue, fn in (("relu", torch.relu), ("elu", torch.nn.functional.elu)):
        y = torch.empty(2, rows, n, device=gpu)
        K.linear_forward(xd, wd, y, rows=rows, in_dim=k, out_dim=n, ensemble=2, x_stride=0, epilogue=epilogue,
                         c=cd, beta=1.0)
        ref = fn(torch.einsum("ri,boi->bro", x.double(), w.double())) + c.double()
        torch.testing.assert_close(y.cpu().double(), ref, rtol=1e-5, atol=1e-5)


def test_bf16_operand_tensors(gpu):
    rows, k, n = 96, 128, 64
    x = _rand(rows, k, seed=8).to(torch.bfloat16)
    w = _rand(n, k, seed=9).to(torch.bfloat16)
    y = torch.empty(rows, n, device=gpu)
    K.linear_forward(x.to(gpu), w.to(gpu), y, rows=rows, in_dim=k, out_dim=n, mode=K.BF16)
    ref = x.double() @ w.double().T
    torch.testing.assert_close(y.cpu().double(), ref, rtol=1e-5, atol=1e-4)


@pytest.mark.parametrize("ensemble,rows,channels,relu", [(1, 1000, 5, False), (2, 777, 130, True), (2, 300, 64, True)])
def test_batchnorm_forward_backward_match_autograd(gpu, ensemble, rows, channels, relu):
    x = _rand(ensemble, rows, channels, seed=10, scale=2.0) + 0.5
    w = _rand(ensemble, channels, seed=11).abs() + 0.5
    b = _rand(ensemble, channels, seed=12)
    rm = _rand(ensemble, channels, seed=13) * 0.1
    rv = _rand(ensemble, channels, seed=14).abs() + 0.5
    dy = _rand(ensemble, rows, channels, seed=15)
    g = {name: t.to(gpu).contiguous() for name, t in dict(x=x, w=w, b=b, rm=rm, rv=rv, dy=dy).items()}
    mean = torch.empty(ensemble, channels, device=gpu)
    var = torch.empty_like(mean)
    partial = torch.empty(ensemble * 2 * K.chunks(rows) * channels, device=gpu)
    y = torch.empty(ensemble, rows, channels, device=gpu)
    K.bn_forward(g["x"], g["w"], g["b"], g["rm"], g["rv"], mean, var, partial, y, rows=rows, channels=channels,
                 ensemble=ensemble, relu=relu)
    xr = x.double().requires_grad_(True)
    wr = w.double().requires_grad_(True)
    br = b.double().requires_grad_(True)
    mu = xr.mean(1, keepdim=True)
    vb = xr.var(1, correction=0, keepdim=True)
    out = (xr - mu) * torch.rsqrt(vb + 1e-5) * wr[:, None] + br[:, None]
    if relu:
        out = torch.relu(out)
    torch.testing.assert_close(y.cpu().double(), out.detach(), rtol=1e-5, atol=1e-5)
    unbiased = vb.squeeze(1) * rows / (rows - 1)
    torch.testing.assert_close(g["rm"].cpu().double(), rm.double() + 0.01 * (mu.squeeze(1) - rm.double()),
                               rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(g["rv"].cpu().double(), rv.double() + 0.01 * (unbiased - rv.double()), rtol=1e-5,
                               atol=1e-6)
    out.backward(dy.double())
    sums = torch.empty(2 * ensemble * channels, device=gpu)
    dx = torch.empty_like(y)
    dw = torch.empty_like(mean)
    db = torch.empty_like(mean)
    K.bn_backward(g["x"], g["dy"], y, g["w"], mean, var, partial, sums, dx, dw, db, rows=rows, channels=channels,
                  ensemble=ensemble, relu=relu)
    torch.testing.assert_close(dx.cpu().double(), xr.grad, rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(dw.cpu().double(), wr.grad, rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(db.cpu().double(), br.grad, rtol=1e-4, atol=1e-4)
    # eval mode uses running statistics
    y2 = torch.empty_like(y)
    K.bn_forward(g["x"], g["w"], g["b"], g["rm"], g["rv"], None, None, None, y2, rows=rows, channels=channels,
                 ensemble=ensemble, training=False)
    rmv, rvv = g["rm"].cpu().double(), g["rv"].cpu().double()
    ref2 = (x.double() - rmv[:, None]) / torch.sqrt(rvv[:, None] + 1e-5) * w.double()[:, None] + b.double()[:, None]
    torch.testing.assert_close(y2.cpu().double(), ref2, rtol=1e-5, atol=1e-5)


def test_rmsnorm_and_bias_grad(gpu):
    ensemble, rows, channels = 2, 333, 96
    x = _rand(ensemble, rows, channels, seed=20)
    w = _rand(ensemble, channels, seed=21).abs() + 0.5
    dy = _rand(ensemble, rows, channels, seed=22)
    xd, wd, dyd = x.to(gpu), w.to(gpu), dy.to(gpu)
    ms = torch.empty(ensemble * rows, device=gpu)
    y = torch.empty_like(xd)
    K.rms_forward(xd, wd, ms, y, rows=rows, channels=channels, ensemble=ensemble)
    xr = x.double().requires_grad_(True)
    wr = w.double().requires_grad_(True)
    out = xr / torch.sqrt((xr * xr).mean(-1, keepdim=True) + 1e-6) * wr[:, None]
    torch.testing.assert_close(y.cpu().double(), out.detach(), rtol=1e-5, atol=1e-5)
    out.backward(dy.double())
    partial = torch.empty(ensemble * K.chunks(rows) * channels, device=gpu)
    dx = torch.empty_like(xd)
    dw = torch.empty(ensemble, channels, device=gpu)
    K.rms_backward(xd, dyd, wd, ms, partial, dx, dw, rows=rows, channels=channels, ensemble=ensemble)
    torch.testing.assert_close(dx.cpu().double(), xr.grad, rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(dw.cpu().double(), wr.grad, rtol=1e-4, atol=1e-4)
    db = torch.empty(ensemble, channels, device=gpu)
    K.bias_grad(dyd, db, partial, rows=rows, channels=channels, ensemble=ensemble)
    torch.testing.assert_close(db.cpu().double(), dy.double().sum(1), rtol=1e-5, atol=1e-4)
