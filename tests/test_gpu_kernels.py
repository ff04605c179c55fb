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


# split-K reductions with every direct-mode epilogue: 4-aligned outputs take the
# float4 reduction, n = 70 the scalar one; 32 splits over a small output the grouped one
@pytest.mark.parametrize("mode", [K.FP32, K.FP32_SPLIT, K.BF16])
@pytest.mark.parametrize("rows,n,k,splits", [(512, 256, 512, 3), (200, 70, 512, 4), (64, 32, 4096, 32)])
def test_split_k_reduction_epilogues(gpu, mode, rows, n, k, splits):
    print(f"case split-K epilogues mode={mode} rows={rows} n={n} k={k} splits={splits}", flush=True)
    x = _rand(2, rows, k, seed=31)
    w = _rand(2, n, k, seed=32, scale=0.05)
    bias = _rand(2, n, seed=33)
    c = _rand(2, rows, n, seed=34)
    if mode == K.BF16:
        x, w = x.to(torch.bfloat16), w.to(torch.bfloat16)
    xd, wd, bd, cd = x.to(gpu), w.to(gpu), bias.to(gpu), c.to(gpu)
    workspace = torch.empty(splits * 2 * rows * n * 4, dtype=torch.uint8, device=gpu)
    product = torch.bmm(x.double(), w.double().transpose(1, 2).contiguous())
    tol = dict(rtol=1e-2, atol=1e-2) if mode == K.BF16 else dict(rtol=1e-5, atol=1e-5 * math.sqrt(k))
    for epilogue, fn in (("relu", torch.relu), ("elu", torch.nn.functional.elu)):
        y = torch.empty(2, rows, n, device=gpu)
        y_h = torch.empty(2, rows, n, dtype=torch.bfloat16, device=gpu)
        K.gemm(xd, wd, y, m=rows, n=n, k=k, batch=2, a_kcontig=True, b_kcontig=True, lda=k, ldb=k, ldd=n,
               stride_a=rows * k, stride_b=n * k, stride_d=rows * n, bias=bd, stride_bias=n, epilogue=epilogue,
               c=cd, beta=0.5, mode=mode, splits=splits, workspace=workspace, d_bf16=y_h)
        ref = fn(product + bias.double()[:, None, :]) + 0.5 * c.double()
        torch.testing.assert_close(y.cpu().double(), ref, **tol)
        assert torch.equal(y_h.cpu().view(torch.int16), y.cpu().to(torch.bfloat16).view(torch.int16))


def test_bf16_operand_tensors(gpu):
    rows, k, n = 96, 128, 64
    x = _rand(rows, k, seed=8).to(torch.bfloat16)
    w = _rand(n, k, seed=9).to(torch.bfloat16)
    y = torch.empty(rows, n, device=gpu)
    K.linear_forward(x.to(gpu), w.to(gpu), y, rows=rows, in_dim=k, out_dim=n, mode=K.BF16)
    ref = x.double() @ w.double().T
    torch.testing.assert_close(y.cpu().double(), ref, rtol=1e-5, atol=1e-4)


# fp16 mode (the reference's mixed-plan precision): float16 operands as stored, float32 operands
# rounded to fp16 on load; both layouts, an edge-tiled shape, split-K and the fused epilogue
@pytest.mark.parametrize("a_dtype,b_dtype", [(torch.float16, torch.float16), (torch.float32, torch.float16),
                                             (torch.float16, torch.float32), (torch.float32, torch.float32)])
@pytest.mark.parametrize("a_kcontig,b_kcontig", [(True, True), (True, False), (False, True), (False, False)])
@pytest.mark.parametrize("batch,m,n,k,splits", [(2, 300, 136, 200, 1), (1, 64, 96, 1024, 4)])
def test_fp16_gemm_matches_rounded_operands(gpu, a_dtype, b_dtype, a_kcontig, b_kcontig, batch, m, n, k, splits):
    print(f"case fp16 gemm {a_dtype}x{b_dtype} a_k={a_kcontig} b_k={b_kcontig} {batch}x{m}x{n}x{k} "
          f"splits={splits}", flush=True)
    g = torch.Generator().manual_seed(m + n + k + 2 * a_kcontig + b_kcontig)
    a = torch.randn(batch, m, k, generator=g) * 4
    b = torch.randn(batch, n, k, generator=g)
    bias = torch.randn(batch, n, generator=g)
    c = torch.randn(batch, m, n, generator=g)
    a_mem = (a if a_kcontig else a.transpose(1, 2)).contiguous().to(a_dtype)
    b_mem = (b if b_kcontig else b.transpose(1, 2)).contiguous().to(b_dtype)
    ref = torch.einsum("bmk,bnk->bmn", a.to(torch.float16).double(), b.to(torch.float16).double())
    scale = torch.einsum("bmk,bnk->bmn", a.to(torch.float16).double().abs(), b.to(torch.float16).double().abs())
    workspace = torch.empty(splits * batch * (m * n + m) * 4, dtype=torch.uint8, device=gpu) if splits > 1 else None
    d = torch.full((batch, m, n), float("nan"), device=gpu)
    K.gemm(a_mem.to(gpu), b_mem.to(gpu), d, m=m, n=n, k=k, batch=batch, a_kcontig=a_kcontig, b_kcontig=b_kcontig,
           lda=k if a_kcontig else m, ldb=k if b_kcontig else n, ldd=n, stride_a=m * k, stride_b=n * k,
           stride_d=m * n, mode=K.FP16, splits=splits, workspace=workspace, bias=bias.to(gpu), stride_bias=n,
           epilogue="relu", c=c.to(gpu), beta=0.5)
    expected = torch.relu(ref + bias.double()[:, None, :]) + 0.5 * c.double()
    # exact fp16 products, fp32 accumulation: a few fp32 ulps of the absolute-value product per term
    err = (d.cpu().double() - expected).abs()
    assert (err <= 2e-7 * scale * math.sqrt(k) + 1e-6).all(), err.max().item()
    with pytest.raises(ValueError, match="float16"):
        K.gemm(a_mem.to(torch.bfloat16).to(gpu), b_mem.to(gpu), d, m=m, n=n, k=k, batch=batch, a_kcontig=a_kcontig,
               b_kcontig=b_kcontig, lda=k if a_kcontig else m, ldb=k if b_kcontig else n, ldd=n, stride_a=m * k,
               stride_b=n * k, stride_d=m * n, mode=K.FP16)


# channels 64, 160 and 1024 take the float4 elementwise kernels (160: a partial
# column block), 5 and 130 the scalar ones
@pytest.mark.parametrize("ensemble,rows,channels,relu", [(1, 1000, 5, False), (2, 777, 130, True), (2, 300, 64, True),
                                                         (1, 257, 160, False), (2, 513, 1024, True)])
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
    # the ReLU mask recomputed from x and the bias (no stored output) gives the same adjoints
    dx2 = torch.empty_like(y)
    dx2_bf16 = torch.empty(y.shape, dtype=torch.bfloat16, device=gpu)
    K.bn_backward(g["x"], g["dy"], None, g["w"], mean, var, partial, sums, dx2, None, None, rows=rows,
                  channels=channels, ensemble=ensemble, relu=relu, b=g["b"], dx_bf16=dx2_bf16)
    torch.testing.assert_close(dx2.cpu(), dx.cpu(), rtol=0, atol=0)
    torch.testing.assert_close(dx2_bf16.cpu(), dx.cpu().to(torch.bfloat16), rtol=0, atol=0)
    # eval mode uses running statistics
    y2 = torch.empty_like(y)
    K.bn_forward(g["x"], g["w"], g["b"], g["rm"], g["rv"], None, None, None, y2, rows=rows, channels=channels,
                 ensemble=ensemble, training=False)
    rmv, rvv = g["rm"].cpu().double(), g["rv"].cpu().double()
    ref2 = (x.double() - rmv[:, None]) / torch.sqrt(rvv[:, None] + 1e-5) * w.double()[:, None] + b.double()[:, None]
    torch.testing.assert_close(y2.cpu().double(), ref2, rtol=1e-5, atol=1e-5)


# channel counts cover the register-cached float4 paths (96, 300, 1024), the
# scalar fallback (6, 37) and the narrow column-sum layouts (1, 3, 6, 37); the
# last two shapes have >= 256 row chunks and take the one-pass backward kernel
@pytest.mark.parametrize("ensemble,rows,channels", [(2, 333, 96), (1, 1000, 1024), (2, 257, 300), (1, 600, 37),
                                                    (2, 513, 6), (1, 700, 3), (1, 2049, 1), (1, 65536, 8),
                                                    (2, 32769, 12)])
def test_rmsnorm_and_bias_grad(gpu, ensemble, rows, channels):
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
    # accumulate into a nonzero dx to cover the accumulate flag as well
    dx_acc = torch.full_like(xd, 0.25)
    K.rms_backward(xd, dyd, wd, ms, partial, dx_acc, None, rows=rows, channels=channels, ensemble=ensemble,
                   accumulate_dx=True)
    torch.testing.assert_close(dx_acc.cpu().double(), xr.grad + 0.25, rtol=1e-4, atol=1e-5)
    dx = torch.empty_like(xd)
    dw = torch.empty(ensemble, channels, device=gpu)
    K.rms_backward(xd, dyd, wd, ms, partial, dx, dw, rows=rows, channels=channels, ensemble=ensemble)
    torch.testing.assert_close(dx.cpu().double(), xr.grad, rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(dw.cpu().double(), wr.grad, rtol=1e-4, atol=1e-4)
    db = torch.empty(ensemble, channels, device=gpu)
    K.bias_grad(dyd, db, partial, rows=rows, channels=channels, ensemble=ensemble)
    torch.testing.assert_close(db.cpu().double(), dy.double().sum(1), rtol=1e-5, atol=1e-4)


@pytest.mark.parametrize("bins", [21, 51, 80, 101, 112, 128, 160, 300])
def test_td_cross_entropy_matches_oracle_projection(gpu, bins):
    """Fused min-Q target, two-hot projection, CE and d-logits against the oracle's
    categorical_td_target (robolearn/flashsac/updates.py:19-80, 254-257).  Rows mix
    terminal transitions, clamped returns, zero and negative discounts (the latter
    take the scan path of the projection)."""
    from oracle import flashsac as O

    B, min_v, max_v = 300, -10.0, 10.0
    g = torch.Generator().manual_seed(bins)
    target_logits = torch.randn(2, B, bins, generator=g)
    online_logits = torch.randn(2, B, bins, generator=g)
    reward = torch.randn(B, generator=g) * 4.0
    reward[:10] = 40.0
    reward[10:20] = -40.0
    terminated = (torch.rand(B, generator=g) < 0.1).float()
    discount = torch.full((B,), 0.99)
    discount[20:30] = 0.0
    discount[30:40] = -0.5
    next_log_probs = torch.randn(B, generator=g)
    alpha = torch.tensor([0.2])
    support = torch.linspace(min_v, max_v, bins)
    d = {k: v.to(gpu).contiguous() for k, v in dict(tl=target_logits, ol=online_logits, r=reward, t=terminated,
                                                     disc=discount, nlp=next_log_probs, a=alpha, z=support).items()}
    dlogits = torch.empty(2, B, bins, device=gpu)
    loss_rows, entropy_rows = torch.empty(2, B, device=gpu), torch.empty(B, device=gpu)
    target_out, q_next = torch.empty(B, bins, device=gpu), torch.empty(2, B, device=gpu)
    scale = 1.0 / (2 * B)
    K.td_cross_entropy(d["tl"], None, B, d["ol"], None, B, d["z"], d["r"], d["t"], d["disc"], d["nlp"], d["a"],
                       min_v=min_v, max_v=max_v, batch=B, bins=bins, scale=scale, dlogits=dlogits,
                       loss_rows=loss_rows, entropy_rows=entropy_rows, target_out=target_out, q_next=q_next)
    torch.cuda.synchronize()
    lp_target = torch.log_softmax(target_logits, -1)
    q = (lp_target.exp() * support).sum(-1)
    selected = O.select_min_q_log_probs(q, lp_target)
    entropy = alpha * next_log_probs
    expected = O.categorical_td_target(selected, reward, terminated, entropy, discount, bins, min_v, max_v)
    torch.testing.assert_close(q_next.cpu(), q, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(target_out.cpu(), expected, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(target_out.cpu().sum(-1), torch.ones(B), rtol=0, atol=1e-5)
    lp_online = torch.log_softmax(online_logits, -1)
    torch.testing.assert_close(loss_rows.cpu(), -(expected[None] * lp_online).sum(-1), rtol=1e-5, atol=1e-5)
    grad = scale * (lp_online.exp() * expected.sum(-1, keepdim=True)[None] - expected[None])
    torch.testing.assert_close(dlogits.cpu(), grad, rtol=1e-4, atol=1e-7)
    torch.testing.assert_close(entropy_rows.cpu(), entropy, rtol=1e-6, atol=0)


# Shapes that take the 256x256-tile bf16 kernel (m, n multiples of 256, K ranges
# multiples of 128): workgroup counts below and at multiples of 8 (the XCD
# renumbering), more tiles than CUs (the persistent loop), partial M-tile groups,
# split-K, and every operand layout (both K-contiguous and both M/N-contiguous
# take the eight-wave DMA kernel, the mixed layouts the register-staged one).
# On a 256-CU part the K-contiguous products with fewer 256-wide tiles than CUs take 128-wide tiles
# (8192 x 512 over 2 members) or 64-wide ones (the smaller shapes).
BIG_SHAPES = [(2, 512, 256, 128, 1), (2, 2560, 512, 256, 1), (1, 3072, 256, 128, 1), (2, 1024, 512, 1024, 4),
              (2, 4096, 4096, 128, 1), (1, 512, 256, 8192, 2),  # a weight gradient's long K, split
              (2, 8192, 512, 256, 1)]


@pytest.mark.parametrize("a_kcontig", [True, False])
@pytest.mark.parametrize("b_kcontig", [True, False])
@pytest.mark.parametrize("batch,m,n,k,splits", BIG_SHAPES)
def test_big_tile_bf16_gemm_layouts(gpu, a_kcontig, b_kcontig, batch, m, n, k, splits):
    print(f"case big a_k={a_kcontig} b_k={b_kcontig} batch={batch} m={m} n={n} k={k} splits={splits}", flush=True)
    g = torch.Generator().manual_seed(m + n + k)
    a = torch.randn(batch, m, k, generator=g).to(torch.bfloat16)
    b = torch.randn(batch, n, k, generator=g).to(torch.bfloat16)
    bias = torch.randn(batch, n, generator=g)
    c = torch.randn(batch, m, n, generator=g)
    a_mem = a if a_kcontig else a.transpose(1, 2).contiguous()
    b_mem = b if b_kcontig else b.transpose(1, 2).contiguous()
    ad, bd = a_mem.to(gpu), b_mem.to(gpu)
    workspace = torch.empty(splits * batch * m * n * 4, dtype=torch.uint8, device=gpu) if splits > 1 else None
    ref = torch.einsum("bmk,bnk->bmn", a.double(), b.double())
    d = torch.empty(batch, m, n, device=gpu)
    d_bf16 = torch.empty(batch, m, n, dtype=torch.bfloat16, device=gpu)
    K.gemm(ad, bd, d, m=m, n=n, k=k, batch=batch, a_kcontig=a_kcontig, b_kcontig=b_kcontig,
           lda=k if a_kcontig else m, ldb=k if b_kcontig else n, ldd=n, stride_a=m * k, stride_b=n * k,
           stride_d=m * n, mode=K.BF16, splits=splits, workspace=workspace, d_bf16=d_bf16)
    torch.testing.assert_close(d.cpu().double(), ref, rtol=1e-5, atol=1e-5 * math.sqrt(k))
    torch.testing.assert_close(d_bf16.cpu(), d.cpu().to(torch.bfloat16), rtol=0, atol=0)
    # fused epilogue: relu(AB + bias) + C
    K.gemm(ad, bd, d, m=m, n=n, k=k, batch=batch, a_kcontig=a_kcontig, b_kcontig=b_kcontig,
           lda=k if a_kcontig else m, ldb=k if b_kcontig else n, ldd=n, stride_a=m * k, stride_b=n * k,
           stride_d=m * n, mode=K.BF16, splits=splits, workspace=workspace, bias=bias.to(gpu), stride_bias=n,
           epilogue="relu", c=c.to(gpu), beta=1.0)
    expected = torch.relu(ref + bias.double()[:, None, :]) + c.double()
    torch.testing.assert_close(d.cpu().double(), expected, rtol=1e-5, atol=1e-5 * math.sqrt(k))


@pytest.mark.parametrize("kcontig", [True, False])
@pytest.mark.parametrize("splits", [1, 2])
def test_wide_gemm_padded_leading_dimensions(gpu, kcontig, splits):
    """The eight-wave kernel's DMA windows at leading dimensions wider than the product: K-contiguous
    operands that are K-slices of wider rows, M/N-contiguous ones that are row slices of wider rows.
    A window offset or extent that assumed ld == K (or M) reads the wrong elements or zeros."""
    batch, m, n, k = 2, 512, 768, 256
    print(f"case padded-ld kcontig={kcontig} splits={splits}", flush=True)
    g = torch.Generator().manual_seed(41 + splits)
    a = torch.randn(batch, m, k, generator=g).to(torch.bfloat16)
    b = torch.randn(batch, n, k, generator=g).to(torch.bfloat16)
    if kcontig:
        lda, ldb = k + 64, k + 192
        a_mem = torch.randn(batch, m, lda, generator=g).to(torch.bfloat16)
        b_mem = torch.randn(batch, n, ldb, generator=g).to(torch.bfloat16)
        a_mem[:, :, :k], b_mem[:, :, :k] = a, b
    else:
        lda, ldb = m + 256, n + 512
        a_mem = torch.randn(batch, k, lda, generator=g).to(torch.bfloat16)
        b_mem = torch.randn(batch, k, ldb, generator=g).to(torch.bfloat16)
        a_mem[:, :, :m], b_mem[:, :, :n] = a.transpose(1, 2), b.transpose(1, 2)
    workspace = torch.empty(splits * batch * m * n * 4, dtype=torch.uint8, device=gpu) if splits > 1 else None
    d = torch.empty(batch, m, n, device=gpu)
    K.gemm(a_mem.to(gpu), b_mem.to(gpu), d, m=m, n=n, k=k, batch=batch, a_kcontig=kcontig, b_kcontig=kcontig,
           lda=lda, ldb=ldb, ldd=n, stride_a=a_mem[0].numel(), stride_b=b_mem[0].numel(), stride_d=m * n,
           mode=K.BF16, splits=splits, workspace=workspace)
    ref = torch.einsum("bmk,bnk->bmn", a.double(), b.double())
    torch.testing.assert_close(d.cpu().double(), ref, rtol=1e-5, atol=1e-5 * math.sqrt(k))


def _chunk_moments(d):
    """Per-256-row-chunk column (mean, M2) in float64: [batch][chunk][2][n]."""
    batch, m, n = d.shape
    out = []
    for e in range(batch):
        rows = []
        for r0 in range(0, m, 256):
            x = d[e, r0:r0 + 256].double()
            mean = x.mean(0)
            rows.append(torch.stack([mean, ((x - mean) ** 2).sum(0)]))
        out.append(torch.stack(rows))
    return torch.stack(out)


# (batch, m, n, k, splits, a_kcontig, b_kcontig): the first three run the
# epilogue path of the 256x256 kernel (DMA and register-staged), the rest the
# separate pass (split-K, a ragged M, fp32-sized shapes the big kernel rejects).
MOMENT_SHAPES = [(2, 512, 256, 256, 1, True, True), (2, 8192, 512, 256, 1, True, True),
                 (1, 1024, 512, 192, 1, True, False),
                 (2, 768, 256, 128, 1, False, False), (2, 1024, 512, 1024, 4, True, True),
                 (2, 300, 256, 64, 1, True, True), (1, 512, 96, 64, 1, True, True)]


@pytest.mark.parametrize("batch,m,n,k,splits,a_kcontig,b_kcontig", MOMENT_SHAPES)
def test_gemm_output_moments_match_chunk_moments(gpu, batch, m, n, k, splits, a_kcontig, b_kcontig):
    print(f"case moments batch={batch} m={m} n={n} k={k} splits={splits} a_k={a_kcontig} b_k={b_kcontig}", flush=True)
    g = torch.Generator().manual_seed(7 * m + n)
    a = (torch.randn(batch, m, k, generator=g) + 0.5).to(torch.bfloat16)
    b = torch.randn(batch, n, k, generator=g).to(torch.bfloat16)
    a_mem = a if a_kcontig else a.transpose(1, 2).contiguous()
    b_mem = b if b_kcontig else b.transpose(1, 2).contiguous()
    workspace = torch.empty(splits * batch * m * n * 4, dtype=torch.uint8, device=gpu) if splits > 1 else None
    d = torch.empty(batch, m, n, device=gpu)
    chunks = (m + 255) // 256
    moments = torch.full((batch, chunks, 2, n), float("nan"), device=gpu)
    K.gemm(a_mem.to(gpu), b_mem.to(gpu), d, m=m, n=n, k=k, batch=batch, a_kcontig=a_kcontig, b_kcontig=b_kcontig,
           lda=k if a_kcontig else m, ldb=k if b_kcontig else n, ldd=n, stride_a=m * k, stride_b=n * k,
           stride_d=m * n, mode=K.BF16, splits=splits, workspace=workspace, moments=moments)
    torch.cuda.synchronize()
    expected = _chunk_moments(d.cpu())
    got = moments.cpu().double()
    torch.testing.assert_close(got[:, :, 0], expected[:, :, 0], rtol=1e-5, atol=1e-4)
    torch.testing.assert_close(got[:, :, 1], expected[:, :, 1], rtol=1e-5, atol=1e-3)
    # the BatchNorm consuming them gives the statistics of its own moments pass
    w, bb = torch.rand(batch, n, device=gpu) + 0.5, torch.randn(batch, n, device=gpu)
    outs = []
    for ready in (True, False):
        mean, var = torch.zeros(batch, n, device=gpu), torch.zeros(batch, n, device=gpu)
        partial = moments.clone() if ready else torch.zeros_like(moments)
        y = torch.empty(batch, m, n, device=gpu)
        K.bn_forward(d, w, bb, torch.zeros(batch, n, device=gpu), torch.ones(batch, n, device=gpu), mean, var,
                     partial, y, rows=m, channels=n, ensemble=batch, relu=True, moments_ready=ready)
        outs.append((mean.cpu(), var.cpu(), y.cpu()))
    for x0, x1 in zip(*outs):
        torch.testing.assert_close(x0, x1, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("batch,m,n,k,splits", [(2, 1024, 256, 1024, 8), (1, 1000, 128, 512, 2), (2, 64, 36, 256, 4)])
def test_split_fp32_product_moments_match_chunk_moments(gpu, batch, m, n, k, splits):
    """fp32-accurate products split over K reduce their partials and take the BatchNorm chunk moments of
    the result in one pass: D against float64, the moments against the chunk moments of D."""
    print(f"case fp32 split moments batch={batch} m={m} n={n} k={k} splits={splits}", flush=True)
    g = torch.Generator().manual_seed(3 * m + k)
    a = torch.randn(batch, m, k, generator=g) + 0.25
    b = torch.randn(batch, n, k, generator=g)
    workspace = torch.empty(splits * batch * (m * n + m) * 4, dtype=torch.uint8, device=gpu)
    d = torch.empty(batch, m, n, device=gpu)
    chunks = (m + 255) // 256
    moments = torch.full((batch, chunks, 2, n), float("nan"), device=gpu)
    K.gemm(a.to(gpu), b.to(gpu), d, m=m, n=n, k=k, batch=batch, a_kcontig=True, b_kcontig=True, lda=k, ldb=k,
           ldd=n, stride_a=m * k, stride_b=n * k, stride_d=m * n, mode=K.FP32_SPLIT, splits=splits,
           workspace=workspace, moments=moments)
    torch.cuda.synchronize()
    ref = a.double() @ b.double().transpose(1, 2)
    torch.testing.assert_close(d.cpu().double(), ref, rtol=1e-5, atol=1e-4)
    expected = _chunk_moments(d.cpu())
    got = moments.cpu().double()
    torch.testing.assert_close(got[:, :, 0], expected[:, :, 0], rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(got[:, :, 1], expected[:, :, 1], rtol=1e-5, atol=1e-3)


@pytest.mark.parametrize("batch,m,n,k,splits,a_kcontig,b_kcontig", MOMENT_SHAPES)
def test_bf16_only_gemm_output(gpu, batch, m, n, k, splits, a_kcontig, b_kcontig):
    """A bfloat16 output is the bf16 copy of the fp32 product, bit for bit, and its moments
    are those of the rounded values."""
    print(f"case bf16-only batch={batch} m={m} n={n} k={k} splits={splits} a_k={a_kcontig} b_k={b_kcontig}",
          flush=True)
    g = torch.Generator().manual_seed(5 * m + n)
    a = (torch.randn(batch, m, k, generator=g) + 0.5).to(torch.bfloat16)
    b = torch.randn(batch, n, k, generator=g).to(torch.bfloat16)
    a_mem = (a if a_kcontig else a.transpose(1, 2).contiguous()).to(gpu)
    b_mem = (b if b_kcontig else b.transpose(1, 2).contiguous()).to(gpu)
    workspace = torch.empty(splits * batch * m * n * 4, dtype=torch.uint8, device=gpu) if splits > 1 else None
    chunks = (m + 255) // 256
    args = dict(m=m, n=n, k=k, batch=batch, a_kcontig=a_kcontig, b_kcontig=b_kcontig, lda=k if a_kcontig else m,
                ldb=k if b_kcontig else n, ldd=n, stride_a=m * k, stride_b=n * k, stride_d=m * n, mode=K.BF16,
                splits=splits, workspace=workspace)
    d = torch.empty(batch, m, n, device=gpu)
    copy = torch.empty(batch, m, n, dtype=torch.bfloat16, device=gpu)
    K.gemm(a_mem, b_mem, d, d_bf16=copy, **args)
    only = torch.full((batch, m, n), float("nan"), dtype=torch.bfloat16, device=gpu)
    moments = torch.full((batch, chunks, 2, n), float("nan"), device=gpu)
    K.gemm(a_mem, b_mem, only, moments=moments, **args)
    plain = torch.full((batch, m, n), float("nan"), dtype=torch.bfloat16, device=gpu)
    K.gemm(a_mem, b_mem, plain, **args)  # the bf16-only epilogue without moments
    torch.cuda.synchronize()
    assert torch.equal(only.cpu().view(torch.int16), copy.cpu().view(torch.int16))
    assert torch.equal(plain.cpu().view(torch.int16), copy.cpu().view(torch.int16))
    expected = _chunk_moments(only.cpu().float())
    got = moments.cpu().double()
    torch.testing.assert_close(got[:, :, 0], expected[:, :, 0], rtol=1e-5, atol=1e-4)
    torch.testing.assert_close(got[:, :, 1], expected[:, :, 1], rtol=1e-5, atol=1e-3)


def test_bf16_only_output_needs_bf16_mode(gpu):
    x = torch.randn(64, 32, device=gpu)
    w = torch.randn(16, 32, device=gpu)
    with pytest.raises(ValueError, match="bf16-mode"):
        K.linear_forward(x, w, torch.empty(64, 16, dtype=torch.bfloat16, device=gpu), rows=64, in_dim=32,
                         out_dim=16, mode=K.FP32)


@pytest.mark.parametrize("ensemble,rows,channels,relu", [(2, 777, 132, True), (1, 512, 1024, True),
                                                         (2, 300, 64, False)])
def test_batchnorm_bf16_inputs_match_fp32_path(gpu, ensemble, rows, channels, relu):
    """bf16 x and dy give the fp32 path's results on the same (widened) values, bit for bit,
    and the input gradient may overwrite a bf16 dy in place."""
    print(f"case bn bf16 inputs ensemble={ensemble} rows={rows} channels={channels} relu={relu}", flush=True)
    x_h = (_rand(ensemble, rows, channels, seed=20, scale=2.0) + 0.5).to(torch.bfloat16).to(gpu)
    dy_h = _rand(ensemble, rows, channels, seed=21).to(torch.bfloat16).to(gpu)
    x_f, dy_f = x_h.float(), dy_h.float()
    w = (_rand(ensemble, channels, seed=22).abs() + 0.5).to(gpu)
    b = _rand(ensemble, channels, seed=23).to(gpu)
    results = []
    for x, dy in ((x_f, dy_f), (x_h, dy_h.clone())):
        rm, rv = torch.zeros(ensemble, channels, device=gpu), torch.ones(ensemble, channels, device=gpu)
        mean, var = torch.empty(ensemble, channels, device=gpu), torch.empty(ensemble, channels, device=gpu)
        partial = torch.empty(ensemble * 2 * K.chunks(rows) * channels, device=gpu)
        y = torch.empty(ensemble, rows, channels, device=gpu)
        y_h = torch.empty(ensemble, rows, channels, dtype=torch.bfloat16, device=gpu)
        K.bn_forward(x, w, b, rm, rv, mean, var, partial, y, rows=rows, channels=channels, ensemble=ensemble,
                     relu=relu, y_bf16=y_h)
        sums = torch.empty(2 * ensemble * channels, device=gpu)
        dw, db = torch.empty_like(mean), torch.empty_like(mean)
        if dy.dtype == torch.bfloat16:
            dx, dx_h = None, dy  # in place over the bf16 gradient
        else:
            dx, dx_h = torch.empty_like(y), torch.empty_like(y_h)
        K.bn_backward(x, dy, None, w, mean, var, partial, sums, dx, dw, db, rows=rows, channels=channels,
                      ensemble=ensemble, relu=relu, b=b, dx_bf16=dx_h)
        results.append([t.cpu() for t in (y, y_h, mean, var, rm, rv, dw, db, dx_h)])
    names = ("y", "y_bf16", "mean", "var", "running_mean", "running_var", "dw", "db", "dx_bf16")
    for name, ref, got in zip(names, *results):
        assert torch.equal(ref.view(torch.int32) if ref.dtype == torch.float32 else ref.view(torch.int16),
                           got.view(torch.int32) if got.dtype == torch.float32 else got.view(torch.int16)), name


def test_batchnorm_bf16_input_needs_vector_layout(gpu):
    x = torch.zeros(1, 64, 6, dtype=torch.bfloat16, device=gpu)
    w, b = torch.ones(1, 6, device=gpu), torch.zeros(1, 6, device=gpu)
    with pytest.raises(RuntimeError, match="bf16 BatchNorm"):
        K.bn_forward(x, w, b, torch.zeros(1, 6, device=gpu), torch.ones(1, 6, device=gpu),
                     torch.empty(1, 6, device=gpu), torch.empty(1, 6, device=gpu),
                     torch.empty(2 * 6, device=gpu), torch.empty(1, 64, 6, device=gpu), rows=64, channels=6)


@pytest.mark.parametrize("batch,rows,cols", [(1, 64, 64), (2, 1024, 4096), (3, 100, 37), (1, 1, 130), (2, 100, 36),
                                             (1, 132, 260)])
def test_transpose16_is_exact(gpu, batch, rows, cols):
    print(f"case transpose16 batch={batch} rows={rows} cols={cols}", flush=True)
    g = torch.Generator().manual_seed(rows * cols)
    src = torch.randn(batch, rows, cols, generator=g).to(torch.bfloat16).to(gpu)
    dst = torch.zeros(batch, cols, rows, dtype=torch.bfloat16, device=gpu)
    K.transpose16(src, dst, batch=batch, rows=rows, cols=cols)
    torch.cuda.synchronize()
    assert torch.equal(dst.cpu(), src.cpu().transpose(1, 2))


def test_transpose16_many_is_exact(gpu):
    """Several bf16 transposes in one launch (a parameter store's transposed copies), edge tiles and
    batches included, against torch's transpose of each source."""
    print("case transpose16_many", flush=True)
    g = torch.Generator().manual_seed(5)
    shapes = [(2, 1024, 256), (1, 100, 36), (3, 64, 68), (2, 4, 1028)]
    srcs = [torch.randn(b, r, c, generator=g).to(torch.bfloat16).to(gpu) for b, r, c in shapes]
    dsts = [torch.full((b, c, r), float("nan"), dtype=torch.bfloat16, device=gpu) for b, r, c in shapes]
    K.transpose16_many([(s, d, b, r, c) for s, d, (b, r, c) in zip(srcs, dsts, shapes)])
    torch.cuda.synchronize()
    for s, d in zip(srcs, dsts):
        assert torch.equal(d.cpu().view(torch.int16), s.cpu().transpose(1, 2).contiguous().view(torch.int16))


def test_input_gradient_with_transposed_weight(gpu):
    print("case linear_backward_input wt", flush=True)
    g = torch.Generator().manual_seed(11)
    E, rows, in_dim, out_dim = 2, 512, 1024, 4096
    dy = torch.randn(E, rows, out_dim, generator=g).to(torch.bfloat16).to(gpu)
    w = torch.randn(E, out_dim, in_dim, generator=g).to(torch.bfloat16).to(gpu)
    wt = torch.empty(E, in_dim, out_dim, dtype=torch.bfloat16, device=gpu)
    K.transpose16(w, wt, batch=E, rows=out_dim, cols=in_dim)
    dx0 = torch.empty(E, rows, in_dim, device=gpu)
    dx1 = torch.empty(E, rows, in_dim, device=gpu)
    K.linear_backward_input(dy, w, dx0, rows=rows, in_dim=in_dim, out_dim=out_dim, ensemble=E, mode=K.BF16)
    K.linear_backward_input(dy, w, dx1, rows=rows, in_dim=in_dim, out_dim=out_dim, ensemble=E, mode=K.BF16, wt=wt)
    ref = torch.matmul(dy.cpu().double(), w.cpu().double())
    # fp32 accumulation over K = 4096 unit-scale products: tolerance as in the other bf16 GEMM tests
    tol = 1e-5 * math.sqrt(out_dim)
    torch.testing.assert_close(dx1.cpu().double(), ref, rtol=1e-5, atol=tol)
    torch.testing.assert_close(dx0.cpu(), dx1.cpu(), rtol=1e-5, atol=tol)


@pytest.mark.parametrize("m,n,k,splits", [(300, 130, 77, 1), (2048, 512, 256, 1), (96, 64, 4096, 16),
                                          (2048, 512, 1024, 4), (300, 130, 1024, 4)])
def test_fp32_elu_gradient_epilogue(gpu, m, n, k, splits):
    print(f"case elu_grad epilogue m={m} n={n} k={k} splits={splits}", flush=True)
    g = torch.Generator().manual_seed(m + n + k)
    a, b = torch.randn(m, k, generator=g), torch.randn(k, n, generator=g)
    y = torch.nn.functional.elu(torch.randn(m, n, generator=g))
    d = torch.empty(m, n, device=gpu)
    workspace = torch.empty(splits * m * n * 4, dtype=torch.uint8, device=gpu) if splits > 1 else None
    K.gemm(a.to(gpu), b.to(gpu), d, m=m, n=n, k=k, a_kcontig=True, b_kcontig=False, lda=k, ldb=n, ldd=n,
           c=y.to(gpu), epilogue="elu_grad", mode=K.FP32, splits=splits, workspace=workspace)
    expected = (a.double() @ b.double()) * torch.where(y > 0, torch.ones_like(y), y + 1).double()
    torch.testing.assert_close(d.cpu().double(), expected, rtol=1e-4, atol=1e-4 * math.sqrt(k))


@pytest.mark.parametrize("rows,in_dim,out_dim,use_ws", [(300, 70, 37, False), (24576, 123, 512, True),
                                                         (24576, 128, 1, True), (5000, 256, 128, True)])
def test_fp32_weight_gradient_with_fused_bias_gradient(gpu, rows, in_dim, out_dim, use_ws):
    print(f"case dW+db rows={rows} in={in_dim} out={out_dim} ws={use_ws}", flush=True)
    g = torch.Generator().manual_seed(rows + in_dim)
    dy, x = torch.randn(rows, out_dim, generator=g), torch.randn(rows, in_dim, generator=g)
    dw = torch.empty(out_dim, in_dim, device=gpu)
    db = torch.full((out_dim,), float("nan"), device=gpu)
    workspace = torch.empty(256 << 20, dtype=torch.uint8, device=gpu) if use_ws else None
    K.linear_backward_weight(dy.to(gpu), x.to(gpu), dw, rows=rows, in_dim=in_dim, out_dim=out_dim, mode=K.FP32,
                             workspace=workspace, bias_grad=db)
    torch.cuda.synchronize()
    torch.testing.assert_close(dw.cpu().double(), dy.double().t() @ x.double(), rtol=1e-4, atol=1e-4 * math.sqrt(rows))
    torch.testing.assert_close(db.cpu().double(), dy.double().sum(0), rtol=1e-4, atol=1e-4 * math.sqrt(rows))


# the last two run the forward products and the split weight gradients on eight-wave 128 x 128 tiles
# (ragged in every dimension in the last)
SPLIT_SHAPES = [(1, 5, 7, 3), (2, 130, 129, 40), (2, 257, 96, 160), (1, 300, 37, 123), (2, 2048, 512, 256),
                (2, 8192, 512, 123), (2, 6000, 300, 130)]


@pytest.mark.parametrize("batch,rows,out_dim,in_dim", SPLIT_SHAPES)
def test_fp32_split_products_are_fp32_accurate(gpu, batch, rows, out_dim, in_dim):
    """Mode 2 (products on the bf16 matrix cores from exact three-piece splits) against float64,
    with the same error budget as the fp32 matrix-core path (mode 0) on the same inputs: forward
    with bias + ELU, input gradient with the ELU-gradient epilogue, weight gradient with the
    bias-gradient row sums, direct and split over K."""
    print(f"case fp32 split batch={batch} rows={rows} out={out_dim} in={in_dim}", flush=True)
    x = _rand(batch, rows, in_dim, seed=21)
    w = _rand(batch, out_dim, in_dim, seed=22, scale=0.2)
    dy = _rand(batch, rows, out_dim, seed=23)
    bias = _rand(batch, out_dim, seed=24)
    xd, wd, dyd, bd = (t.to(gpu) for t in (x, w, dy, bias))
    ws = torch.empty(64 << 20, dtype=torch.uint8, device=gpu)
    x64, w64, dy64 = x.double(), w.double(), dy.double()
    ref_y = torch.nn.functional.elu(torch.einsum("bri,boi->bro", x64, w64) + bias.double()[:, None, :])
    ref_dx = torch.einsum("bro,boi->bri", dy64, w64)
    c = ref_y.float()  # ELU outputs of the layer below, for the ELU-gradient epilogue of a [rows, out] product
    c64 = c.double()
    elu_grad = torch.where(c64 > 0, torch.ones_like(c64), c64 + 1)
    ref_dw = torch.einsum("bro,bri->boi", dy64, x64)
    ref_db = dy64.sum(1)

    def run(mode):
        y = torch.empty(batch, rows, out_dim, device=gpu)
        K.linear_forward(xd, wd, y, rows=rows, in_dim=in_dim, out_dim=out_dim, ensemble=batch, bias=bd,
                         epilogue="elu", mode=mode)
        # [rows, out] input-gradient-shaped product dy' = x' w'^T with the ELU-gradient epilogue
        g = torch.empty(batch, rows, out_dim, device=gpu)
        K.gemm(xd, wd, g, m=rows, n=out_dim, k=in_dim, batch=batch, a_kcontig=True, b_kcontig=True, lda=in_dim,
               ldb=in_dim, ldd=out_dim, stride_a=rows * in_dim, stride_b=out_dim * in_dim, stride_d=rows * out_dim,
               c=c.to(gpu), epilogue="elu_grad", mode=mode)
        dx = torch.empty(batch, rows, in_dim, device=gpu)
        K.linear_backward_input(dyd, wd, dx, rows=rows, in_dim=in_dim, out_dim=out_dim, ensemble=batch, mode=mode)
        out = {"y": y, "g": g, "dx": dx}
        for label, workspace in (("direct", None), ("split", ws)):
            dw = torch.empty(batch, out_dim, in_dim, device=gpu)
            db = torch.empty(batch, out_dim, device=gpu)
            K.linear_backward_weight(dyd, xd, dw, rows=rows, in_dim=in_dim, out_dim=out_dim, ensemble=batch, mode=mode,
                                     workspace=workspace, bias_grad=db)
            out[f"dw_{label}"], out[f"db_{label}"] = dw, db
        torch.cuda.synchronize()
        return {k: v.cpu().double() for k, v in out.items()}

    native, split = run(K.FP32), run(K.FP32_SPLIT)
    refs = {"y": ref_y, "g": torch.einsum("bri,boi->bro", x64, w64) * elu_grad, "dx": ref_dx,
            "dw_direct": ref_dw, "db_direct": ref_db, "dw_split": ref_dw, "db_split": ref_db}
    # reduction length of each product: fp32 accumulation error grows as its square root
    length = {"y": in_dim, "g": in_dim, "dx": out_dim, "dw_direct": rows, "db_direct": rows, "dw_split": rows,
              "db_split": rows}
    for key, ref in refs.items():
        scale = ref.abs().max().item() + 1e-30
        err_native = (native[key] - ref).abs().max().item()
        err_split = (split[key] - ref).abs().max().item()
        assert err_split <= 4.0 * err_native + 2e-7 * scale, (key, err_split, err_native, scale)
        assert err_split <= 2e-6 * scale * max(1.0, math.sqrt(length[key] / 2048)), (key, err_split, scale)
