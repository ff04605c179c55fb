"""The reference-named operator entry points on the GPU, against float64.

These are the symbols the reference's own ctypes layer binds
(robolearn/cuda/_runtime.py:77-113, flash.py:14-41, categorical.py:16-31), so
a reference caller pointed at this library runs exactly these:

* rl_plan_create / rl_plan_create_mixed / rl_plan_run: column-major
  D = op(A) op(B) + beta C + bias[m] (robolearn/cuda/kernels.cu:528-538,
  698-731; cuBLASLt semantics), all four transpose combinations, beta 0 and 1,
  with and without bias, padded leading dimensions, split-K shapes; fp32
  operands (input_dtype 0), IEEE fp16 operands written by rl_cast_f32_f16
  (input_dtype 1, the CudaLinear path, robolearn/cuda/linear.py:82-138, 190),
  and this library's bf16 precisions: fp32 storage with bf16 compute
  (input_dtype 2) and bf16 operands written by rl_cast_f32_bf16 (input_dtype 3).
  The 16-bit reference is the float64 product of the operands rounded by
  torch to float16 (bfloat16), which also shows that each 16-bit producer and
  the mixed plan agree on the format;
* rl_flash_categorical_forward / _backward / _target
  (categorical_kernels.cuh:31-110, 126-176): log-softmax and expectation;
  the gradient from both dlog_probs and dvalues accumulated into draw and the
  bias gradient accumulated into dbias; the min-Q two-hot target with support
  min_v + j (max_v - min_v) / (bins - 1) and the running maximum of the entropy;
* rl_flash_rms_forward / _backward (flash_kernels.cuh:322-379, 611-634):
  var = mean(x^2), y = x / sqrt(var + eps) w; dx and dw accumulate;
* rl_bias_grad (kernels.cu:237-251, 742-758): db += column sums.
"""

import pytest
import torch

from robolearn_amd import _native
from robolearn_amd import kernels as K

pytestmark = pytest.mark.gpu


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _column_major(matrix, ld, device, dtype=torch.float32):
    """Column-major storage of a (rows, cols) float64 matrix with leading dimension ld >= rows."""
    rows, cols = matrix.shape
    storage = torch.full((cols, ld), float("nan"), dtype=torch.float32)
    storage[:, :rows] = matrix.t().to(torch.float32)
    return storage.to(device).contiguous()


def _round16(x, dtype):
    return x.to(torch.float32).to(dtype).to(torch.float64)


@pytest.mark.parametrize("input_dtype", [0, 1, 2, 3])
@pytest.mark.parametrize("transa,transb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("m,n,k", [(96, 80, 72), (300, 257, 1100)])
def test_plan_run_matches_float64(gpu, input_dtype, transa, transb, m, n, k):
    print(f"case plan input_dtype={input_dtype} trans=({transa},{transb}) m={m} n={n} k={k}", flush=True)
    g = torch.Generator().manual_seed(m * 7 + n + 3 * transa + transb + 11 * input_dtype)
    opa = torch.randn(m, k, generator=g, dtype=torch.float64)
    opb = torch.randn(k, n, generator=g, dtype=torch.float64)
    a_stored = opa if transa == 0 else opa.t()  # column-major A: m x k, or k x m when transposed
    b_stored = opb if transb == 0 else opb.t()
    lda, ldb, ldd = a_stored.shape[0] + 3, b_stored.shape[0] + 5, m + 2
    a_dev = _column_major(a_stored, lda, gpu)
    b_dev = _column_major(b_stored, ldb, gpu)
    half = {1: torch.float16, 2: torch.bfloat16, 3: torch.bfloat16}.get(input_dtype)
    if input_dtype in (1, 3):  # 16-bit operands written by the cast entry point of that format
        cast = "rl_cast_f32_f16" if input_dtype == 1 else "rl_cast_f32_bf16"
        a16 = torch.empty(a_dev.numel(), dtype=half, device=gpu)
        b16 = torch.empty(b_dev.numel(), dtype=half, device=gpu)
        for src, dst in ((a_dev, a16), (b_dev, b16)):
            _native.call(cast, src.data_ptr(), dst.data_ptr(), src.numel(), _stream())
        a_arg, b_arg = a16, b16
    else:
        a_arg, b_arg = a_dev, b_dev
    c = torch.randn(n, ldd, generator=g, dtype=torch.float64)  # column-major m x n with ld ldd
    bias = torch.randn(m, generator=g, dtype=torch.float64)
    c_dev, bias_dev = c.to(torch.float32).to(gpu), bias.to(torch.float32).to(gpu)
    library = _native.load()

    def make(use_bias):
        args = (m, n, k, transa, transb, lda, ldb, ldd, int(use_bias), 0)
        if input_dtype == 0:
            return _native.create("rl_plan_create", *args, 64 << 20)
        return _native.create("rl_plan_create_mixed", *args, input_dtype, 64 << 20)

    plans = {True: make(True), False: make(False)}
    try:
        exact_a, exact_b = (opa, opb) if input_dtype == 0 else (_round16(opa, half), _round16(opb, half))
        product = exact_a @ exact_b  # m x n
        scale = (exact_a.abs() @ exact_b.abs()).max().item()
        tol = 2e-6 * scale * max(1.0, k / 256)
        for beta in (0.0, 1.0):
            for use_bias, plan in plans.items():
                ws_bytes = library.rl_plan_workspace(plan)
                workspace = torch.empty(max(ws_bytes, 4), dtype=torch.uint8, device=gpu)
                d_dev = torch.full((n, ldd), float("nan"), device=gpu)
                _native.call("rl_plan_run", plan, a_arg.data_ptr(), b_arg.data_ptr(),
                             c_dev.data_ptr() if beta else None, d_dev.data_ptr(),
                             bias_dev.data_ptr() if use_bias else None, workspace.data_ptr(), workspace.numel(),
                             beta, _stream())
                torch.cuda.synchronize()
                expected = product + beta * c[:, :m].t().to(torch.float32).double()
                if use_bias:
                    expected = expected + bias.to(torch.float32).double()[:, None]
                got = d_dev[:, :m].t().cpu().double()
                err = (got - expected).abs().max().item()
                assert err <= tol, (beta, use_bias, err, tol)
                # the rows of D past m (leading-dimension padding) stay untouched
                assert torch.isnan(d_dev[:, m:]).all()
    finally:
        for plan in plans.values():
            library.rl_plan_destroy(plan)


@pytest.mark.parametrize("batch,bins", [(1000, 101), (37, 11), (300, 512), (129, 513), (64, 1024), (33, 4096),
                                        (17, 5000)])
def test_flash_categorical_forward_backward(gpu, batch, bins):
    print(f"case categorical forward/backward batch={batch} bins={bins}", flush=True)
    g = torch.Generator().manual_seed(batch + bins)
    raw = torch.randn(batch, bins, generator=g, dtype=torch.float64) * 2
    bias = torch.randn(bins, generator=g, dtype=torch.float64) * 0.3
    support = torch.linspace(-10.0, 10.0, bins, dtype=torch.float64)
    d = lambda x: x.to(torch.float32).to(gpu).contiguous()  # noqa: E731
    raw_d, bias_d, support_d = d(raw), d(bias), d(support)
    lp, values = torch.empty(batch, bins, device=gpu), torch.empty(batch, device=gpu)
    _native.call("rl_flash_categorical_forward", raw_d.data_ptr(), bias_d.data_ptr(), support_d.data_ptr(),
                 lp.data_ptr(), values.data_ptr(), batch, bins, _stream())
    torch.cuda.synchronize()
    raw_r = raw.to(torch.float32).double().requires_grad_(True)
    bias_r = bias.to(torch.float32).double().requires_grad_(True)
    lp_ref = torch.log_softmax(raw_r + bias_r, -1)
    q_ref = (lp_ref.exp() * support.to(torch.float32).double()).sum(-1)
    torch.testing.assert_close(lp.cpu().double(), lp_ref.detach(), rtol=0, atol=2e-5)
    torch.testing.assert_close(values.cpu().double(), q_ref.detach(), rtol=1e-5, atol=2e-5)
    # backward from both outputs, accumulating into draw and dbias
    dlp = torch.randn(batch, bins, generator=g, dtype=torch.float64) * 0.1
    dq = torch.randn(batch, generator=g, dtype=torch.float64)
    draw0 = torch.randn(batch, bins, generator=g, dtype=torch.float64) * 0.01
    dbias0 = torch.randn(bins, generator=g, dtype=torch.float64) * 0.01
    draw, dbias = d(draw0), d(dbias0)
    dlp_d, dq_d = d(dlp), d(dq)  # held: a temporary's memory could be reused before the launch runs
    scratch = torch.empty(batch, bins, device=gpu)
    _native.call("rl_flash_categorical_backward", lp.data_ptr(), support_d.data_ptr(), dlp_d.data_ptr(),
                 dq_d.data_ptr(), scratch.data_ptr(), draw.data_ptr(), dbias.data_ptr(), batch, bins, _stream())
    torch.cuda.synchronize()
    (lp_ref * dlp.to(torch.float32).double()).sum().backward(retain_graph=True)
    (q_ref * dq.to(torch.float32).double()).sum().backward()
    torch.testing.assert_close(draw.cpu().double(), draw0.to(torch.float32).double() + raw_r.grad, rtol=0, atol=2e-5)
    torch.testing.assert_close(dbias.cpu().double(), dbias0.to(torch.float32).double() + bias_r.grad, rtol=1e-5,
                               atol=2e-4)
    torch.testing.assert_close(scratch.cpu().double(), raw_r.grad, rtol=0, atol=2e-5)


@pytest.mark.parametrize("batch,bins", [(500, 101), (64, 21), (200, 513), (64, 1024), (40, 4096)])
def test_flash_categorical_target(gpu, batch, bins):
    print(f"case categorical target batch={batch} bins={bins}", flush=True)
    from oracle import flashsac as O

    min_v, max_v = -10.0, 10.0
    g = torch.Generator().manual_seed(batch * 3 + bins)
    q = torch.randn(2, 2 * batch, generator=g)
    lp = torch.log_softmax(torch.randn(2, 2 * batch, bins, generator=g), -1)
    reward = torch.randn(batch, generator=g) * 4
    reward[:5] = 60.0
    terminated = (torch.rand(batch, generator=g) < 0.1).float()
    discount = torch.full((batch,), 0.97)
    discount[5:8] = -0.5  # decreasing bin indices: the rows take the full-scan projection
    next_log_probs = torch.randn(batch, generator=g)
    alpha = torch.tensor([0.3])
    start_max = torch.tensor([-1e30])
    inputs = [t.to(gpu).contiguous() for t in (q, lp, reward, terminated, discount, next_log_probs, alpha)]
    target, maximum = torch.empty(batch, bins, device=gpu), start_max.to(gpu)
    _native.call("rl_flash_categorical_target", *[t.data_ptr() for t in inputs], target.data_ptr(),
                 maximum.data_ptr(), batch, bins, min_v, max_v, _stream())
    torch.cuda.synchronize()
    # the reference kernel's support min_v + j * width (not linspace) and its min-Q rule on the
    # next-observation half (critic 1 only where its Q is strictly smaller)
    width = (max_v - min_v) / (bins - 1)
    z = min_v + torch.arange(bins, dtype=torch.float64) * width
    next_q = q[:, batch:].double()
    selected = (next_q[1] < next_q[0]).long()
    src = lp[:, batch:].double()[selected, torch.arange(batch)]
    entropy = alpha.double() * next_log_probs.double()
    v = reward.double()[:, None] + discount.double()[:, None] * (z[None] - entropy[:, None]) * (
        1 - terminated.double()[:, None])
    loc = (v.clamp(min_v, max_v) - min_v) / width
    lower = loc.floor().clamp(0, bins - 1).long()
    upper = (lower + 1).clamp(max=bins - 1)
    frac = loc - lower.double()
    prob = src.exp()
    expected = torch.zeros(batch, bins, dtype=torch.float64)
    expected.scatter_add_(1, lower, prob * (1 - frac))
    expected.scatter_add_(1, upper, prob * frac)
    # The kernel forms b = (v - min_v) / width in fp32, as the reference kernel does: b (up to K - 1) and the
    # return v carry a few ulps, so each source's split fraction may differ from float64 by db, and bin k's
    # mass by at most 2 db times the mass landing on bins k - 1 .. k + 1 (a clamped row moves up to db of
    # its whole mass: 2.4e-4 at 4096 bins).
    db = 2.0 ** -22 * ((bins - 1) + 10.0 / width)
    padded = torch.nn.functional.pad(expected, (1, 1))
    tol = 2 * db * (padded[:, :-2] + padded[:, 1:-1] + padded[:, 2:]) + 1e-6
    err = (target.cpu().double() - expected).abs()
    assert bool((err <= tol).all()), (err / tol).max().item()
    torch.testing.assert_close(target.cpu().double().sum(-1), torch.ones(batch, dtype=torch.float64), rtol=0,
                               atol=1e-5)
    assert maximum.item() == pytest.approx(entropy.max().item(), rel=1e-6)
    # the oracle's linspace-support projection agrees to the support's rounding
    oracle = O.categorical_td_target(src, reward.double(), terminated.double(), entropy, discount.double(), bins,
                                     min_v, max_v)
    torch.testing.assert_close(oracle, expected, rtol=0, atol=1e-4 if bins <= 512 else 1e-3)


@pytest.mark.parametrize("batch,channels", [(300, 256), (2049, 1024), (70, 37)])
def test_flash_rms_forward_backward(gpu, batch, channels):
    print(f"case rms reference entries batch={batch} channels={channels}", flush=True)
    g = torch.Generator().manual_seed(batch + channels)
    x = torch.randn(batch, channels, generator=g, dtype=torch.float64)
    w = torch.rand(channels, generator=g, dtype=torch.float64) + 0.5
    dy = torch.randn(batch, channels, generator=g, dtype=torch.float64)
    dx0 = torch.randn(batch, channels, generator=g, dtype=torch.float64) * 0.1
    dw0 = torch.randn(channels, generator=g, dtype=torch.float64) * 0.1
    d = lambda t: t.to(torch.float32).to(gpu).contiguous()  # noqa: E731
    xd, wd = d(x), d(w)
    var, y = torch.empty(batch, device=gpu), torch.empty(batch, channels, device=gpu)
    eps = 1e-6
    _native.call("rl_flash_rms_forward", xd.data_ptr(), wd.data_ptr(), var.data_ptr(), y.data_ptr(), batch, channels,
                 eps, _stream())
    dx, dw, dyd = d(dx0), d(dw0), d(dy)
    partial = torch.empty((batch + 255) // 256 * channels, device=gpu)
    _native.call("rl_flash_rms_backward", xd.data_ptr(), dyd.data_ptr(), wd.data_ptr(), var.data_ptr(),
                 partial.data_ptr(), dx.data_ptr(), dw.data_ptr(), batch, channels, eps, _stream())
    torch.cuda.synchronize()
    xr = x.to(torch.float32).double().requires_grad_(True)
    wr = w.to(torch.float32).double().requires_grad_(True)
    ms = (xr * xr).mean(-1)
    out = xr / torch.sqrt(ms + eps)[:, None] * wr
    torch.testing.assert_close(var.cpu().double(), ms.detach(), rtol=1e-5, atol=1e-7)
    torch.testing.assert_close(y.cpu().double(), out.detach(), rtol=1e-5, atol=1e-5)
    out.backward(dy.to(torch.float32).double())
    torch.testing.assert_close(dx.cpu().double(), dx0.to(torch.float32).double() + xr.grad, rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(dw.cpu().double(), dw0.to(torch.float32).double() + wr.grad, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("batch,channels", [(1000, 101), (16384, 8), (3, 700)])
def test_bias_grad_accumulates_column_sums(gpu, batch, channels):
    print(f"case bias grad batch={batch} channels={channels}", flush=True)
    g = torch.Generator().manual_seed(batch * 5 + channels)
    dy = torch.randn(batch, channels, generator=g, dtype=torch.float64)
    db0 = torch.randn(channels, generator=g, dtype=torch.float64)
    dyd = dy.to(torch.float32).to(gpu)
    db = db0.to(torch.float32).to(gpu)
    _native.call("rl_bias_grad", dyd.data_ptr(), db.data_ptr(), batch, channels, _stream())
    torch.cuda.synchronize()
    expected = db0.to(torch.float32).double() + dy.to(torch.float32).double().sum(0)
    torch.testing.assert_close(db.cpu().double(), expected, rtol=1e-5, atol=1e-6 * batch ** 0.5 * 4)
