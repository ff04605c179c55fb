"""Reference-named plan entry points driven through the C ABI exactly as the
reference's ctypes wrappers call them (robolearn/cuda/adam.py, zero.py,
flash.py): grouped zero, native Adam with dynamic loss scaling, projection,
EMA, and the 16-bit operand copies.  Checked against oracle/optim.py and
oracle/flashsac.py."""

import ctypes
import math
from collections import OrderedDict

import numpy as np
import pytest
import torch

from oracle import flashsac as O
from oracle import optim as OO
from robolearn_amd import _native as N

pytestmark = pytest.mark.gpu

STREAM = None  # the null stream; every call below synchronizes before reading back


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def test_grouped_zero_clears_exactly_the_spans(gpu):
    pool = torch.full((40000,), 7.0, device=gpu)
    # sorted, disjoint spans: 16-byte aligned, misaligned starts, lengths around the 4096 chunk
    spans = [(0, 1), (4, 4096), (4101, 4097), (8201, 3), (8300, 12000), (20303, 5)]
    plan = N.create("rl_zero_create", len(spans), N.pointer_array([pool[o:].data_ptr() for o, _ in spans]),
                    N.size_array([n for _, n in spans]))
    try:
        for _ in range(2):
            pool.fill_(7.0)
            N.call("rl_zero_step", plan, STREAM)
            torch.cuda.synchronize()
            expected = torch.full_like(pool, 7.0)
            for o, n in spans:
                expected[o:o + n] = 0.0
            assert torch.equal(pool, expected)
    finally:
        N.call("rl_zero_destroy", plan)
    with pytest.raises(RuntimeError, match="sorted"):
        N.create("rl_zero_create", 2, N.pointer_array([pool[100:].data_ptr(), pool.data_ptr()]), N.size_array([4, 4]))


def _adam_plan(gpu, sizes, seed, lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8):
    g = torch.Generator().manual_seed(seed)
    params = [torch.randn(n, generator=g) for n in sizes]
    dev = {
        "p": [p.to(gpu) for p in params],
        "g": [torch.zeros(n, device=gpu) for n in sizes],
        "m1": [torch.zeros(n, device=gpu) for n in sizes],
        "m2": [torch.zeros(n, device=gpu) for n in sizes],
        "timestep": torch.zeros(1, device=gpu),
        "lr": torch.tensor([lr], device=gpu),
    }
    plan = N.create("rl_adam_create", len(sizes), *(N.pointer_array([t.data_ptr() for t in dev[k]])
                                                  for k in ("p", "g", "m1", "m2")),
                    N.size_array(sizes), _ptr(dev["timestep"]), _ptr(dev["lr"]), beta1, beta2, eps)
    host = {"p": [p.numpy().copy() for p in params], "m1": [np.zeros(n, np.float32) for n in sizes],
            "m2": [np.zeros(n, np.float32) for n in sizes]}
    return plan, dev, host


def _check_adam(dev, host, rtol=2e-5):
    for key in ("p", "m1", "m2"):
        for d, h in zip(dev[key], host[key]):
            np.testing.assert_allclose(d.cpu().numpy(), h, rtol=rtol, atol=1e-7)


def test_native_adam_matches_oracle(gpu):
    sizes = [1, 1000, 5003]
    plan, dev, host = _adam_plan(gpu, sizes, seed=0)
    state = {"timestep": np.float32(0)}
    rng = np.random.default_rng(1)
    try:
        for _ in range(4):
            grads = [rng.standard_normal(n).astype(np.float32) for n in sizes]
            for d, g in zip(dev["g"], grads):
                d.copy_(torch.from_numpy(g))
            N.call("rl_adam_step", plan, STREAM)
            OO.native_adam_step(host["p"], grads, host["m1"], host["m2"], state, 1e-3, 0.9, 0.999, 1e-8)
        torch.cuda.synchronize()
        assert float(dev["timestep"][0]) == float(state["timestep"]) == 4.0
        _check_adam(dev, host)
    finally:
        N.call("rl_adam_destroy", plan)


def test_dynamic_loss_scaling_sequence_matches_oracle(gpu):
    """Unscale, overflow skip, backoff and growth over a scripted sequence of
    steps; the scaler state is compared after every step and the gradients
    after every unscale (bitwise: both sides compute g * (1 / scale))."""
    sizes = [3, 2048, 777]
    plan, dev, host = _adam_plan(gpu, sizes, seed=2)
    scaler = {
        "scale": torch.tensor([1024.0], device=gpu),
        "tracker": torch.zeros(1, dtype=torch.int32, device=gpu),
        "found": torch.zeros(1, dtype=torch.int32, device=gpu),
        "skipped_flag": torch.zeros(1, dtype=torch.int32, device=gpu),
        "attempted": torch.zeros(1, dtype=torch.int64, device=gpu),
        "skipped": torch.zeros(1, dtype=torch.int64, device=gpu),
    }
    growth, backoff, interval = 2.0, 0.5, 2
    N.call("rl_adam_set_scaler", plan, *(_ptr(scaler[k]) for k in ("scale", "tracker", "found", "skipped_flag",
                                                                     "attempted", "skipped")),
           growth, backoff, interval)
    state = {"loss_scale": np.float32(1024.0), "growth_tracker": 0, "step_skipped": 0, "attempted": 0, "skipped": 0,
             "timestep": np.float32(0), "found_inf": 0}
    rng = np.random.default_rng(5)
    poison = {2: (1, 100, np.inf), 4: (2, 0, np.nan), 5: (0, 2, -np.inf)}
    try:
        for step in range(9):
            grads = [(rng.standard_normal(n) * float(state["loss_scale"])).astype(np.float32) for n in sizes]
            if step in poison:
                t, i, v = poison[step]
                grads[t][i] = v
            for d, g in zip(dev["g"], grads):
                d.copy_(torch.from_numpy(g))
            N.call("rl_adam_unscale", plan, STREAM)
            state["found_inf"] = OO.unscale(grads, state["loss_scale"])
            torch.cuda.synchronize()
            assert int(scaler["found"][0]) == state["found_inf"] == int(step in poison), step
            for d, g in zip(dev["g"], grads):
                np.testing.assert_array_equal(d.cpu().numpy(), g)
            N.call("rl_adam_step", plan, STREAM)
            OO.scaled_adam_step(host["p"], grads, host["m1"], host["m2"], state, 1e-3, 0.9, 0.999, 1e-8,
                                growth, backoff, interval)
            torch.cuda.synchronize()
            assert float(scaler["scale"][0]) == float(state["loss_scale"]), step
            assert int(scaler["tracker"][0]) == state["growth_tracker"], step
            assert int(scaler["skipped_flag"][0]) == state["step_skipped"], step
            assert int(scaler["attempted"][0]) == state["attempted"] == step + 1
            assert int(scaler["skipped"][0]) == state["skipped"]
            assert float(dev["timestep"][0]) == float(state["timestep"]), step
            _check_adam(dev, host)
        assert state["skipped"] == 3 and float(state["loss_scale"]) != 1024.0
    finally:
        N.call("rl_adam_destroy", plan)


def test_scaler_validation(gpu):
    plan, dev, _ = _adam_plan(gpu, [8], seed=0)
    try:
        with pytest.raises(RuntimeError, match="dynamic loss scaling"):
            N.call("rl_adam_unscale", plan, STREAM)
        state = [torch.zeros(2, dtype=torch.int64, device=gpu) for _ in range(6)]
        with pytest.raises(RuntimeError, match="invalid"):
            N.call("rl_adam_set_scaler", plan, *(_ptr(s) for s in state), 1.0, 0.5, 10)
    finally:
        N.call("rl_adam_destroy", plan)


def test_projection_and_ema_plans_match_oracle(gpu):
    torch.manual_seed(0)
    rows, cols, channels = 5, 37, 24
    host = OrderedDict([("block.weight", torch.randn(rows, cols)), ("block.norm.weight", torch.randn(channels)),
                        ("block.norm.bias", torch.randn(channels)), ("post_norm.weight", torch.randn(channels) * 3)])
    dev = OrderedDict((k, v.to(gpu)) for k, v in host.items())
    # the reference's shadows are __half (flash_kernels.cuh:63-70, 128, 138): IEEE fp16
    shadows = OrderedDict((k, torch.zeros(v.shape, dtype=torch.float16, device=gpu)) for k, v in host.items())
    first, second, lengths, kinds, shadow = [], [], [], [], []
    for r in range(rows):  # one descriptor per unit row (flash_kernels.cuh:398-445)
        first.append(dev["block.weight"][r].data_ptr()); second.append(None); lengths.append(cols); kinds.append(0)
        shadow.append(shadows["block.weight"][r].data_ptr())
    first.append(dev["block.norm.weight"].data_ptr()); second.append(dev["block.norm.bias"].data_ptr())
    lengths.append(channels); kinds.append(1); shadow.append(shadows["block.norm.weight"].data_ptr())
    first.append(dev["post_norm.weight"].data_ptr()); second.append(None); lengths.append(channels); kinds.append(2)
    shadow.append(shadows["post_norm.weight"].data_ptr())
    plan = N.create("rl_flash_projection_create_with_shadows", len(first), N.pointer_array(first),
                    N.pointer_array(second), N.size_array(lengths), N.int_array(kinds), N.pointer_array(shadow))
    target = OrderedDict((k, torch.randn_like(v)) for k, v in host.items())
    target_dev = OrderedDict((k, v.to(gpu)) for k, v in target.items())
    tau = 0.125
    target_shadows = OrderedDict((k, torch.zeros(v.shape, dtype=torch.float16, device=gpu)) for k, v in host.items())
    ema = N.create("rl_flash_ema_create_with_shadows", len(dev), N.pointer_array([v.data_ptr() for v in dev.values()]),
                   N.pointer_array([v.data_ptr() for v in target_dev.values()]),
                   N.size_array([v.numel() for v in dev.values()]), tau,
                   N.pointer_array([v.data_ptr() for v in target_shadows.values()]))
    try:
        N.call("rl_flash_projection_step", plan, STREAM)
        N.call("rl_flash_ema_step", ema, STREAM)
        torch.cuda.synchronize()
        O.normalize_parameters(host)
        O.ema_update(target, host, tau)
        for k in host:
            torch.testing.assert_close(dev[k].cpu(), host[k], rtol=1e-5, atol=1e-6)
            torch.testing.assert_close(target_dev[k].cpu(), target[k], rtol=1e-5, atol=1e-6)
        for k in ("block.weight", "block.norm.weight", "post_norm.weight"):
            assert torch.equal(shadows[k], dev[k].to(torch.float16)), k
        for k in host:
            assert torch.equal(target_shadows[k], target_dev[k].to(torch.float16)), k
        norms = dev["block.weight"].norm(dim=1)
        torch.testing.assert_close(norms, torch.ones_like(norms), rtol=1e-5, atol=1e-5)
    finally:
        N.call("rl_flash_projection_destroy", plan)
        N.call("rl_flash_ema_destroy", ema)


# IEEE binary16 edge cases: ties to even, the largest finite half, the overflow threshold
# (65520 rounds to infinity), subnormals down to half the smallest one, signed zero, infinities
F16_EDGES = [1.0 + 2.0**-11, 1.0 + 3 * 2.0**-11, 65504.0, 65519.0, 65520.0, -65520.0, 1e6, 2.0**-14, 2.0**-24,
             2.0**-25, 3 * 2.0**-26, 2.0**-26, -0.0, float("inf"), float("-inf"), 6.1e-5, 1e-8, -3.0e-7]


@pytest.mark.parametrize("count,offset", [(1, 0), (3, 1), (1001, 0), (4096, 1), (70001, 3)])
def test_cast_f32_f16_writes_ieee_half(gpu, count, offset):
    """rl_cast_f32_f16 (kernels.cu:663-687, __float2half_rn): round-to-nearest-even IEEE fp16,
    bit for bit against torch's float32 -> float16 conversion, on the vector path (16-byte aligned
    source) and the element path, with the count % 4 tail."""
    source = torch.randn(count + offset, device=gpu) * 100
    edges = torch.tensor(F16_EDGES, device=gpu)
    source[offset:offset + min(count, len(edges))] = edges[:count]
    if count > len(edges):
        source[-1] = float("nan")
    out = torch.zeros(count + offset, dtype=torch.float16, device=gpu)
    N.call("rl_cast_f32_f16", _ptr(source[offset:]), _ptr(out[offset:]), count, STREAM)
    torch.cuda.synchronize()
    expected = source[offset:].to(torch.float16)
    got = out[offset:]
    nan = torch.isnan(expected)
    assert torch.equal(torch.isnan(got), nan)
    assert torch.equal(got[~nan].view(torch.int16), expected[~nan].view(torch.int16))
    if count >= 7:
        host = got[:7].cpu().double().tolist()
        assert host[:2] == [1.0, 1.0 + 2.0**-9]  # ties to the even neighbour
        assert host[2:5] == [65504.0, 65504.0, float("inf")] and host[5:7] == [float("-inf"), float("inf")]
    if count >= 13:
        host = got[7:13].cpu().double().tolist()
        # 2^-25 is the tie between 0 and the smallest subnormal: even is 0
        assert host == [2.0**-14, 2.0**-24, 0.0, 2.0**-24, 0.0, 0.0]
        assert got[12].view(torch.int16).item() == -32768  # -0.0 keeps its sign


@pytest.mark.parametrize("count", [1, 1001, 70001])
def test_cast_f32_bf16_rounds_to_nearest_even(gpu, count):
    source = torch.randn(count + 1, device=gpu) * 100
    source[1] = 1.0 + 2.0**-8  # a tie: round-to-nearest-even keeps 1.0
    out = torch.zeros(count + 1, dtype=torch.bfloat16, device=gpu)
    for offset in (0, 1):
        N.call("rl_cast_f32_bf16", _ptr(source[offset:]), _ptr(out[offset:]), count, STREAM)
        torch.cuda.synchronize()
        assert torch.equal(out[offset:offset + count], source[offset:offset + count].to(torch.bfloat16))
    assert float(out[1]) == 1.0


def test_batchnorm_16bit_side_outputs(gpu):
    torch.manual_seed(1)
    batch, channels, eps, momentum = 300, 40, 1e-5, 0.01
    x = torch.randn(batch, channels, device=gpu)
    w = torch.randn(channels, device=gpu)
    b = torch.randn(channels, device=gpu)
    chunks = math.ceil(batch / 256)

    def run(with_half):
        rm, rv = torch.zeros(channels, device=gpu), torch.ones(channels, device=gpu)
        mean, var = torch.zeros(channels, device=gpu), torch.zeros(channels, device=gpu)
        partial = torch.zeros(2 * chunks * channels, device=gpu)
        y = torch.zeros(batch, channels, device=gpu)
        half = torch.zeros(batch, channels, dtype=torch.float16, device=gpu)
        args = [_ptr(t) for t in (x, w, b, rm, rv, mean, var, partial, y)]
        if with_half:
            N.call("rl_flash_bn_forward_with_fp16", *args, _ptr(half), batch, channels, eps, momentum, 1, 1, STREAM)
        else:
            N.call("rl_flash_bn_forward", *args, batch, channels, eps, momentum, 1, 1, STREAM)
        dy = torch.randn(batch, channels, device=gpu, generator=torch.Generator(device=gpu).manual_seed(3))
        sums = torch.zeros(2 * channels, device=gpu)
        dx, dw, db = (torch.zeros(batch, channels, device=gpu), torch.zeros(channels, device=gpu),
                      torch.zeros(channels, device=gpu))
        half_dx = torch.zeros(batch, channels, dtype=torch.float16, device=gpu)
        back = [_ptr(t) for t in (x, dy, y, w, mean, var, partial, sums, dx, dw, db)]
        if with_half:
            N.call("rl_flash_bn_backward_with_fp16", *back, _ptr(half_dx), batch, channels, eps, 1, 1, STREAM)
        else:
            N.call("rl_flash_bn_backward", *back, batch, channels, eps, 1, 1, STREAM)
        torch.cuda.synchronize()
        return y, half, dx, half_dx, dw, db

    y0, _, dx0, _, dw0, db0 = run(False)
    y1, half, dx1, half_dx, dw1, db1 = run(True)
    assert torch.equal(y0, y1) and torch.equal(dx0, dx1) and torch.equal(dw0, dw1) and torch.equal(db0, db1)
    # flash_kernels.cuh:28: the 16-bit outputs are the exact IEEE fp16 rounding of the retained fp32 values
    assert torch.equal(half, y1.to(torch.float16))
    assert torch.equal(half_dx, dx1.to(torch.float16))
    # this library's bf16 form writes the bf16 (RNE) rounding of the same y, from the apply pass itself
    rm, rv = torch.zeros(channels, device=gpu), torch.ones(channels, device=gpu)
    mean, var = torch.zeros(channels, device=gpu), torch.zeros(channels, device=gpu)
    partial = torch.zeros(2 * chunks * channels, device=gpu)
    y2 = torch.zeros(batch, channels, device=gpu)
    y2_bf16 = torch.zeros(batch, channels, dtype=torch.bfloat16, device=gpu)
    N.call("rl_flash_bn_forward_with_bf16", *[_ptr(t) for t in (x, w, b, rm, rv, mean, var, partial, y2, y2_bf16)],
           batch, channels, eps, momentum, 1, 1, STREAM)
    torch.cuda.synchronize()
    assert torch.equal(y2, y1) and torch.equal(y2_bf16, y1.to(torch.bfloat16))
    with pytest.raises(RuntimeError, match="nonnull"):
        N.call("rl_flash_bn_forward_with_fp16", *[_ptr(t) for t in (x, w, b, x, x, x, x, x, x)], None, batch,
               channels, eps, momentum, 1, 1, STREAM)
    # rl_flash_bn_backward_controlled (flash_kernels.cuh:598-609): overwrite_dx 1 replaces dx, 0 adds to it
    dy = torch.randn(batch, channels, device=gpu, generator=torch.Generator(device=gpu).manual_seed(3))
    mean, var = torch.zeros(channels, device=gpu), torch.zeros(channels, device=gpu)
    partial = torch.zeros(2 * chunks * channels, device=gpu)
    y = torch.zeros(batch, channels, device=gpu)
    N.call("rl_flash_bn_forward", *[_ptr(t) for t in (x, w, b, torch.zeros(channels, device=gpu),
                                                      torch.ones(channels, device=gpu), mean, var, partial, y)],
           batch, channels, eps, momentum, 1, 1, STREAM)
    prefill = torch.randn(batch, channels, device=gpu)
    for overwrite in (1, 0):
        dx = prefill.clone()
        dw, db = torch.zeros(channels, device=gpu), torch.zeros(channels, device=gpu)
        half_dx = torch.zeros(batch, channels, dtype=torch.float16, device=gpu)
        sums = torch.zeros(2 * channels, device=gpu)
        N.call("rl_flash_bn_backward_controlled", *[_ptr(t) for t in (x, dy, y, w, mean, var, partial, sums, dx, dw,
                                                                      db, half_dx)],
               overwrite, batch, channels, eps, 1, 1, STREAM)
        torch.cuda.synchronize()
        expected = dx0 if overwrite else prefill + dx0
        assert torch.equal(dx, expected), overwrite
        assert torch.equal(half_dx, dx.to(torch.float16)), overwrite
        assert torch.equal(dw, dw0) and torch.equal(db, db0)
    with pytest.raises(RuntimeError, match="dx"):
        N.call("rl_flash_bn_backward_controlled", *[_ptr(t) for t in (x, dy, y, w, mean, var, partial, sums)], None,
               _ptr(dw), _ptr(db), None, 1, batch, channels, eps, 1, 1, STREAM)
