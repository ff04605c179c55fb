"""No-allocation BatchNorm forward against the workspace entry point.

rl_flash_bn_forward_static runs the same kernels as rl_flash_bn_forward with
the chunk moments in the library's static device array instead of the caller's
`partial` buffer, so its outputs (y, batch mean / variance, running statistics)
must equal the workspace entry point's bit for bit.  Two calls in a row, the
second on a smaller input, check that the array's leftover contents from the
first call do not leak into the second.  Sizes beyond the array are refused on
the host before any launch.
"""

import pytest
import torch

from robolearn_amd import _native

pytestmark = pytest.mark.gpu


def _case(rows, channels, seed, device):
    g = torch.Generator(device="cpu").manual_seed(seed)
    x = (torch.randn(rows, channels, generator=g) * 2.0 + 0.5).to(device)
    w = (torch.rand(channels, generator=g) + 0.5).to(device)
    b = (torch.randn(channels, generator=g) * 0.1).to(device)
    rm = (torch.randn(channels, generator=g) * 0.1).to(device)
    rv = (torch.rand(channels, generator=g) + 0.5).to(device)
    return x, w, b, rm, rv


def _run_reference(x, w, b, rm, rv, training, relu):
    rows, channels = x.shape
    chunks = (rows + 255) // 256
    partial = torch.empty(2 * chunks * channels, device=x.device)
    mean, var, y = torch.empty(channels, device=x.device), torch.empty(channels, device=x.device), torch.empty_like(x)
    rm, rv = rm.clone(), rv.clone()
    _native.call("rl_flash_bn_forward", x.data_ptr(), w.data_ptr(), b.data_ptr(), rm.data_ptr(), rv.data_ptr(),
                 mean.data_ptr(), var.data_ptr(), partial.data_ptr(), y.data_ptr(), rows, channels, 1e-5, 0.01,
                 int(training), int(relu), torch.cuda.current_stream().cuda_stream)
    return y, mean, var, rm, rv


def _run_static(x, w, b, rm, rv, training, relu):
    rows, channels = x.shape
    mean, var, y = torch.empty(channels, device=x.device), torch.empty(channels, device=x.device), torch.empty_like(x)
    rm, rv = rm.clone(), rv.clone()
    _native.call("rl_flash_bn_forward_static", x.data_ptr(), w.data_ptr(), b.data_ptr(), rm.data_ptr(), rv.data_ptr(),
                 mean.data_ptr(), var.data_ptr(), y.data_ptr(), rows, channels, 1e-5, 0.01, int(training), int(relu),
                 torch.cuda.current_stream().cuda_stream)
    return y, mean, var, rm, rv


def test_static_bn_forward_matches_workspace_entry_point(gpu):
    # two calls in a row, the second smaller; then an fp32 non-multiple-of-4 width (scalar kernels)
    for rows, channels, training, relu in ((4096, 1024, True, True), (300, 64, True, False), (777, 37, True, True),
                                           (513, 96, False, True)):
        print(f"case static bn forward rows={rows} channels={channels} training={training}", flush=True)
        inputs = _case(rows, channels, rows + channels, gpu)
        expected = _run_reference(*inputs, training, relu)
        actual = _run_static(*inputs, training, relu)
        torch.cuda.synchronize()
        for name, a, e in zip(("y", "mean", "var", "running_mean", "running_var"), actual, expected):
            if not training and name in ("mean", "var"):
                continue  # eval mode reads the running statistics and leaves mean/var unwritten
            assert torch.equal(a, e), (rows, channels, name)


def test_static_bn_forward_refuses_sizes_beyond_the_scratch(gpu):
    # 2 * ceil(65536 / 256) * 8192 floats = 4 Mi floats > 2 Mi: rejected on the host, nothing launched
    with pytest.raises(RuntimeError, match="static scratch"):
        _native.call("rl_flash_bn_forward_static", None, None, None, None, None, None, None, None, 65536, 8192,
                     1e-5, 0.01, 1, 1, None)
