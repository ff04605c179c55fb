"""Thin tensor-level wrappers over the C ABI.

Every wrapper takes torch tensors that already live on the GPU, validates the
shapes the kernel assumes, and enqueues on torch's current stream.  Nothing
here computes on the host; a missing library raises from ``_native.load``.
"""

import torch

from . import _native

FP32 = 0
BF16 = 1
# fp32 operands and results with the products formed on the bf16 matrix cores from exact
# three-piece bf16 splits of every operand value (fp32-accurate)
FP32_SPLIT = 2
# IEEE fp16 operands on the fp16 matrix cores (float16 tensors as stored, float32 ones rounded to fp16 on
# load), fp32 accumulation and output: the precision of the reference's mixed dense plans
FP16 = 3
EPILOGUES = {None: 0, "relu": 1, "elu": 2, "elu_grad": 3}


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def ptr(tensor: torch.Tensor | None) -> int | None:
    return None if tensor is None else tensor.data_ptr()


def _check(tensor: torch.Tensor, numel: int, name: str, dtype=torch.float32):
    if not tensor.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor.")
    if tensor.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {tensor.dtype}.")
    if not tensor.is_contiguous():
        raise ValueError(f"{name} must be contiguous.")
    if tensor.numel() < numel:
        raise ValueError(f"{name} holds {tensor.numel()} elements, {numel} are needed.")


def _check_optional(tensor, numel: int, name: str, dtype=torch.float32):
    if tensor is not None:
        _check(tensor, numel, name, dtype)


def _is_bf16(tensor: torch.Tensor) -> int:
    return 1 if tensor.dtype == torch.bfloat16 else 0


def _operand_flag(tensor: torch.Tensor, mode: int) -> int:
    """1 for a 16-bit operand (bfloat16 in the bf16 mode, float16 in the fp16 mode), 0 for float32."""
    if tensor.dtype == torch.float32:
        return 0
    expected = torch.float16 if mode == FP16 else torch.bfloat16
    if tensor.dtype != expected:
        raise ValueError(f"GEMM mode {mode} takes float32 or {expected} operands, got {tensor.dtype}.")
    return 1


def gemm(
    a, b, d, *, m, n, k, batch=1, a_kcontig, b_kcontig, lda, ldb, ldd, stride_a=0, stride_b=0, stride_d=0,
    c=None, beta=0.0, bias=None, stride_bias=0, epilogue=None, mode=FP32, splits=1, workspace=None, d_bf16=None,
    moments=None, a_sums=None,
):
    """Row-major batched D = act(op(A) op(B) + bias) + beta * C (optional bf16 copy of D,
    per-256-row-chunk column moments of D for a following BatchNorm, and, fp32 mode, the
    row sums of op(A) over K).  A bfloat16 d (bf16 mode) receives D rounded to bf16 as the
    only output."""
    if d is not None and d.dtype == torch.bfloat16:
        if d_bf16 is not None or mode != BF16:
            raise ValueError("A bfloat16 output is the bf16-mode product's only output.")
        d, d_bf16 = None, d
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    _native.call(
        "rl_gemm", mode, _operand_flag(a, mode), _operand_flag(b, mode), int(a_kcontig), int(b_kcontig), m, n, k, batch, ptr(a), lda,
        stride_a, ptr(b), ldb, stride_b, ptr(c), ptr(d), ldd, stride_d, ptr(bias), stride_bias, float(beta),
        EPILOGUES[epilogue], splits, ptr(workspace), ws_bytes, ptr(d_bf16), ptr(moments), ptr(a_sums), stream(),
    )


def forward_split_count(m, n, k, batch, mode, kcontig=True):
    """K splits for a forward or input-gradient product whose output tiles cannot fill the GPU (a
    narrow head, or a narrow layer over a long K at a small batch).

    bf16 (heads, embedder input gradients, block input gradients): at least 256 workgroups.  Products
    the eight-wave kernel takes (both operands K-contiguous, m and n multiples of 256, K of 128) count
    its narrowest tiles, 256 x 64, which fill the GPU without partials or a reduction launch, and split
    only in multiples of 128 of K; the others count 256x128 tiles, each split >= 128 of K.  A bf16 block
    forward product is not split even where its tiles leave CUs idle (README shape): the split loses
    the BatchNorm moments of the epilogue and adds a reduction, which measured slower.
    fp32: 64x64 tiles, whose K loop is latency-bound when few workgroups share a CU; at least 1024
    workgroups, each split >= 256 of K: a split costs a reduction launch, which a shorter K loop
    repays only past that (Cartpole input gradient 1024 x 1024 over K = 256: 17.8 us unsplit, 25.2 us
    in two splits)."""
    splits = 1
    if mode == BF16:
        if kcontig and m % 256 == 0 and n % 256 == 0 and k % 128 == 0:
            tiles = (m // 256) * (n // 64) * batch
            while tiles * splits < 256 and (k // (2 * splits)) % 128 == 0 and splits < 16:
                splits *= 2
            return splits
        tiles = ((m + 255) // 256) * ((n + 127) // 128) * batch
        ktiles = (k + 31) // 32
        while tiles * splits < 256 and splits * 2 <= max(1, ktiles // 4) and splits < 16:
            splits *= 2
        return splits
    tiles = ((m + 63) // 64) * ((n + 63) // 64) * batch
    while tiles * splits < 1024 and k // (2 * splits) >= 256 and splits < 16:
        splits *= 2
    return splits


def _split_for(m, n, k, batch, mode, workspace, kcontig=True):
    """forward_split_count, limited to what the workspace holds (1 without one)."""
    if workspace is None:
        return 1
    splits = forward_split_count(m, n, k, batch, mode, kcontig)
    if splits > 1:
        need = _native.load().rl_gemm_workspace(mode, m, n, k, batch, splits)
        if need > workspace.numel() * workspace.element_size():
            splits = 1
    return splits


def linear_forward(x, w, y, *, rows, in_dim, out_dim, ensemble=1, x_stride=None, bias=None, epilogue=None,
                   mode=FP32, c=None, beta=0.0, d_bf16=None, moments=None, workspace=None, x_ld=None):
    """y[e] = act(x[e] w[e]^T + bias[e]) (+ beta c); x_stride 0 broadcasts x; moments receives
    y's per-256-row-chunk column moments (the BatchNorm partial layout).  With a workspace,
    a product too small to fill the GPU is split over K (fixed-order reduction).  x_ld: row
    pitch of x (default in_dim)."""
    x_ld = x_ld or in_dim
    if x_stride is None:
        x_stride = rows * x_ld
    _check(w, ensemble * out_dim * in_dim, "weight", w.dtype)
    _check(y, ensemble * rows * out_dim, "output", y.dtype)
    splits = _split_for(rows, out_dim, in_dim, ensemble, mode, workspace)
    gemm(x, w, y, m=rows, n=out_dim, k=in_dim, batch=ensemble, a_kcontig=True, b_kcontig=True, lda=x_ld,
         ldb=in_dim, ldd=out_dim, stride_a=x_stride, stride_b=out_dim * in_dim, stride_d=rows * out_dim, bias=bias,
         stride_bias=out_dim, epilogue=epilogue, mode=mode, c=c, beta=beta, d_bf16=d_bf16, moments=moments,
         splits=splits, workspace=workspace if splits > 1 else None)


def linear_backward_input(dy, w, dx, *, rows, in_dim, out_dim, ensemble=1, mode=FP32, c=None, beta=0.0,
                          d_bf16=None, wt=None, epilogue=None, workspace=None):
    """dx[e] = dy[e] w[e] (+ beta c).  wt: optional [ensemble, in_dim, out_dim] transposed copy of w,
    which lets both operands be read K-contiguously.  epilogue "elu_grad" (fp32) multiplies by
    elu'(c), c holding the ELU outputs of the layer below.  With a workspace, a product too small
    to fill the GPU is split over K (fixed-order reduction)."""
    _check(dx, ensemble * rows * in_dim, "input gradient", dx.dtype)
    splits = _split_for(rows, in_dim, out_dim, ensemble, mode, workspace, kcontig=wt is not None)
    ws = workspace if splits > 1 else None
    if wt is not None:
        _check(wt, ensemble * out_dim * in_dim, "transposed weight", wt.dtype)
        gemm(dy, wt, dx, m=rows, n=in_dim, k=out_dim, batch=ensemble, a_kcontig=True, b_kcontig=True, lda=out_dim,
             ldb=out_dim, ldd=in_dim, stride_a=rows * out_dim, stride_b=out_dim * in_dim, stride_d=rows * in_dim,
             mode=mode, c=c, beta=beta, d_bf16=d_bf16, splits=splits, workspace=ws)
        return
    gemm(dy, w, dx, m=rows, n=in_dim, k=out_dim, batch=ensemble, a_kcontig=True, b_kcontig=False, lda=out_dim,
         ldb=in_dim, ldd=in_dim, stride_a=rows * out_dim, stride_b=out_dim * in_dim, stride_d=rows * in_dim,
         mode=mode, c=c, beta=beta, d_bf16=d_bf16, epilogue=epilogue, splits=splits, workspace=ws)


def transpose16(src, dst, *, batch, rows, cols):
    """dst[b] = src[b]^T for 16-bit [batch, rows, cols] -> [batch, cols, rows]."""
    _check(src, batch * rows * cols, "transpose source", src.dtype)
    _check(dst, batch * rows * cols, "transpose destination", dst.dtype)
    _native.call("rl_transpose16", ptr(src), ptr(dst), batch, rows, cols, stream())


def transpose16_many(jobs):
    """Several transpose16 calls in one launch: jobs is a list of (src, dst, batch, rows, cols) with rows and
    cols multiples of 4 (at most 8 jobs)."""
    for src, dst, batch, rows, cols in jobs:
        _check(src, batch * rows * cols, "transpose source", src.dtype)
        _check(dst, batch * rows * cols, "transpose destination", dst.dtype)
    _native.call("rl_transpose16_many", len(jobs), _native.pointer_array([j[0].data_ptr() for j in jobs]),
                 _native.pointer_array([j[1].data_ptr() for j in jobs]), _native.int_array([j[2] for j in jobs]),
                 _native.int_array([j[3] for j in jobs]), _native.int_array([j[4] for j in jobs]), stream())


def split_count(m, n, k, batch, mode):
    """K splits for a weight-gradient product (small output, K = rows).

    bf16: at least two 256x128-tile workgroups per CU, each split >= 1024 of K; >= 128 of K
    when the output does not tile by 256 (a narrow head or embedder: those products run on
    the 256x128 kernel, whose workgroups are short enough that more of them pays: README head
    dW 101 x 512 over 2048 rows 30.7 us in 8 splits, 22.6 in 16; embedder dW 256 x 31 over 4096
    rows 24.0 us in 16, 17.5 in 32).  For the
    256x256-tile kernel a longer split beats more workgroups: its partials cost a write and a
    read of splits x M x N floats (README dW 2048 x 512 over 4096 rows: 44 us at 4 splits, 52 us
    at 8).
    fp32: the MFMA-issue-bound fp32 kernel runs 64x64 tiles for such products; at least 1024
    workgroups (four per CU), each split >= 256 of K, whose reduction then costs less than the
    shorter K loops save (Cartpole 256 x 1024 over 1024 rows: 23.6 us in 4 splits, 25.9 in 8); an
    output of at most 65,536 values (a head) takes splits down to 64 of K, since its reduction is
    nearly free.  Mode 2 outputs of more than 64 rows and columns whose splits reach 256 of the
    eight-wave 128x128-tile workgroups run there: at least 512 of them (two per CU), each split
    >= 384 of K (PPO c3 dW 256 x 512 over 24576 rows: 105.7 us in 16 splits, 98.0 in 32; 128 x 256:
    36.6 us in 64, 39.2 in 128)."""
    splits = 1
    if mode == BF16:
        tiles = ((m + 255) // 256) * ((n + 127) // 128) * batch
        ktiles = (k + 31) // 32
        min_ktiles = 32 if m % 256 == 0 and n % 256 == 0 else 4
        while tiles * splits < 512 and splits * 2 <= max(1, ktiles // min_ktiles) and splits < 64:
            splits *= 2
        return splits
    if mode == FP32_SPLIT and m > 64 and n > 64:
        wide = ((m + 127) // 128) * ((n + 127) // 128) * batch
        while wide * splits < 512 and splits * 2 <= k // 384 and splits < 256:
            splits *= 2
        if wide * splits >= 256:
            return splits
        splits = 1
    tiles = ((m + 63) // 64) * ((n + 63) // 64) * batch
    steps = (k + 15) // 16
    min_steps = 4 if m * n * batch <= 65536 else 16
    while tiles * splits < 1024 and splits * 2 <= max(1, steps // min_steps) and splits < 256:
        splits *= 2
    return splits


def linear_backward_weight(dy, x, dw, *, rows, in_dim, out_dim, ensemble=1, x_stride=None, mode=FP32,
                           workspace=None, beta=0.0, x_ld=None, bias_grad=None):
    """dw[e] = dy[e]^T x[e] (+ beta dw), split-K over rows when the tile grid is small.
    x_ld: row pitch of x (default in_dim).  bias_grad (fp32 mode): receives sum_rows dy[e]
    from the same product (overwritten)."""
    if bias_grad is not None:
        if mode == BF16:
            raise ValueError("The fused bias gradient needs the fp32 GEMM family.")
        _check(bias_grad, ensemble * out_dim, "bias gradient")
    x_ld = x_ld or in_dim
    if x_stride is None:
        x_stride = rows * x_ld
    _check(dw, ensemble * out_dim * in_dim, "weight gradient")
    splits = split_count(out_dim, in_dim, rows, ensemble, mode) if workspace is not None else 1
    if splits > 1:
        need = _native.load().rl_gemm_workspace(mode, out_dim, in_dim, rows, ensemble, splits)
        if need > workspace.numel() * workspace.element_size():
            splits = 1
    gemm(dy, x, dw, m=out_dim, n=in_dim, k=rows, batch=ensemble, a_kcontig=False, b_kcontig=False, lda=out_dim,
         ldb=x_ld, ldd=in_dim, stride_a=rows * out_dim, stride_b=x_stride, stride_d=out_dim * in_dim, mode=mode,
         splits=splits, workspace=workspace if splits > 1 else None, c=dw if beta else None, beta=beta,
         a_sums=bias_grad)


# ---------------------------------------------------------------------------
# Normalization
# ---------------------------------------------------------------------------
def bn_forward(x, w, b, running_mean, running_var, mean, var, partial, y, *, rows, channels, ensemble=1,
               x_stride=None, eps=1e-5, momentum=0.01, training=True, relu=False, update_running=True, y_bf16=None,
               residual=None, moments_ready=False):
    """y = act(BN(x)) [+ residual]; x_stride 0 broadcasts one input to every member; x may
    be float32 or bfloat16.

    moments_ready: partial already holds x's chunk moments (written by the producing GEMM)."""
    if x_stride is None:
        x_stride = rows * channels
    # the kernels write whole rows of the dtype each output pointer is declared with
    total = ensemble * rows * channels
    _check_optional(y, total, "BatchNorm output")
    _check_optional(y_bf16, total, "BatchNorm bf16 output", torch.bfloat16)
    _check_optional(residual, total, "BatchNorm residual")
    _native.call("rl_bn_forward_ex", ensemble, ptr(x), _is_bf16(x), x_stride, ptr(w), ptr(b), ptr(running_mean),
                 ptr(running_var), ptr(mean), ptr(var), ptr(partial), ptr(residual), ptr(y), ptr(y_bf16), rows,
                 channels, eps, momentum, int(training), int(relu), int(update_running), int(moments_ready), stream())


def bn_backward(x, dy, y, w, mean, var, partial, sums, dx, dw, db, *, rows, channels, ensemble=1, x_stride=None,
                eps=1e-5, training=True, relu=False, accumulate_dx=False, accumulate_params=False, dx_bf16=None,
                b=None):
    """BN backward; with relu and y=None the ReLU mask is recomputed from x and (w, b).  x and
    dy may be float32 or bfloat16; dx_bf16 may be dy itself (updated in place)."""
    if x_stride is None:
        x_stride = rows * channels
    total = ensemble * rows * channels
    _check_optional(dx, total, "BatchNorm input gradient")
    _check_optional(dx_bf16, total, "BatchNorm bf16 input gradient", torch.bfloat16)
    _check_optional(y, total, "BatchNorm forward output")
    _native.call("rl_bn_backward_ex", ensemble, ptr(x), _is_bf16(x), x_stride, ptr(dy), _is_bf16(dy), ptr(y), ptr(w),
                 ptr(b), ptr(mean), ptr(var), ptr(partial), ptr(sums), ptr(dx), ptr(dw), ptr(db), ptr(dx_bf16), rows,
                 channels, eps, int(training), int(relu), int(accumulate_dx), int(accumulate_params), stream())


def rms_forward(x, w, ms, y, *, rows, channels, ensemble=1, eps=1e-6, member_stride=0, y_bf16=None):
    """Row RMSNorm over `rows` rows per member; member_stride (elements) defaults to rows * channels."""
    _native.call("rl_rms_forward_ex", ensemble, ptr(x), ptr(w), ptr(ms), ptr(y), ptr(y_bf16), rows, channels,
                 member_stride, eps, stream())


def rms_backward(x, dy, w, ms, partial, dx, dw, *, rows, channels, ensemble=1, eps=1e-6, accumulate_dx=False,
                 accumulate_dw=False, member_stride=0, dx_bf16=None):
    _native.call("rl_rms_backward_ex", ensemble, ptr(x), ptr(dy), ptr(w), ptr(ms), ptr(partial), ptr(dx),
                 ptr(dx_bf16), ptr(dw), rows, channels, member_stride, eps, int(accumulate_dx), int(accumulate_dw),
                 stream())


def cast_bf16(source, destination):
    _native.call("rl_cast_f32_bf16", ptr(source), ptr(destination), source.numel(), stream())


def bias_grad(dy, db, partial, *, rows, channels, ensemble=1, accumulate=False):
    _native.call("rl_bias_grad_ex", ensemble, ptr(dy), ptr(db), ptr(partial), rows, channels, int(accumulate),
                 stream())


def chunks(rows: int) -> int:
    return (rows + 255) // 256


# ---------------------------------------------------------------------------
# Categorical head
# ---------------------------------------------------------------------------
def reduce_sum(x, out, *, scale=1.0):
    _native.call("rl_reduce", ptr(x), x.numel(), float(scale), 0, ptr(out), stream())


def reduce_max(x, out):
    _native.call("rl_reduce", ptr(x), x.numel(), 1.0, 1, ptr(out), stream())


def categorical_head_forward(logits, support, values, *, rows, bins, ensemble=1, bias=None, log_probs=None):
    _native.call("rl_categorical_head_forward", ptr(logits), ptr(bias), bins, ptr(support), ptr(log_probs),
                 ptr(values), rows, bins, ensemble, stream())


def categorical_head_backward_q(logits, support, dvalues, dlogits, *, rows, bins, ensemble=1, bias=None,
                                dlogits_bf16=None):
    _native.call("rl_categorical_head_backward_q", ptr(logits), ptr(bias), bins, ptr(support), ptr(dvalues),
                 ptr(dlogits), ptr(dlogits_bf16), rows, bins, ensemble, stream())


def td_cross_entropy(target_logits, target_bias, target_rows, online_logits, online_bias, online_rows, support,
                     reward, terminated, discount, next_log_probs, alpha, *, min_v, max_v, batch, bins, scale,
                     dlogits, loss_rows, entropy_rows, target_out=None, q_next=None, dlogits_bf16=None):
    _native.call("rl_categorical_td_cross_entropy", ptr(target_logits), ptr(target_bias), target_rows,
                 ptr(online_logits), ptr(online_bias), online_rows, ptr(support), ptr(reward), ptr(terminated),
                 ptr(discount), ptr(next_log_probs), ptr(alpha), float(min_v), float(max_v), batch, bins,
                 float(scale), ptr(target_out), ptr(dlogits), ptr(dlogits_bf16), ptr(loss_rows), ptr(entropy_rows),
                 ptr(q_next), stream())


# ---------------------------------------------------------------------------
# Policy / replay
# ---------------------------------------------------------------------------
def philox_normal(out, *, seed, counter=None, stream_id=0):
    _native.call("rl_philox_normal", int(seed), ptr(counter), int(stream_id), ptr(out), out.numel(), stream())


def sample_indices(idx, *, seed, count=None, fixed_count=0, counter=None, stream_id=0):
    _native.call("rl_replay_sample_indices", int(seed), ptr(counter), int(stream_id), ptr(count), int(fixed_count),
                 ptr(idx), idx.numel(), stream())


def concat_columns(out, ld_out, rows, a, lda, ca, b=None, ldb=0, cb=0):
    _native.call("rl_concat_columns", ptr(out), ld_out, rows, ptr(a), lda, ca, ptr(b), ldb, cb, stream())


def tanh_gaussian_forward(head, noise, actions, log_probs, *, rows, action_dim, ld_actions=None,
                          deterministic=False):
    _native.call("rl_tanh_gaussian_forward", ptr(head), ptr(noise), ptr(actions),
                 action_dim if ld_actions is None else ld_actions, ptr(log_probs), rows, action_dim,
                 int(deterministic), stream())


def tanh_gaussian_backward(head, noise, dactions, dlog_probs, dhead, *, rows, action_dim, grad_rows,
                           ld_dactions=None, dhead_bf16=None):
    _native.call("rl_tanh_gaussian_backward", ptr(head), ptr(noise), ptr(dactions),
                 action_dim if ld_dactions is None else ld_dactions, grad_rows, ptr(dlog_probs), ptr(dhead),
                 ptr(dhead_bf16), rows, action_dim, stream())


def fill(x, value):
    _native.call("rl_fill", ptr(x), x.numel(), float(value), stream())
