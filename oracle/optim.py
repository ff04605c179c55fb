"""CPU restatement of the reference's native optimizer plans (TEST INFRASTRUCTURE ONLY).

numpy float32 arithmetic, one function per reference kernel:
  native_adam_step    robolearn/cuda/kernels.cu:310-337 (adam_prepare + adam_update):
                      bias-corrected Adam over flat fp32 tensors, float timestep
  unscale             robolearn/cuda/kernels.cu:358-376 (adam_unscale)
  scaled_prepare      robolearn/cuda/kernels.cu:378-405 (adam_scaled_prepare)
  scaled_adam_step    robolearn/cuda/kernels.cu:878-904 (rl_adam_step with a scaler)

Parity pinning (tests/test_oracle.py):
  * native_adam_step against torch.optim.Adam (the same update written with the
    bias corrections on the other side of the division) and the first-step
    closed form lr * g / (|g| + eps);
  * scaled_prepare against torch._amp_update_scale_ (the same growth/backoff
    rule without the 2^-126 floor) and the floor itself;
  * unscale against torch._amp_foreach_non_finite_check_and_unscale_ where
    both definitions agree, and the reference-only cases (a finite gradient
    whose unscaled value overflows, a non-positive scale) by hand.
"""

import numpy as np

SCALE_FLOOR = np.float32(2.0**-126)


def native_adam_step(params, grads, m1, m2, state, lr, beta1, beta2, eps):
    """One plan step over lists of float32 arrays, updated in place.

    state["timestep"] is the float32 step counter (kernels.cu:310-315)."""
    f = np.float32
    t = f(state["timestep"]) + f(1.0)
    state["timestep"] = t
    c1 = f(1.0) / (f(1.0) - np.power(f(beta1), t, dtype=np.float32))
    c2 = f(1.0) / (f(1.0) - np.power(f(beta2), t, dtype=np.float32))
    b1, b2 = f(beta1), f(beta2)
    omb1, omb2 = f(1.0 - beta1), f(1.0 - beta2)
    for p, g, a, b in zip(params, grads, m1, m2):
        a[...] = b1 * a + omb1 * g
        b[...] = b2 * b + omb2 * (g * g)
        p[...] = p - f(lr) * ((a * c1) / (np.sqrt(b * c2) + f(eps)))


def unscale(grads, scale):
    """g *= 1/scale in place; returns found_inf (kernels.cu:358-376)."""
    f = np.float32
    scale = f(scale)
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        inverse = f(1.0) / scale
        found = False
        for g in grads:
            unscaled = (g * inverse).astype(np.float32)
            bad = ~np.isfinite(g) | ~np.isfinite(unscaled) | (not np.isfinite(scale)) | (not scale > 0)
            found = found or bool(bad.any())
            g[...] = unscaled
    return int(found)


def scaled_prepare(state, found_inf, growth_factor, backoff_factor, growth_interval):
    """Scale/skip bookkeeping of one attempted step (kernels.cu:378-405).

    state keys: loss_scale (float32), growth_tracker, step_skipped, attempted,
    skipped, timestep.  Returns True when the Adam update runs."""
    f = np.float32
    state["attempted"] += 1
    state["step_skipped"] = int(found_inf != 0)
    if state["step_skipped"]:
        state["skipped"] += 1
        state["growth_tracker"] = 0
        state["loss_scale"] = max(f(state["loss_scale"]) * f(backoff_factor), SCALE_FLOOR)
        return False
    growth = state["growth_tracker"] + 1
    if growth >= growth_interval:
        with np.errstate(over="ignore"):
            increased = f(state["loss_scale"]) * f(growth_factor)
        if np.isfinite(increased):
            state["loss_scale"] = increased
        state["growth_tracker"] = 0
    else:
        state["growth_tracker"] = growth
    return True


def scaled_adam_step(params, grads, m1, m2, state, lr, beta1, beta2, eps, growth_factor, backoff_factor,
                     growth_interval):
    """rl_adam_step on a plan with a scaler, after rl_adam_unscale set found_inf."""
    if scaled_prepare(state, state["found_inf"], growth_factor, backoff_factor, growth_interval):
        native_adam_step(params, grads, m1, m2, state, lr, beta1, beta2, eps)
