"""ctypes boundary to librl_mi355x.so.

Mirrors the reference loader (robolearn/cuda/_runtime.py:77-135): symbols are
declared once, every status-returning call is checked and a -1 status becomes
a RuntimeError carrying rl_last_error().  There is no fallback: a missing or
unloadable library raises immediately.
"""

import ctypes
import threading
from pathlib import Path

from .build import library_path

_LOCK = threading.RLock()
_LIBRARY = None

c_int = ctypes.c_int
c_uint = ctypes.c_uint
c_ll = ctypes.c_longlong
c_ull = ctypes.c_ulonglong
c_float = ctypes.c_float
c_double = ctypes.c_double
c_size = ctypes.c_size_t
c_void = ctypes.c_void_p
c_char_p = ctypes.c_char_p
P = ctypes.c_void_p  # every device pointer crosses the ABI as void*
PP = ctypes.POINTER(ctypes.c_void_p)

# name: (restype, argtypes)
SIGNATURES = {
    "rl_last_error": (c_char_p, []),
    # dense
    "rl_gemm": (c_int, [c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int, P, c_ll, c_ll, P, c_ll, c_ll,
                        P, P, c_ll, c_ll, P, c_ll, c_float, c_int, c_int, P, c_size, P, P, P, P]),
    "rl_gemm_workspace": (c_size, [c_int, c_int, c_int, c_int, c_int, c_int]),
    "rl_transpose16": (c_int, [P, P, c_int, c_int, c_int, P]),
    "rl_transpose16_many": (c_int, [c_int, PP, PP, P, P, P, P]),
    "rl_plan_create": (c_void, [c_int] * 10 + [c_size]),
    "rl_plan_create_mixed": (c_void, [c_int] * 11 + [c_size]),
    "rl_plan_workspace": (c_size, [P]),
    "rl_plan_autotune": (c_int, [P, c_float, P]),
    "rl_plan_tuning_metadata": (c_char_p, [P]),
    "rl_plan_run": (c_int, [P, P, P, P, P, P, P, c_size, c_float, P]),
    "rl_plan_destroy": (c_int, [P]),
    # optimizer
    "rl_fused_optimizer_create": (c_void, [c_size, P, P, P, PP, PP, PP, PP, PP, PP, PP, P, P, P, c_double, c_double,
                                           c_double, c_double, c_int, c_int, c_double, c_double, c_double, c_ll,
                                           c_ll]),
    "rl_fused_optimizer_step": (c_int, [P, c_int, c_int, c_int, P, P]),
    "rl_fused_optimizer_step_clipped": (c_int, [P, c_int, c_int, P, c_ll, P, P, c_float, P]),
    "rl_fused_optimizer_destroy": (c_int, [P]),
    "rl_adam_create": (c_void, [c_size, PP, PP, PP, PP, P, P, P, c_double, c_double, c_double]),
    "rl_adam_step": (c_int, [P, P]),
    "rl_adam_destroy": (c_int, [P]),
    "rl_adam_set_scaler": (c_int, [P] * 7 + [c_double, c_double, c_int]),
    "rl_adam_unscale": (c_int, [P, P]),
    "rl_zero_create": (c_void, [c_size, PP, P]),
    "rl_zero_step": (c_int, [P, P]),
    "rl_zero_destroy": (c_int, [P]),
    "rl_flash_projection_create": (c_void, [c_size, PP, PP, P, P]),
    "rl_flash_projection_create_with_shadows": (c_void, [c_size, PP, PP, P, P, PP]),
    "rl_flash_projection_step": (c_int, [P, P]),
    "rl_flash_projection_destroy": (c_int, [P]),
    "rl_flash_ema_create": (c_void, [c_size, PP, PP, P, c_float]),
    "rl_flash_ema_create_with_shadows": (c_void, [c_size, PP, PP, P, c_float, PP]),
    "rl_flash_ema_step": (c_int, [P, P]),
    "rl_flash_ema_destroy": (c_int, [P]),
    # normalization
    "rl_bn_forward_ex": (c_int, [c_int, P, c_int, c_ll, P, P, P, P, P, P, P, P, P, P, c_int, c_int, c_float,
                                 c_float, c_int, c_int, c_int, c_int, P]),
    "rl_bn_backward_ex": (c_int, [c_int, P, c_int, c_ll, P, c_int, P, P, P, P, P, P, P, P, P, P, P, c_int, c_int,
                                  c_float, c_int, c_int, c_int, c_int, P]),
    "rl_rms_forward_ex": (c_int, [c_int, P, P, P, P, P, c_int, c_int, c_ll, c_float, P]),
    "rl_rms_backward_ex": (c_int, [c_int, P, P, P, P, P, P, P, P, c_int, c_int, c_ll, c_float, c_int, c_int, P]),
    "rl_cast_f32_bf16": (c_int, [P, P, c_ll, P]),
    "rl_cast_f32_f16": (c_int, [P, P, c_size, P]),
    "rl_bias_grad_ex": (c_int, [c_int, P, P, P, c_int, c_int, c_int, P]),
    "rl_flash_bn_forward": (c_int, [P] * 9 + [c_int, c_int, c_float, c_float, c_int, c_int, P]),
    "rl_flash_bn_forward_with_bf16": (c_int, [P] * 10 + [c_int, c_int, c_float, c_float, c_int, c_int, P]),
    "rl_flash_bn_forward_with_fp16": (c_int, [P] * 10 + [c_int, c_int, c_float, c_float, c_int, c_int, P]),
    "rl_flash_bn_forward_static": (c_int, [P] * 8 + [c_int, c_int, c_float, c_float, c_int, c_int, P]),
    "rl_flash_bn_backward_with_fp16": (c_int, [P] * 12 + [c_int, c_int, c_float, c_int, c_int, P]),
    "rl_flash_bn_backward": (c_int, [P] * 11 + [c_int, c_int, c_float, c_int, c_int, P]),
    "rl_flash_bn_backward_controlled": (c_int, [P] * 12 + [c_int, c_int, c_int, c_float, c_int, c_int, P]),
    "rl_flash_rms_forward": (c_int, [P, P, P, P, c_int, c_int, c_float, P]),
    "rl_flash_rms_backward": (c_int, [P, P, P, P, P, P, P, c_int, c_int, c_float, P]),
    "rl_bias_grad": (c_int, [P, P, c_int, c_int, P]),
    # categorical
    "rl_reduce": (c_int, [P, c_ll, c_float, c_int, P, P]),
    "rl_categorical_head_forward": (c_int, [P, P, c_ll, P, P, P, c_ll, c_int, c_int, P]),
    "rl_categorical_head_backward_q": (c_int, [P, P, c_ll, P, P, P, P, c_ll, c_int, c_int, P]),
    "rl_categorical_td_cross_entropy": (c_int, [P, P, c_ll, P, P, c_ll, P, P, P, P, P, P, c_float, c_float, c_ll, c_int,
                                                c_float, P, P, P, P, P, P, P]),
    "rl_flash_categorical_forward": (c_int, [P, P, P, P, P, c_int, c_int, P]),
    "rl_flash_categorical_backward": (c_int, [P, P, P, P, P, P, P, c_int, c_int, P]),
    "rl_flash_categorical_target": (c_int, [P] * 9 + [c_int, c_int, c_float, c_float, P]),
    # policy / replay
    "rl_philox_normal": (c_int, [c_ull, P, c_uint, P, c_ll, P]),
    "rl_replay_sample_indices": (c_int, [c_ull, P, c_uint, P, c_ll, P, c_ll, P]),
    "rl_replay_gather": (c_int, [P, c_ll, c_ll, c_int, c_int] + [P] * 15 + [P]),
    "rl_concat_columns": (c_int, [P, c_ll, c_ll, P, c_ll, c_int, P, c_ll, c_int, P]),
    "rl_tanh_gaussian_forward": (c_int, [P, P, P, c_ll, P, c_ll, c_int, c_int, P]),
    "rl_tanh_gaussian_backward": (c_int, [P, P, P, c_ll, c_ll, P, P, P, c_ll, c_int, P]),
    "rl_actor_objective": (c_int, [P, P, P, P, c_ll, P, P, c_float, c_ll, c_ll, c_int, P, P, P, P, P, P, P]),
    "rl_temperature_objective": (c_int, [P, P, c_float, P, P, P]),
    "rl_exp_scalar": (c_int, [P, P, P]),
    "rl_fill": (c_int, [P, c_ll, c_float, P]),
    "rl_add": (c_int, [P, P, c_ll, P]),
    "rl_advance_counters": (c_int, [P, c_int, P]),
    "rl_scale_rewards": (c_int, [P, c_ll, P, P, c_float, c_float, P]),
    "rl_exploration_noise": (c_int, [c_ull, P, P, c_int, P, P, c_ll, P, P, P]),
    "rl_ppo_sample": (c_int, [P, c_ll, P, c_ll, P, c_int, c_float, c_float, P, c_ll, c_int, P, P, P, P, P, P]),
    "rl_ppo_store": (c_int, [c_int, c_ll, c_int, c_int] + [P] * 8 + [c_ll, P, c_ll, P] + [P] * 10 + [P]),
    "rl_replay_ingest": (c_int, [c_ll, c_int, c_int, c_int, c_ll, c_float] + [P] * 6 + [P] * 4 + [P] * 7
                         + [P, P]),
    "rl_reward_stats_update": (c_int, [c_ll, c_float, P, P, P, P, P, P, P]),
    # PPO
    "rl_gae": (c_int, [c_int, c_int, c_float, c_float, c_int, P, P, P, P, P, P, P, P]),
    "rl_normalize_advantages": (c_int, [P, c_ll, c_int, P, P]),
    "rl_permutation": (c_int, [c_ll, c_ull, P, P, P, P]),
    "rl_advance_int": (c_int, [P, P]),
    "rl_ppo_gather": (c_int, [P, c_ll, c_ll, c_int, c_int, c_int] + [P] * 16 + [P]),
    "rl_ppo_kl_adapt": (c_int, [P, c_ll, P, P, P, c_ll, c_int, c_int, c_float, c_float, c_float, c_int, P, P, P, P]),
    "rl_ppo_loss": (c_int, [P, c_ll, P, P, P, P, P, P, P, c_ll, c_int, c_int, c_float, c_float, c_float, c_float,
                            c_float, c_float, c_int, P, P, P, P, P, P]),
    "rl_ppo_minibatch_loss": (c_int, [P, c_ll, P, c_ll, P, P, P, P, P, P, P, P, c_ll, c_int, c_int, c_float,
                                      c_float, c_float, c_float, c_float, c_float, c_int, c_float, c_int, P, P, c_ll]
                              + [P] * 5 + [P]),
    "rl_sum_squares": (c_int, [P, c_ll, P, P, P]),
    "rl_clip_by_norm": (c_int, [P, c_ll, P, c_float, P]),
    "rl_clip_grad_norm": (c_int, [P, c_ll, P, P, c_float, P]),
    "rl_elu_backward": (c_int, [P, P, c_ll, P]),
}

# Entry points whose return value is a handle (null on failure) or size.
_HANDLE_RETURNS = {name for name, (res, _) in SIGNATURES.items() if res is c_void}


def load(path: Path | None = None):
    """Load and declare the library once; raises if it is missing."""
    global _LIBRARY
    with _LOCK:
        if _LIBRARY is not None:
            return _LIBRARY
        target = Path(path) if path is not None else library_path()
        if not target.exists():
            raise RuntimeError(
                f"{target} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`."
            )
        library = ctypes.CDLL(str(target))
        for name, (restype, argtypes) in SIGNATURES.items():
            function = getattr(library, name)
            function.restype = restype
            function.argtypes = argtypes
        _LIBRARY = library
        return library


def last_error() -> str:
    message = load().rl_last_error()
    return message.decode() if message else ""


def call(name: str, *args) -> int:
    """Call a status-returning entry point and raise on -1."""
    result = getattr(load(), name)(*args)
    if result != 0:
        raise RuntimeError(f"{name}: {last_error()}")
    return result


def create(name: str, *args) -> int:
    """Call a handle-returning entry point and raise on null."""
    handle = getattr(load(), name)(*args)
    if not handle:
        raise RuntimeError(f"{name}: {last_error()}")
    return handle


def pointer_array(values) -> ctypes.Array:
    array = (ctypes.c_void_p * len(values))()
    for i, value in enumerate(values):
        array[i] = value
    return array


def int_array(values) -> ctypes.Array:
    return (ctypes.c_int * len(values))(*values)


def ll_array(values) -> ctypes.Array:
    return (ctypes.c_longlong * len(values))(*values)


def size_array(values) -> ctypes.Array:
    return (ctypes.c_size_t * len(values))(*values)


def exported_symbols() -> list[str]:
    return sorted(SIGNATURES)
