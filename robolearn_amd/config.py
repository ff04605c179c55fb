"""Learner configuration dataclasses.

Field names, defaults and validation mirror the reference so that existing
configurations load unchanged:
  FlashSACConfig  robolearn/flashsac/config.py:11-85
  PPOConfig       robolearn/warp/config.py:8-34, validated as in
                  robolearn/warp/ppo.py:372-395
On MI355X ``use_amp`` selects bf16 dense-layer operands with fp32
accumulation, activations, master weights and Adam state (the reference's
AMP path uses fp16 operands with loss scaling, which bf16 does not need).
"""

from dataclasses import dataclass


@dataclass
class FlashSACConfig:
    device: str = "cuda:0"
    buffer_device: str | None = None
    seed: int = 0
    normalize_reward: bool = True
    normalized_G_max: float = 5.0
    asymmetric_observation: bool = False
    buffer_max_length: int = 1_000_000
    buffer_min_length: int = 100_000
    sample_batch_size: int = 2048
    learning_rate_init: float = 3e-4
    learning_rate_peak: float = 3e-4
    learning_rate_end: float = 1.5e-4
    learning_rate_warmup_rate: float = 1e-6
    learning_rate_warmup_step: int = 0
    learning_rate_decay_rate: float = 1.0
    learning_rate_decay_step: int = 10_000
    actor_num_blocks: int = 2
    actor_hidden_dim: int = 128
    actor_bc_alpha: float = 0.0
    actor_noise_zeta_mu: float = 2.0
    actor_noise_zeta_max: int = 16
    actor_update_period: int = 2
    critic_num_blocks: int = 2
    critic_hidden_dim: int = 256
    critic_num_bins: int = 101
    critic_min_v: float = -5.0
    critic_max_v: float = 5.0
    critic_target_update_tau: float = 0.01
    temp_initial_value: float = 0.01
    temp_target_sigma: float = 0.15
    temp_target_entropy: float | None = None
    gamma: float = 0.99
    n_step: int = 3
    use_compile: bool = False
    compile_mode: str = "auto"
    use_amp: bool = False
    load_optimizer: bool = True
    load_reward_normalizer: bool = True

    def __post_init__(self):
        # Same acceptance conditions as robolearn/flashsac/config.py:59-79, checked field by field
        # so the message names the offending field.
        for field_name in ("buffer_max_length", "buffer_min_length", "sample_batch_size", "n_step",
                           "actor_update_period", "learning_rate_decay_step"):
            if getattr(self, field_name) <= 0:
                raise ValueError(f"FlashSACConfig.{field_name} must be a positive integer, "
                                 f"got {getattr(self, field_name)}.")
        if self.buffer_max_length < self.buffer_min_length:
            raise ValueError(f"FlashSACConfig.buffer_min_length ({self.buffer_min_length}) is larger than the "
                             f"replay capacity buffer_max_length ({self.buffer_max_length}).")
        if self.gamma < 0 or self.gamma > 1:
            raise ValueError(f"FlashSACConfig.gamma={self.gamma} lies outside [0, 1].")
        if self.critic_num_bins < 2:
            raise ValueError(f"FlashSACConfig.critic_num_bins={self.critic_num_bins}: a categorical critic "
                             "needs two or more bins.")
        if not self.critic_min_v < self.critic_max_v:
            raise ValueError(f"FlashSACConfig value support [{self.critic_min_v}, {self.critic_max_v}] "
                             "is empty or reversed.")

    # Device accessors of the reference config (robolearn/flashsac/config.py:81-87).
    device_type = property(lambda self: self.device)
    buffer_device_type = property(lambda self: self.buffer_device if self.buffer_device else self.device)


@dataclass(frozen=True)
class PPOConfig:
    hidden_dims: tuple[int, ...] = (64, 64)
    learning_rate: float = 3e-4
    gamma: float = 0.99
    gae_lambda: float = 0.95
    clip_ratio: float = 0.2
    value_coefficient: float = 0.5
    entropy_coefficient: float = 0.0
    epochs: int = 4
    max_grad_norm: float = 1.0
    initial_std: float = 1.0
    normalize_advantages: bool = True
    clip_value: bool = True
    seed: int = 42
    optimized_linear_backward: bool = False
    activation: str = "tanh"
    std_type: str = "log"
    std_range: tuple[float, float] = (1.0e-6, 1.0e6)
    num_mini_batches: int = 1
    schedule: str = "fixed"
    desired_kl: float = 0.01
    value_loss_scale: float = 0.5
    advantage_sample_std: bool = False
    timeout_bootstrap: str = "next"
    separate_grad_clipping: bool = False
    dense_backend: str = "warp"
