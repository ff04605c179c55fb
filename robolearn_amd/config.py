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
        if (
            min(
                self.buffer_max_length,
                self.buffer_min_length,
                self.sample_batch_size,
                self.n_step,
                self.actor_update_period,
                self.learning_rate_decay_step,
            )
            <= 0
        ):
            raise ValueError("Buffer sizes, batch size, horizons, and update periods must be positive.")
        if self.buffer_min_length > self.buffer_max_length:
            raise ValueError("Replay warmup cannot exceed buffer capacity.")
        if not 0 <= self.gamma <= 1:
            raise ValueError("gamma must be in [0, 1].")
        if self.critic_num_bins < 2 or self.critic_min_v >= self.critic_max_v:
            raise ValueError("The categorical critic needs at least two bins and an increasing support.")

    @property
    def device_type(self) -> str:
        return self.device

    @property
    def buffer_device_type(self) -> str:
        return self.buffer_device or self.device


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
