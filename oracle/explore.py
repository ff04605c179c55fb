"""CPU restatement of FlashSAC's exploration-noise repeats (TEST INFRASTRUCTURE ONLY).

PyTorch-CPU float32, following robolearn/flashsac/agent.py:
  zeta_cdf        :159-167 _build_truncated_zeta_cdf: pmf(n) ∝ n^-mu on 1..max_n, cumsum
  sample_length   :170-177 _sample_integer_from_cdf: argmax(u < cdf) + 1, with the
                  uniform u injected (an all-false mask gives 1)
  Exploration     :180-214 _sample_flashsac_actions at temperature 1: a new noise
                  and repeat length when count == 0 or count >= n, else the held
                  noise; actions tanh(mean + std * noise); count advances

Parity pinning (tests/test_oracle.py):
  * zeta_cdf against the float64 closed form H(k, mu) / H(max_n, mu) with the
    generalized harmonic numbers H, and the uniform case mu = 0;
  * sample_length against a brute-force count of CDF entries <= u, and the
    all-false case against torch.argmax itself (the routine the reference calls);
  * Exploration against the refresh schedule a scripted sequence of lengths
    fixes: fresh noise exactly at steps 0, L0, L0 + L1, ... and held between.
"""

import torch


def zeta_cdf(mu: float, max_n: int) -> torch.Tensor:
    ns = torch.arange(1, max_n + 1, dtype=torch.float32)
    pmf = ns ** (-mu)
    pmf = pmf / torch.sum(pmf)
    return torch.cumsum(pmf, dim=0)


def sample_length(u: float, cdf: torch.Tensor) -> int:
    idx = torch.argmax((torch.tensor(u, dtype=torch.float32) < cdf).to(torch.int32))
    return int(idx) + 1


class Exploration:
    """Repeat state of one agent: the held noise, its age `count` and its length `n`."""

    def __init__(self, noise_shape):
        self.noise = torch.zeros(noise_shape)
        self.count = 0
        self.n = 1

    def step(self, u: float, fresh_noise: torch.Tensor, cdf: torch.Tensor) -> bool:
        """Advance one act(training=True) call; returns whether the noise was refreshed."""
        reinit = self.count == 0 or self.count >= self.n
        new_n = sample_length(u, cdf)
        if reinit:
            self.noise = fresh_noise.clone()
            self.n = new_n
            self.count = 0
        self.count += 1
        return reinit

    def actions(self, mean: torch.Tensor, std: torch.Tensor) -> torch.Tensor:
        return torch.tanh(mean + std * self.noise * 1.0)
