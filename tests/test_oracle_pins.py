"""Known answers for two scalar rules that the oracle restates and the product computes.

* The PPO adaptive learning-rate rule, robolearn/warp/ppo.py:233-238: lr / 1.5 (floor 1e-5) when
  KL > 2 * desired_kl, lr * 1.5 (cap 1e-2) when 0 < KL < desired_kl / 2, both comparisons strict.
  The expected values below are worked out by hand from those six lines, so a restatement with a
  non-strict comparison, a swapped branch, a missing floor or cap, or a factor other than 1.5 fails.
* The temperature target entropy, robolearn/flashsac/agent.py:329, 0.5 A ln(2 pi e sigma^2): the
  differential entropy of an A-dimensional Normal with standard deviation sigma per dimension, which
  torch.distributions.Normal(0, sigma).entropy() computes independently.
"""

import math

import pytest
import torch

from oracle import flashsac as OF
from oracle import ppo as OP

DESIRED_KL = 0.01

# (learning rate, KL, expected learning rate) for desired_kl = 0.01
KNOWN = [
    (1e-3, 0.0, 1e-3),                      # KL = 0 is not > 0: unchanged
    (1e-3, -1e-9, 1e-3),                    # a rounding-level negative KL: unchanged
    (1e-3, 0.0025, 1.5e-3),                 # 0 < KL < 0.005: raised by 1.5
    (1e-3, 0.005, 1e-3),                    # KL == target / 2 (strict): unchanged
    (1e-3, 0.0049999, 1.5e-3),              # just below target / 2: raised
    (1e-3, 0.01, 1e-3),                     # on target: unchanged
    (1e-3, 0.02, 1e-3),                     # KL == 2 * target (strict): unchanged
    (1e-3, 0.0200001, 1e-3 / 1.5),          # just above 2 * target: lowered
    (1e-3, 0.03, 6.666666666666667e-4),     # lowered by 1.5
    (1.2e-5, 0.03, 1e-5),                   # 8e-6 floored at 1e-5
    (8e-3, 0.001, 1e-2),                    # 1.2e-2 capped at 1e-2
    (1e-2, 0.001, 1e-2),                    # already at the cap
    (1e-5, 0.5, 1e-5),                      # already at the floor
]


@pytest.mark.parametrize("lr, kl, expected", KNOWN)
def test_adaptive_learning_rate_known_answers(lr, kl, expected):
    assert OP.adapt_learning_rate(lr, kl, DESIRED_KL) == pytest.approx(expected, rel=1e-12, abs=0.0)


@pytest.mark.parametrize("action_dim", [1, 8, 37])
@pytest.mark.parametrize("sigma", [0.05, 0.15, 1.0])
def test_target_entropy_is_the_normal_entropy(action_dim, sigma):
    from robolearn_amd.flashsac import target_entropy

    normal = action_dim * torch.distributions.Normal(torch.tensor(0.0, dtype=torch.float64),
                                                     torch.tensor(sigma, dtype=torch.float64)).entropy().item()
    assert OF.target_entropy(action_dim, sigma) == pytest.approx(normal, rel=1e-12)
    assert target_entropy(action_dim, sigma) == pytest.approx(normal, rel=1e-12)


def test_target_entropy_reference_default():
    # agent.py:329 with the default temp_target_sigma 0.15 (config.py) at the G1 action size 37:
    # 0.5 * 37 * ln(2 pi e 0.0225) = 18.5 * (1.837877 + 1 - 3.794240) = -17.69271...
    expected = 0.5 * 37 * (math.log(2 * math.pi) + 1.0 + 2 * math.log(0.15))
    assert OF.target_entropy(37, 0.15) == pytest.approx(expected, rel=1e-12)
    assert expected == pytest.approx(-17.69271, abs=1e-5)
