"""Shared comparison rules of the GPU parity tests (imported by the test modules; collects nothing).

Reference-relative tolerance.  Two rounding-decided effects move a correct fp32 update away from the
float64 one by far more than 1e-4 on some tensors:

* Adam's first step maps a gradient g to -lr g / (|g| + eps), so elements with |g| near eps move by an
  amount their rounding decides (up to 2 lr);
* ReLU masks: a FlashSAC update at the README shape has about 35 ReLU inputs within 1e-7 and 300
  within 1e-6 of zero (relative to their row's largest input), each passed or blocked by rounding,
  and one flipped element changes its row's gradient.

The reference's own fp32 path, run as the oracle in float32, shows both: on the same update with
its batch rows permuted (mathematically the same update; the BatchNorm statistics, and with them
every ReLU input, round differently) its gradient error against float64 falls either near 1e-5 or
near 3e-4 .. 2e-3 per tensor, depending on which near-zero inputs flip.  A GPU result is therefore
held to 1e-4 relative L2 against float64 or, where the float32 oracle errs more, to 3x the largest
error over an ensemble of float32 oracle runs (the original row order and seeded permutations).
"""

import torch


def rel(actual, reference):
    """(max-norm, L2) errors of actual against reference, relative to the reference's max and L2 norms."""
    actual = torch.as_tensor(actual).double().reshape(-1)
    reference = torch.as_tensor(reference).double().reshape(-1)
    diff = actual - reference
    return (diff.abs().max().item() / max(reference.abs().max().item(), 1e-30),
            diff.norm().item() / max(reference.norm().item(), 1e-30))


def compare(label, gpu_values, cpu_values, reference, report, check=True):
    """Per tensor: the GPU's relative L2 error against `reference` (float64) may exceed 1e-4 only where
    the float32 oracle's does, and then by at most 3x the largest error over `cpu_values` (one dict or a
    list of dicts: float32 oracle runs).  Appends (label, name, GPU max, fp32 max, GPU L2, fp32 L2)
    rows to `report`; returns the worst error / allowance ratio (asserted <= 1 when `check`)."""
    runs = cpu_values if isinstance(cpu_values, (list, tuple)) else [cpu_values]
    worst = 0.0
    for name, ref in reference.items():
        gpu_max, gpu_l2 = rel(gpu_values[name], ref)
        errors = [rel(run[name], ref) for run in runs]
        cpu_max, cpu_l2 = max(e[0] for e in errors), max(e[1] for e in errors)
        report.append((label, name, gpu_max, cpu_max, gpu_l2, cpu_l2))
        allowed = max(1e-4, 3.0 * cpu_l2)
        worst = max(worst, gpu_l2 / allowed)
        assert not check or gpu_l2 <= allowed, (label, name, gpu_l2, cpu_l2)
    return worst


def permuted(batch, actor_noise, next_noise, seed):
    """The same update's inputs with the batch rows permuted (seeded): batch fields and next-action
    noise by row, the actor noise's two halves (current and next observations) by the same row map."""
    import numpy as np

    rows = next_noise.shape[0]
    perm = torch.as_tensor(np.random.default_rng(seed).permutation(rows))
    batch = {k: torch.as_tensor(v)[perm] for k, v in batch.items()}
    actor_noise = torch.cat([actor_noise[:rows][perm], actor_noise[rows:][perm]])
    return batch, actor_noise, next_noise[perm]


def delta_stats(before, after, reference):
    """The reference's delta policy (examples/diagnose_warp_flashsac.py:114-129) per parameter tensor:
    (max error of the change, bound 5e-7 + 0.02 max|reference change|, elements beyond it, L2 error)."""
    stats = {}
    for key, expected in reference.items():
        if "running" in key:
            continue
        actual = torch.as_tensor(after[key]).double()
        delta_ref = expected.double() - before[key].double()
        err = (actual - before[key].double() - delta_ref).abs()
        bound = 5e-7 + 0.02 * delta_ref.abs().max().item()
        stats[key] = (err.max().item(), bound, int((err > bound).sum()), err.norm().item())
    return stats
