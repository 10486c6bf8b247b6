"""Error statistics and bounds of the per-layer, teacher-forced parity test.

Shared by ``test_gpu_layer.py`` (GPU stages against the bf16 oracle) and
``test_layer_sensitivity.py`` (the same bounds applied on the CPU to a
correct stage summed in float64 and to stages with a planted rounding slip).
"""

import torch

# Bounds per stage: the largest fraction of elements that may differ from the
# bf16 oracle, and the largest 99.9th percentile of the error in ulps.
MAX_DIFF_FRAC = {"q": 0.02, "k": 0.02, "v": 0.02, "residual": 0.02, "normed": 1e-3}
MAX_P999_ULP = 2.0


def bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    """Spacing of bf16 values at |x| (8 significant bits); the smallest normal's at 0."""
    a = x.float().abs().clamp_min(2.0 ** -126)
    return torch.exp2(torch.floor(torch.log2(a)) - 7)


def stats(got: torch.Tensor, ref: torch.Tensor, mag: torch.Tensor):
    """Fraction of elements not bit-equal; 99.9th percentile and max of |got - ref| in ulps of mag."""
    u = ((got.float() - ref.float()).abs() / bf16_ulp(mag)).flatten()
    return (got != ref).float().mean().item(), torch.quantile(u[: 1 << 22], 0.999).item(), u.max().item()


def within(name: str, s) -> bool:
    """Whether stage ``name``'s statistics ``s`` (from ``stats``) meet the bounds."""
    return s[0] <= MAX_DIFF_FRAC[name] and s[1] <= MAX_P999_ULP
