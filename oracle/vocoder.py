"""CPU restatement of the HiFT vocoder's elementwise family (test
infrastructure only).

Follows the kernels of server/kernels.py: ``snake_value`` (:35-38), the
per-element ops of ``snake_kernel`` / ``snake_bias_kernel`` (:40-47),
``residual_bias_kernel`` (:48-51), ``mean3_kernel`` (:52-55),
``residual_bias_snake_kernel`` (:56-61) and ``branch_start_kernel``
(:62-67), on [B, C, T] float32 arrays with per-channel alpha / bias.

The adds are restated in float32 in the reference's order, so their results
are exact references.  Snake itself is evaluated in float64 on the float32
argument (the activation's value; sin is not correctly rounded on any GPU),
in the HiFT module's form ``v + (1 / (a + 1e-9)) * sin(v * a)^2``, which is
the reference kernel's ``v + sin(v a)^2 / (a + 1e-9)`` up to one rounding.
"""

from __future__ import annotations

from typing import Optional, Tuple

import numpy as np

EPS = 1e-9  # no_div_by_zero of the Snake module (server/kernels.py:37)


def _chan(v: np.ndarray) -> np.ndarray:
    """Per-channel vector [C] broadcast over [B, C, T]."""
    return np.asarray(v, dtype=np.float32)[None, :, None]


def snake64(v: np.ndarray, alpha: np.ndarray) -> np.ndarray:
    """Snake of float32 arguments evaluated in float64 (server/kernels.py:35-38)."""
    a = _chan(alpha).astype(np.float64)
    v = np.asarray(v, dtype=np.float32).astype(np.float64)
    return v + (1.0 / (a + EPS)) * np.sin(v * a) ** 2


def snake(x: np.ndarray, alpha: np.ndarray, bias: Optional[np.ndarray] = None) -> np.ndarray:
    """snake_kernel / snake_bias_kernel (server/kernels.py:40-47): the biased
    argument is formed in float32 first, as the kernel does."""
    v = np.asarray(x, dtype=np.float32)
    if bias is not None:
        v = (v + _chan(bias)).astype(np.float32)
    return snake64(v, alpha)


def residual_bias(x: np.ndarray, residual: np.ndarray, bias: np.ndarray) -> np.ndarray:
    """(x + residual) + bias in float32 (server/kernels.py:48-51)."""
    x = np.asarray(x, dtype=np.float32)
    r = np.asarray(residual, dtype=np.float32)
    return ((x + r).astype(np.float32) + _chan(bias)).astype(np.float32)


def mean3(a: np.ndarray, b: np.ndarray, c: np.ndarray) -> np.ndarray:
    """((a + b) + c) * float32(1/3) (server/kernels.py:52-55)."""
    a, b, c = (np.asarray(t, dtype=np.float32) for t in (a, b, c))
    return ((((a + b).astype(np.float32) + c).astype(np.float32)) * np.float32(1.0 / 3.0)).astype(np.float32)


def residual_bias_snake(x: np.ndarray, residual: np.ndarray, bias: np.ndarray,
                        alpha: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """raw = (x + residual) + bias, act = snake(raw) (server/kernels.py:56-61)."""
    raw = residual_bias(x, residual, bias)
    return raw, snake64(raw, alpha)


def branch_start(x: np.ndarray, source: np.ndarray, alpha0: np.ndarray, alpha1: np.ndarray,
                 alpha2: np.ndarray) -> Tuple[np.ndarray, np.ndarray, np.ndarray, np.ndarray]:
    """raw = x + source, out_j = snake(raw, alpha_j) (server/kernels.py:62-67)."""
    raw = (np.asarray(x, dtype=np.float32) + np.asarray(source, dtype=np.float32)).astype(np.float32)
    return raw, snake64(raw, alpha0), snake64(raw, alpha1), snake64(raw, alpha2)
