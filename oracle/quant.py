"""Oracle: MLX-layout affine group quantisation.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

The reference quantises its Metal backbone with ``mlx.nn.quantize(...,
group_size=64, bits=b)`` (engines/mlx.py:221-255; bits from
``CHATTERBOX_FLASH_MLX_QUANT_BITS`` at :224, group at :235, predicate
``in % group == 0`` at :242-246).  mlx 0.31.2 is not installed here, so its
documented formula is restated: per group of ``g`` consecutive input
features, ``s = (max - min) / (2^b - 1)``, ``beta = min``,
``q = round((w - beta) / s)`` clipped to ``[0, 2^b - 1]``, and
``w_hat = s*q + beta``.  Codes are packed LSB-first into uint32 words
(word ``j*b // 32`` holds element ``j`` at bit ``(j % (32/b)) * b``).
MLX's extra refinement that makes one group edge exactly representable is
not verifiable offline; it changes only which scales/biases are stored, not
the dequantise-then-matmul contract the kernel is checked against.
"""

from __future__ import annotations

import numpy as np


def quantize(w: np.ndarray, bits: int, group: int = 64, scale_dtype=np.float16):
    """``w [out, in]`` fp32 -> (packed uint32 ``[out, in*bits/32]``, scales, biases ``[out, in/group]``)."""
    assert bits in (4, 8) and w.ndim == 2 and w.shape[1] % group == 0
    out, inn = w.shape
    wg = w.astype(np.float32).reshape(out, inn // group, group)
    wmin = wg.min(-1)
    wmax = wg.max(-1)
    nbins = (1 << bits) - 1
    s = np.maximum((wmax - wmin) / nbins, 1e-12).astype(scale_dtype)
    b = wmin.astype(scale_dtype)
    s32 = s.astype(np.float32)[..., None]
    b32 = b.astype(np.float32)[..., None]
    q = np.clip(np.rint((wg - b32) / s32), 0, nbins).astype(np.uint32).reshape(out, inn)
    per = 32 // bits
    qw = q.reshape(out, inn // per, per)
    shifts = (np.arange(per, dtype=np.uint32) * bits)[None, None, :]
    packed = np.bitwise_or.reduce(qw << shifts, axis=-1).astype(np.uint32)
    return packed, s, b


def unpack(packed: np.ndarray, bits: int, n_in: int) -> np.ndarray:
    """Integer codes ``[out, in]`` from the LSB-first packed words."""
    per = 32 // bits
    shifts = (np.arange(per, dtype=np.uint32) * bits)[None, None, :]
    codes = (packed[..., None] >> shifts) & np.uint32((1 << bits) - 1)
    return codes.reshape(packed.shape[0], -1)[:, :n_in]


def dequantize(packed: np.ndarray, scales: np.ndarray, biases: np.ndarray, bits: int,
               group: int = 64) -> np.ndarray:
    """``w_hat = s*q + beta`` in fp32 ``[out, in]``."""
    n_in = scales.shape[1] * group
    q = unpack(packed, bits, n_in).astype(np.float32)
    s = np.repeat(scales.astype(np.float32), group, axis=1)
    b = np.repeat(biases.astype(np.float32), group, axis=1)
    return s * q + b
