"""Pins the MLX affine quantisation oracle (engines/mlx.py:221-255 ->
mlx.nn.quantize, documented formula) by its invariants -- |w_hat - w| <= s/2
inside each group, codes in range, exact LSB-first pack/unpack, the group
min and max represented -- and checks the product's torch quantiser
against it bit for bit."""

import numpy as np
import pytest
import torch

from oracle import quant as Q
from yapd_amd.quant import quantize_affine


@pytest.mark.parametrize("bits", [4, 8])
def test_roundtrip_bound(bits):
    rng = np.random.default_rng(bits)
    w = (rng.normal(size=(64, 256)) * 0.02).astype(np.float32)
    packed, s, b = Q.quantize(w, bits)
    assert packed.dtype == np.uint32 and packed.shape == (64, 256 * bits // 32)
    assert s.shape == (64, 4) and s.dtype == np.float16
    codes = Q.unpack(packed, bits, 256)
    assert codes.max() <= (1 << bits) - 1
    w_hat = Q.dequantize(packed, s, b, bits)
    s_full = np.repeat(s.astype(np.float32), 64, axis=1)
    # half a step plus the fp16 rounding of scale/bias (relative 2^-11 each)
    slack = 0.5 * s_full + np.abs(w) * 2e-3 + 1e-7
    assert np.all(np.abs(w_hat - w) <= slack)


def test_pack_unpack_exact_codes():
    for bits in (4, 8):
        rng = np.random.default_rng(0)
        codes = rng.integers(0, 1 << bits, size=(3, 128)).astype(np.uint32)
        per = 32 // bits
        words = np.zeros((3, 128 // per), dtype=np.uint32)
        for j in range(128):  # LSB-first by hand
            words[:, j // per] |= codes[:, j] << np.uint32((j % per) * bits)
        assert np.array_equal(Q.unpack(words, bits, 128), codes)


def test_known_group():
    # one group 0..63 scaled: min 0, max 63*0.01 -> 4-bit scale 0.042, codes round(i*0.01/0.042)
    w = (np.arange(64, dtype=np.float32) * 0.01)[None, :]
    packed, s, b = Q.quantize(w, 4)
    assert float(b[0, 0]) == 0.0
    assert float(s[0, 0]) == pytest.approx(0.63 / 15, rel=1e-3)
    codes = Q.unpack(packed, 4, 64)[0]
    assert codes[0] == 0 and codes[-1] == 15


@pytest.mark.parametrize("bits", [4, 8])
def test_product_quantiser_matches_oracle(bits):
    g = torch.Generator().manual_seed(bits)
    w = torch.randn(96, 512, generator=g) * 0.02
    p_t, s_t, b_t = quantize_affine(w, bits)
    p_o, s_o, b_o = Q.quantize(w.numpy(), bits)
    assert np.array_equal(p_t.numpy().view(np.uint32), p_o)
    assert np.array_equal(s_t.numpy(), s_o) and np.array_equal(b_t.numpy(), b_o)
