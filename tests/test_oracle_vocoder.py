"""Pins for oracle.vocoder (server/kernels.py:35-67) from closed forms and
operation-order cases, so that a dropped square, a missing bias or a
reassociated sum fails."""

import math

import numpy as np
import torch

from oracle import vocoder as OV


def test_snake_closed_forms():
    a = np.array([0.5, 1.0, 2.0, 3.0], dtype=np.float32)
    # v = 0 -> 0; v*a = pi/2 -> v + 1/(a+eps); v*a = pi -> v (sin^2 vanishes)
    v0 = np.zeros((1, 4, 1), np.float32)
    assert np.all(OV.snake(v0, a) == 0.0)
    a64 = a.astype(np.float64)[None, :, None]
    half = (np.float32(math.pi / 2) / a).astype(np.float32)[None, :, None]
    want = half.astype(np.float64) + 1.0 / (a64 + 1e-9) * np.sin(half.astype(np.float64) * a64) ** 2
    np.testing.assert_allclose(OV.snake(half, a), want, rtol=0, atol=1e-15)
    np.testing.assert_allclose(OV.snake(half, a) - half, 1.0 / (a64 + 1e-9), rtol=1e-6)
    full = (np.float32(math.pi) / a).astype(np.float32)[None, :, None]
    np.testing.assert_allclose(OV.snake(full, a), full, rtol=0, atol=1e-6)


def test_snake_forms_and_bounds():
    rng = np.random.default_rng(0)
    x = rng.normal(0, 3, (2, 8, 64)).astype(np.float32)
    a = rng.uniform(0.1, 4, 8).astype(np.float32)
    got = OV.snake(x, a)
    # the reference kernel's form, s^2 / (a + 1e-9), and torch's float64 sin
    a64 = torch.tensor(a, dtype=torch.float64)[None, :, None]
    x64 = torch.tensor(x, dtype=torch.float64)
    ref = (x64 + torch.sin(x64 * a64) ** 2 / (a64 + 1e-9)).numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-13, atol=1e-13)
    # 0 <= snake(v) - v <= 1/a
    d = got - x.astype(np.float64)
    assert d.min() >= 0 and np.all(d <= 1.0 / a.astype(np.float64)[None, :, None] + 1e-12)


def test_bias_is_added_before_the_activation():
    rng = np.random.default_rng(1)
    x = rng.normal(0, 1, (1, 3, 10)).astype(np.float32)
    a = np.array([1.0, 2.0, 0.5], np.float32)
    b = np.array([0.25, -1.0, 3.0], np.float32)
    v = (x + b[None, :, None]).astype(np.float32)
    np.testing.assert_array_equal(OV.snake(x, a, b), OV.snake(v, a))
    assert not np.allclose(OV.snake(x, a, b), OV.snake(x, a) + b[None, :, None])


def test_residual_bias_order_and_mean3():
    # (x + r) + b is not x + (r + b) in float32: 1e8 - 1e8 + 1 = 1, but -1e8 + 1 rounds to -1e8
    x = np.full((1, 1, 1), 1e8, np.float32)
    r = np.full((1, 1, 1), -1e8, np.float32)
    assert OV.residual_bias(x, r, np.array([1.0], np.float32)).item() == 1.0
    raw, act = OV.residual_bias_snake(x, r, np.array([1.0], np.float32), np.array([1.0], np.float32))
    assert raw.item() == 1.0 and act.item() == 1.0 + math.sin(1.0) ** 2 / (1.0 + 1e-9)
    # mean3 = ((a + b) + c) * fl(1/3): two rounded sums (each off by at most 2^-24 of a partial sum
    # bounded by |a|+|b|+|c|), then fl(1/3) and the product (2^-24 each, relative)
    rng = np.random.default_rng(2)
    a, b, c = (rng.normal(0, 10, 1000).astype(np.float32) for _ in range(3))
    m = OV.mean3(a, b, c).astype(np.float64)
    a64, b64, c64 = (t.astype(np.float64) for t in (a, b, c))
    exact = (a64 + b64 + c64) / 3.0
    bound = (np.abs(a64) + np.abs(b64) + np.abs(c64)) * 2.0 ** -24 * 2 / 3 + np.abs(exact) * 2.0 ** -23
    assert np.all(np.abs(m - exact) <= bound)
    big = OV.mean3(np.float32([3e7]), np.float32([-3e7]), np.float32([1.5]))
    assert big.item() == np.float32(np.float32(1.5) * np.float32(1 / 3))


def test_branch_start_is_three_snakes_of_one_sum():
    rng = np.random.default_rng(3)
    x = rng.normal(0, 1, (2, 4, 9)).astype(np.float32)
    s = rng.normal(0, 1, (2, 4, 9)).astype(np.float32)
    al = [rng.uniform(0.2, 3, 4).astype(np.float32) for _ in range(3)]
    raw, o0, o1, o2 = OV.branch_start(x, s, *al)
    np.testing.assert_array_equal(raw, (x + s).astype(np.float32))
    for o, a in zip((o0, o1, o2), al):
        np.testing.assert_array_equal(o, OV.snake(raw, a))
