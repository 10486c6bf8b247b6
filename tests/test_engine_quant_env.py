"""How ``HipEngine`` picks its weight format from ``quant_bits`` or from the Metal engine's environment
variables (chatterbox_flash/engines/mlx.py:224-235): unset runs bf16; an unparsable value or a width
the Metal engine does not quantise to is ignored with a warning; 4 and 8 quantise; the widths the
Metal engine accepts but this engine does not build (2, 3, 6), and a group size other than 64, raise.
"""

import logging

import pytest

from yapd_amd.engines.hip import _quant_bits_from


@pytest.fixture
def env(monkeypatch):
    monkeypatch.delenv("CHATTERBOX_FLASH_MLX_QUANT_BITS", raising=False)
    monkeypatch.delenv("CHATTERBOX_FLASH_MLX_QUANT_GROUP", raising=False)
    return monkeypatch


def test_unset_runs_bf16(env):
    assert _quant_bits_from(None) == 0
    env.setenv("CHATTERBOX_FLASH_MLX_QUANT_BITS", "  ")
    assert _quant_bits_from(None) == 0


@pytest.mark.parametrize("raw,bits", [("4", 4), ("8", 8), (" 8 ", 8)])
def test_supported_widths(env, raw, bits):
    env.setenv("CHATTERBOX_FLASH_MLX_QUANT_BITS", raw)
    assert _quant_bits_from(None) == bits


@pytest.mark.parametrize("raw", ["four", "4.0", "5", "0", "16", "-4"])
def test_values_the_metal_engine_ignores_warn_and_run_bf16(env, caplog, raw):
    env.setenv("CHATTERBOX_FLASH_MLX_QUANT_BITS", raw)
    with caplog.at_level(logging.WARNING):
        assert _quant_bits_from(None) == 0
    assert "QUANT_BITS" in caplog.text or "quant bits" in caplog.text


@pytest.mark.parametrize("raw", ["2", "3", "6"])
def test_widths_not_built_here_raise(env, raw):
    env.setenv("CHATTERBOX_FLASH_MLX_QUANT_BITS", raw)
    with pytest.raises(ValueError, match="4 or 8 bits"):
        _quant_bits_from(None)


def test_group_size_other_than_64_raises(env):
    env.setenv("CHATTERBOX_FLASH_MLX_QUANT_BITS", "4")
    env.setenv("CHATTERBOX_FLASH_MLX_QUANT_GROUP", "32")
    with pytest.raises(ValueError, match="group size 64"):
        _quant_bits_from(None)


@pytest.mark.parametrize("bits", [0, 4, 8])
def test_explicit_argument_overrides_the_environment(env, bits):
    env.setenv("CHATTERBOX_FLASH_MLX_QUANT_BITS", "8")
    assert _quant_bits_from(bits) == bits


@pytest.mark.parametrize("bits", [2, 3, 5, 6, 16])
def test_explicit_unsupported_width_raises(env, bits):
    with pytest.raises(ValueError, match="4 or 8 bits"):
        _quant_bits_from(bits)
