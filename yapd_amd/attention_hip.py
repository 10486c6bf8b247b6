"""Re-export shim for the HIP engine, in the style of
chatterbox_flash/attention_flashinfer.py:15-20 (``FlashInferEngine`` and
``flashinfer_available``)."""

from __future__ import annotations

from .engines import _hip_available
from .engines.hip import HipEngine


def hip_available() -> bool:
    """True when libyapd_t3.so is built and a GPU is visible."""
    return _hip_available()


__all__ = ["HipEngine", "hip_available"]
