"""Engine selection with the ``hip`` backend.

Mirrors chatterbox_flash/engines/__init__.py:53-135: ``build_engine`` picks
a backend, honours ``CHATTERBOX_FLASH_ENGINE`` (the env var wins, :55-57),
raises ``ImportError`` when the requested backend cannot run (:61-75) and
``ValueError`` on an unknown name (:78-81).  This package provides the
``hip`` backend; ``auto`` resolves to it when it can run.  The reference's
own backends (``flashinfer``, ``torch``/``sdpa``, ``mlx``) live in
``chatterbox_flash.engines``.
"""

from __future__ import annotations

import logging
import os
from typing import Literal

import torch

from .. import kernels
from .base import InferenceEngine

logger = logging.getLogger(__name__)


def _hip_available() -> bool:
    return kernels.library_built() and torch.cuda.is_available()


HIP_AVAILABLE: bool = _hip_available()

_REFERENCE_BACKENDS = ("flashinfer", "torch", "sdpa", "mlx")


def _resolve_backend(requested: str) -> Literal["hip"]:
    env = os.environ.get("CHATTERBOX_FLASH_ENGINE", "").strip().lower()
    if env:
        requested = env
    if requested in ("auto", "hip"):
        if not _hip_available():
            raise ImportError(
                "backend 'hip' needs libyapd_t3.so (python -m yapd_amd.build) and a visible "
                "MI355X (gfx950) GPU")
        return "hip"
    if requested in _REFERENCE_BACKENDS:
        raise ImportError(
            f"backend {requested!r} is provided by chatterbox_flash.engines, not by yapd_amd")
    raise ValueError(f"backend must be one of 'auto', 'hip'; got {requested!r}")


def build_engine(model: torch.nn.Module, max_seq_len: int, dtype: torch.dtype, *,
                 backend: str = "auto", batch_size: int = 1, page_size: int = 16):
    """Construct the HIP engine (engines/__init__.py:84-135 signature)."""
    _resolve_backend(backend)
    from .hip import HipEngine
    logger.debug("build_engine: backend=hip max_seq=%d dtype=%s batch=%d page=%d",
                 max_seq_len, dtype, batch_size, page_size)
    return HipEngine(model, max_seq_len, dtype, batch_size=batch_size, page_size=page_size)


def __getattr__(name: str):
    if name == "HipEngine":
        from .hip import HipEngine
        return HipEngine
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")


__all__ = ["InferenceEngine", "HipEngine", "HIP_AVAILABLE", "build_engine"]
