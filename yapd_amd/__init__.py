"""yapd_amd -- MI355X-native (gfx950) T3 block-diffusion decode step.

A drop-in ``backend="hip"`` engine for Chatterbox-Flash's block-diffusion
T3 loop: the engine protocol and ``build_engine`` of
chatterbox_flash/engines/{base,__init__}.py, an ``attention_hip`` shim in the
style of chatterbox_flash/attention_flashinfer.py, and a native library
(``libyapd_t3.so``) of hand-written HIP kernels behind a C ABI
(``include/yapd_t3.h``).
"""

from .engines import HIP_AVAILABLE, InferenceEngine, build_engine

__version__ = "0.1.0"

__all__ = ["HIP_AVAILABLE", "InferenceEngine", "build_engine", "__version__"]
