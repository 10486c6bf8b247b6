"""Loader and typed wrappers for the native gfx950 library ``libyapd_t3.so``.

The counterpart of the reference's native-kernel convention in
server/kernels.py:103-165: the library is loaded once (``lru_cache``, as
``load_snake_extension`` at server/kernels.py:103-106), every wrapper checks
its tensors before launching (as the ``TORCH_CHECK``s of
server/kernels.py:69-75), launches on the caller's current stream
(server/kernels.py:79) and lets the caller own the outputs.  Unlike
server/kernels.py:110-112 there is no torch fallback: a missing library or
a failed precondition raises.
"""

from __future__ import annotations

import ctypes
import functools
from pathlib import Path
from typing import Optional

import torch

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libyapd_t3.so"

c_int, c_i64, c_u64, c_float, c_size, c_void = (
    ctypes.c_int, ctypes.c_int64, ctypes.c_uint64, ctypes.c_float, ctypes.c_size_t, ctypes.c_void_p)

# name -> (restype, argtypes); mirrors include/yapd_t3.h.
_SIGNATURES = {
    "yapd_last_error": (ctypes.c_char_p, []),
    "yapd_abi_version": (c_int, []),
    "yapd_score_cfg_pmi_unmask": (c_int, [
        c_void, c_i64, c_i64, c_int, c_int, c_int, c_int, c_int, c_int, c_int,
        c_void, c_void, c_void, c_void, c_void, c_void, c_int, c_float, c_int, c_i64, c_i64,
        c_float, c_int, c_u64, c_u64, c_void, c_void, c_void, c_void, c_void, c_void, c_void]),
}


class HipKernelError(RuntimeError):
    """A native entry point returned a nonzero status."""


def library_built() -> bool:
    return LIB_PATH.exists()


@functools.lru_cache(maxsize=1)
def load_library() -> ctypes.CDLL:
    """Load ``libyapd_t3.so`` once; raise ``ImportError`` if it was never built."""
    if not LIB_PATH.exists():
        raise ImportError(f"{LIB_PATH} is missing; build it with `python -m yapd_amd.build`")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def check(rc: int) -> None:
    if rc != 0:
        msg = load_library().yapd_last_error().decode(errors="replace")
        if rc == 1:
            raise ValueError(msg)
        raise HipKernelError(msg)


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def require(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def require_cuda(t: torch.Tensor, name: str, dtype: torch.dtype, device: torch.device,
                 contiguous: bool = True) -> None:
    require(t.is_cuda, f"{name} must be a GPU tensor")
    require(t.device == device, f"{name} is on {t.device}, expected {device}")
    require(t.dtype == dtype, f"{name} must be {dtype}, got {t.dtype}")
    if contiguous:
        require(t.is_contiguous(), f"{name} must be contiguous")


# --------------------------------------------------------------------------- #
# (c) scoring
# --------------------------------------------------------------------------- #

def score_cfg_pmi_unmask(
    logits: torch.Tensor, *, n_pairs: int, cond_row0: int, pair_row_step: int,
    null_row_offset: Optional[int], log_prior: torch.Tensor, xt_blk: torch.Tensor,
    k_step: torch.Tensor, sched: torch.Tensor, q_tab: torch.Tensor, cfg_w: float,
    quantile_on: bool, mask_id: int, stop_id: int, out: dict, active: Optional[torch.Tensor] = None, temperature: float = 0.0,
    pos_gumbel: bool = False, seed: int = 0, rng_offset: int = 0,
) -> None:
    """Launch the scoring kernel; results land in the tensors of ``out``.

    ``logits`` is bf16 ``[rows, bl, V]`` with a unit last stride (a padded
    row pitch is fine); ``out`` holds ``sampled`` (int64), ``pmi`` (fp32),
    ``unmask`` (uint8), ``xt_out`` (int64) of shape ``[n_pairs, bl]`` and
    ``n_mask_after`` (int32), ``hit_eos`` (uint8) of shape ``[n_pairs]``.
    """
    lib = load_library()
    dev = logits.device
    require_cuda(logits, "logits", torch.bfloat16, dev, contiguous=False)
    require(logits.dim() == 3 and logits.stride(2) == 1, "logits must be [rows, bl, V] with unit last stride")
    rows, bl, V = logits.shape
    last_row = cond_row0 + (n_pairs - 1) * pair_row_step + max(0, null_row_offset or 0)
    require(0 <= cond_row0 and last_row < rows, f"pair layout reaches row {last_row} of {rows}")
    require(null_row_offset is None or cond_row0 + null_row_offset >= 0, "null rows out of range")
    require_cuda(log_prior, "log_prior", torch.float32, dev)
    require(log_prior.numel() == V, "log_prior must have V entries")
    require_cuda(xt_blk, "xt_blk", torch.int64, dev)
    require(tuple(xt_blk.shape) == (n_pairs, bl), f"xt_blk must be [{n_pairs}, {bl}]")
    require_cuda(k_step, "k_step", torch.int64, dev)
    require(k_step.numel() == n_pairs, "k_step must have n_pairs entries")
    require_cuda(sched, "sched", torch.int32, dev)
    require_cuda(q_tab, "q_tab", torch.float32, dev)
    require(sched.numel() == q_tab.numel() and sched.numel() >= 1, "sched/q_tab must both have K entries")
    if active is not None:
        require_cuda(active, "active", torch.uint8, dev)
        require(active.numel() == n_pairs, "active must have n_pairs entries")
    for name, dt, shape in (("sampled", torch.int64, (n_pairs, bl)), ("pmi", torch.float32, (n_pairs, bl)),
                            ("unmask", torch.uint8, (n_pairs, bl)), ("xt_out", torch.int64, (n_pairs, bl)),
                            ("n_mask_after", torch.int32, (n_pairs,)), ("hit_eos", torch.uint8, (n_pairs,))):
        t = out[name]
        require_cuda(t, name, dt, dev)
        require(tuple(t.shape) == shape, f"{name} must be {shape}")
    check(lib.yapd_score_cfg_pmi_unmask(
        logits.data_ptr(), logits.stride(0), logits.stride(1), n_pairs, bl, V,
        cond_row0, pair_row_step, 0 if null_row_offset is None else 1, null_row_offset or 0,
        log_prior.data_ptr(), xt_blk.data_ptr(), k_step.data_ptr(), ptr(active),
        sched.data_ptr(), q_tab.data_ptr(), sched.numel(), float(cfg_w), int(bool(quantile_on)),
        int(mask_id), int(stop_id), float(temperature), int(bool(pos_gumbel)),
        int(seed) & (2**64 - 1), int(rng_offset) & (2**64 - 1),
        out["sampled"].data_ptr(), out["pmi"].data_ptr(), out["unmask"].data_ptr(),
        out["xt_out"].data_ptr(), out["n_mask_after"].data_ptr(), out["hit_eos"].data_ptr(),
        stream_ptr(dev)))
