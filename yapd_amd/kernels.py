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

# name -> (restype, argtypes); mirrors include/yapd_t3.h, yapd_probe.h and yapd_vocoder.h.
_SIGNATURES = {
    "yapd_last_error": (ctypes.c_char_p, []),
    "yapd_abi_version": (c_int, []),
    "yapd_score_cfg_pmi_unmask": (c_int, [
        c_void, c_i64, c_i64, c_int, c_int, c_int, c_int, c_int, c_int, c_int,
        c_void, c_void, c_void, c_void, c_void, c_void, c_int, c_float, c_int, c_i64, c_i64,
        c_float, c_int, c_u64, c_u64, c_void, c_void, c_void, c_void, c_void, c_void, c_void]),
    "yapd_attn_plan": (c_int, [c_void, c_int, c_int, c_int, c_void, c_int, c_void, c_int, c_void, c_void, c_void]),
    "yapd_attn_paged_block": (c_int, [
        c_void, c_void, c_i64, c_void, c_int, c_int, c_void, c_int, c_int, c_int, c_void, c_int, c_void, c_int,
        c_void, c_void, c_void, c_int, c_float, c_int, c_void, c_void]),
    "yapd_attn_paged_block_noalloc": (c_int, [
        c_void, c_void, c_i64, c_void, c_int, c_int, c_void, c_int, c_int, c_int, c_void, c_int, c_void, c_int,
        c_void, c_int, c_float, c_int, c_void, c_void]),
    "yapd_kv_write": (c_int, [c_void, c_void, c_i64, c_i64, c_void, c_i64, c_void, c_int, c_int, c_void, c_int,
                              c_int, c_int, c_void]),
    "yapd_kv_gather": (c_int, [c_void, c_i64, c_void, c_int, c_int, c_int, c_void, c_void, c_void]),
    "yapd_gemm_bf16": (c_int, [c_void, c_i64, c_void, c_i64, c_int, c_int, c_int, c_void, c_i64, c_void]),
    "yapd_gemm_bf16_residual": (c_int, [c_void, c_i64, c_void, c_i64, c_int, c_int, c_int, c_void, c_i64, c_void]),
    "yapd_gemm_head_shift": (c_int, [c_void, c_void, c_int, c_int, c_int, c_void, c_i64, c_int, c_void, c_i64,
                                     c_void]),
    "yapd_gemm_swiglu": (c_int, [c_void, c_i64, c_void, c_int, c_int, c_int, c_void, c_i64, c_void]),
    "yapd_gemm_qkv_rope_kv": (c_int, [c_void, c_i64, c_void, c_int, c_int, c_int, c_void, c_void, c_int, c_void,
                                      c_int, c_void, c_void, c_i64, c_void, c_int, c_int, c_void]),
    "yapd_rmsnorm": (c_int, [c_void, c_void, c_void, c_void, c_float, c_int, c_int, c_void, c_void]),
    "yapd_gemm_rmsnorm_qkv_rope_kv": (c_int, [c_void, c_void, c_float, c_void, c_void, c_int, c_int, c_int, c_void,
                                              c_void, c_int, c_void, c_int, c_void, c_void, c_i64, c_void, c_int,
                                              c_int, c_void]),
    "yapd_qgemm_affine": (c_int, [c_void, c_i64, c_void, c_void, c_void, c_int, c_int, c_int, c_int, c_int,
                                  c_void, c_i64, c_void]),
    "yapd_dequant_affine": (c_int, [c_void, c_void, c_void, c_int, c_int, c_int, c_int, c_void, c_void]),
    "yapd_mfma_peak_probe": (c_int, [c_int, c_int, c_int, c_void, c_void]),
    "yapd_hbm_read_probe": (c_int, [c_void, c_i64, c_int, c_void, c_void]),
    "yapd_tick_update": (c_int, [c_int, c_int, c_int, c_int, c_int, c_i64, c_i64, c_i64, c_i64, c_void, c_i64,
                                 c_void, c_void, c_void, c_void, c_void, c_void, c_void, c_void, c_void, c_void,
                                 c_void, c_void]),
    "yapd_t3_block_forward": (c_int, [c_void, c_void, c_void, c_int, c_int, c_void, c_void, c_int, c_void,
                                      c_void, c_int, c_void, c_void, c_i64, c_void]),
    "yapd_t3_prefill_packed": (c_int, [c_void, c_void, c_void, c_int, c_int, c_int, c_void, c_void, c_void, c_void,
                                       c_void, c_void]),
    # include/yapd_vocoder.h
    "yapd_snake": (c_int, [c_void, c_void, c_void, c_void, c_i64, c_int, c_i64, c_void]),
    "yapd_residual_bias": (c_int, [c_void, c_void, c_void, c_void, c_i64, c_int, c_i64, c_void]),
    "yapd_mean3": (c_int, [c_void, c_void, c_void, c_void, c_i64, c_void]),
    "yapd_residual_bias_snake": (c_int, [c_void, c_void, c_void, c_void, c_void, c_void, c_i64, c_int, c_i64,
                                         c_void]),
    "yapd_branch_start": (c_int, [c_void, c_void, c_void, c_void, c_void, c_void, c_void, c_void, c_void, c_i64,
                                  c_int, c_i64, c_void]),
    "yapd_voc_stitch": (c_int, [c_void, c_i64, c_i64, c_int, c_void, c_int, c_void, c_void, c_int, c_void, c_int,
                                c_void, c_int, c_void, c_int, c_void, c_i64, c_void]),
}

STITCH_JOB_INTS = 12  # YAPD_STITCH_JOB_INTS of include/yapd_vocoder.h


class T3QWeight(ctypes.Structure):
    """``yapd_t3_qweight`` of include/yapd_t3.h (MLX-layout codes, fp16 scales and biases)."""
    _fields_ = [("packed", c_void), ("scales", c_void), ("biases", c_void)]


class T3Layer(ctypes.Structure):
    """``yapd_t3_layer`` of include/yapd_t3.h (``qbits`` 0: the bf16 weights; 4 or 8: ``q_*``)."""
    _fields_ = [("w_qkv", c_void), ("w_o", c_void), ("w_gate_up", c_void), ("w_down", c_void),
                ("ln_in", c_void), ("ln_post", c_void), ("eps_in", c_float), ("eps_post", c_float),
                ("kv_pool", c_void), ("qbits", c_int), ("q_qkv", T3QWeight), ("q_o", T3QWeight),
                ("q_gate_up", T3QWeight), ("q_down", T3QWeight)]


class T3Model(ctypes.Structure):
    """``yapd_t3_model`` of include/yapd_t3.h."""
    _fields_ = [("n_layers", c_int), ("hidden", c_int), ("n_heads", c_int), ("ffn", c_int),
                ("layers", ctypes.POINTER(T3Layer)), ("final_norm", c_void), ("final_eps", c_float),
                ("rope_cos", c_void), ("rope_sin", c_void), ("rope_positions", c_int), ("n_pages", c_i64),
                ("page_table", c_void), ("table_stride", c_int), ("table_cols", c_int)]


class T3Workspace(ctypes.Structure):
    """``yapd_t3_workspace`` of include/yapd_t3.h."""
    _fields_ = [("residual", c_void), ("q", c_void), ("attn", c_void), ("normed", c_void), ("delta", c_void),
                ("act", c_void), ("work", c_void), ("n_work", c_int), ("merge", c_void), ("n_merge", c_int),
                ("counts", c_void), ("part_o", c_void), ("part_ml", c_void), ("n_slots", c_int),
                ("wdq", c_void), ("wdq_elems", c_i64)]


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


# --------------------------------------------------------------------------- #
# (a) paged block attention
# --------------------------------------------------------------------------- #

def attn_plan(kv_len, target_items: int = 192, min_split_keys: int = 1024):
    """Host planner: ``(work [n,4] int32, merge [m,3] int32, n_slots)`` numpy arrays.

    Rows are cut into work items of whole 32-key chunks so that about
    ``target_items`` items exist (192 is roughly how many four-head work items
    the MI355X keeps in flight, so only rows longer than the average share are
    split), never into items shorter than ``min_split_keys``; items are ordered
    longest first.  1024 keys (1 MB of K/V per four-head item) is where the
    split rows' merges and per-item start-up cost less than the tail they
    remove: on 256 rows of log-uniform [64, 2048] keys, 1024 runs 125 us per
    layer against 128 us at 128 keys and 131 us at 1280 keys.
    """
    import numpy as np
    kv = np.ascontiguousarray(np.asarray(kv_len, dtype=np.int32))
    rows = int(kv.size)
    unit = 32
    cap = int(sum((int(x) + unit - 1) // unit for x in kv)) + rows
    work = np.zeros((cap, 4), dtype=np.int32)
    merge = np.zeros((rows, 3), dtype=np.int32)
    nw, nm, ns = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    check(load_library().yapd_attn_plan(
        kv.ctypes.data, rows, int(target_items), int(min_split_keys), work.ctypes.data, cap,
        merge.ctypes.data, rows, ctypes.byref(nw), ctypes.byref(nm), ctypes.byref(ns)))
    return work[: nw.value].copy(), merge[: nm.value].copy(), ns.value


def attn_paged_block(q: torch.Tensor, pool: torch.Tensor, table: torch.Tensor, kv_len: torch.Tensor,
                     work: torch.Tensor, merge: Optional[torch.Tensor], part_o: Optional[torch.Tensor],
                     part_ml: Optional[torch.Tensor], out: torch.Tensor, scale: float,
                     causal: bool = False) -> None:
    """``out [rows, bl, H, 64] = softmax(q K^T * scale) V`` over each row's pages.

    ``causal``: query ``i`` of the block sees keys ``< kv_len - bl + i + 1`` (prefill).
    """
    dev = q.device
    require_cuda(q, "q", torch.bfloat16, dev)
    require(q.dim() == 4 and q.shape[3] == 64, "q must be [rows, bl, H, 64]")
    rows, bl, H, _ = q.shape
    require_cuda(pool, "pool", torch.bfloat16, dev)
    require(pool.dim() == 4 and pool.shape[1] == 2 and pool.shape[2] == H and pool.shape[3] == 1024,
            "pool must be [pages, 2, H, 16*64]")
    require_cuda(table, "table", torch.int32, dev, contiguous=False)
    require(table.dim() == 2 and table.shape[0] >= rows and table.stride(1) == 1,
            "table must be [>= rows, max_pages] with unit column stride")
    require_cuda(kv_len, "kv_len", torch.int32, dev)
    require(kv_len.numel() >= rows, "kv_len must have rows entries")
    require_cuda(work, "work", torch.int32, dev)
    require(work.dim() == 2 and work.shape[1] == 4, "work must be [n, 4]")
    n_merge = 0 if merge is None else int(merge.shape[0])
    n_slots = 0
    if n_merge:
        require_cuda(merge, "merge", torch.int32, dev)
        require_cuda(part_o, "part_o", torch.float32, dev)
        require_cuda(part_ml, "part_ml", torch.float32, dev)
        n_slots = int(part_o.shape[0])
        require(tuple(part_o.shape[1:]) == (bl, H, 64) and tuple(part_ml.shape) == (n_slots, bl, H, 2),
                "part_o/part_ml shapes")
    require_cuda(out, "out", torch.bfloat16, dev)
    require(tuple(out.shape) == (rows, bl, H, 64), "out must match q")
    check(load_library().yapd_attn_paged_block(
        q.data_ptr(), pool.data_ptr(), pool.shape[0], table.data_ptr(), table.stride(0), table.shape[1],
        kv_len.data_ptr(),
        rows, bl, H, work.data_ptr(), int(work.shape[0]), ptr(merge), n_merge, None, ptr(part_o), ptr(part_ml),
        n_slots, float(scale), int(bool(causal)), out.data_ptr(), stream_ptr(dev)))


def kv_write(k: torch.Tensor, v: torch.Tensor, pool: torch.Tensor, table: torch.Tensor,
             pos0: torch.Tensor, bl: int) -> None:
    """Scatter ``k, v`` (``[rows*bl, H, 64]`` views, unit last strides) into the pages."""
    dev = k.device
    for name, t in (("k", k), ("v", v)):
        require_cuda(t, name, torch.bfloat16, dev, contiguous=False)
        require(t.dim() == 3 and t.shape[2] == 64 and t.stride(2) == 1 and t.stride(1) == 64,
                f"{name} must be [tokens, H, 64] with packed heads")
    H = k.shape[1]
    require_cuda(pool, "pool", torch.bfloat16, dev)
    require(pool.dim() == 4 and pool.shape[2] == H and pool.shape[3] == 1024, "pool must be [pages, 2, H, 1024]")
    require_cuda(table, "table", torch.int32, dev)
    require_cuda(pos0, "pos0", torch.int32, dev)
    rows = int(pos0.numel())
    require(k.shape[0] == rows * bl and v.shape[0] == rows * bl, "k/v must hold rows*bl tokens")
    check(load_library().yapd_kv_write(
        k.data_ptr(), v.data_ptr(), k.stride(0), v.stride(0), pool.data_ptr(), pool.shape[0],
        table.data_ptr(), table.stride(0), table.shape[1], pos0.data_ptr(), rows, bl, H, stream_ptr(dev)))


def kv_gather(pool: torch.Tensor, table_row: torch.Tensor, kv_len: int):
    """Dense ``K, V [kv_len, H, 64]`` of one row (page-table gather, debug/test path)."""
    dev = pool.device
    require_cuda(pool, "pool", torch.bfloat16, dev)
    require_cuda(table_row, "table_row", torch.int32, dev)
    H = pool.shape[2]
    require(table_row.numel() * 16 >= kv_len, "table_row too short for kv_len")
    k = torch.empty(kv_len, H, 64, dtype=torch.bfloat16, device=dev)
    v = torch.empty_like(k)
    check(load_library().yapd_kv_gather(pool.data_ptr(), pool.shape[0], table_row.data_ptr(), table_row.numel(),
                                        int(kv_len), H, k.data_ptr(), v.data_ptr(), stream_ptr(dev)))
    return k, v


# --------------------------------------------------------------------------- #
# (b) GEMMs and norms
# --------------------------------------------------------------------------- #

def _mat(t: torch.Tensor, name: str, dev) -> None:
    require_cuda(t, name, torch.bfloat16, dev, contiguous=False)
    require(t.dim() == 2 and t.stride(1) == 1, f"{name} must be a 2-D row-major view")


def gemm_bf16(A: torch.Tensor, W: torch.Tensor, out: torch.Tensor) -> None:
    """``out[M, N] = A[M, K] @ W[N, K]^T`` in bf16 with fp32 accumulation."""
    dev = A.device
    _mat(A, "A", dev)
    _mat(W, "W", dev)
    _mat(out, "out", dev)
    M, K = A.shape
    N = W.shape[0]
    require(W.shape[1] == K and tuple(out.shape) == (M, N), "gemm shapes")
    check(load_library().yapd_gemm_bf16(A.data_ptr(), A.stride(0), W.data_ptr(), W.stride(0), M, N, K,
                                        out.data_ptr(), out.stride(0), stream_ptr(dev)))


def gemm_bf16_residual(A: torch.Tensor, W: torch.Tensor, residual: torch.Tensor) -> None:
    """``residual = bf16(residual + bf16(A @ W^T))`` in place (projection + residual add)."""
    dev = A.device
    _mat(A, "A", dev)
    _mat(W, "W", dev)
    _mat(residual, "residual", dev)
    M, K = A.shape
    N = W.shape[0]
    require(W.shape[1] == K and tuple(residual.shape) == (M, N), "gemm shapes")
    check(load_library().yapd_gemm_bf16_residual(A.data_ptr(), A.stride(0), W.data_ptr(), W.stride(0), M, N, K,
                                                 residual.data_ptr(), residual.stride(0), stream_ptr(dev)))


def gemm_head_shift(hidden: torch.Tensor, shift_ctx: torch.Tensor, W: torch.Tensor, logits: torch.Tensor) -> None:
    """Token-shifted head: ``logits[r, j] = W @ (j ? hidden[r, j-1] : shift_ctx[r])``.

    ``hidden [rows, bl, D]`` contiguous, ``shift_ctx [rows, 1, D]`` contiguous,
    ``logits [rows, bl, V]`` with a unit last stride (padded pitch allowed).
    """
    dev = hidden.device
    require_cuda(hidden, "hidden", torch.bfloat16, dev)
    require_cuda(shift_ctx, "shift_ctx", torch.bfloat16, dev)
    _mat(W, "W", dev)
    rows, bl, D = hidden.shape
    require(tuple(shift_ctx.shape) == (rows, 1, D), "shift_ctx must be [rows, 1, D]")
    require_cuda(logits, "logits", torch.bfloat16, dev, contiguous=False)
    V = W.shape[0]
    require(tuple(logits.shape) == (rows, bl, V) and logits.stride(2) == 1 and logits.stride(0) == bl * logits.stride(1),
            "logits must be [rows, bl, V] with rows packed")
    check(load_library().yapd_gemm_head_shift(hidden.data_ptr(), shift_ctx.data_ptr(), rows, bl, D, W.data_ptr(),
                                              W.stride(0), V, logits.data_ptr(), logits.stride(1), stream_ptr(dev)))


def gemm_swiglu(A: torch.Tensor, W_gu_interleaved: torch.Tensor, act: torch.Tensor) -> None:
    """``act[M, F] = silu(A Wg^T) * (A Wu^T)`` with gate/up rows interleaved per 32 (see interleave_gate_up)."""
    dev = A.device
    _mat(A, "A", dev)
    require_cuda(W_gu_interleaved, "W_gu", torch.bfloat16, dev)
    _mat(act, "act", dev)
    M, K = A.shape
    F = W_gu_interleaved.shape[0] // 2
    require(W_gu_interleaved.shape[1] == K and tuple(act.shape) == (M, F), "swiglu shapes")
    check(load_library().yapd_gemm_swiglu(A.data_ptr(), A.stride(0), W_gu_interleaved.data_ptr(), M, F, K,
                                          act.data_ptr(), act.stride(0), stream_ptr(dev)))


def interleave_gate_up(w_gate: torch.Tensor, w_up: torch.Tensor) -> torch.Tensor:
    """Rows ``[g(32w..32w+31); u(32w..32w+31)]`` for w = 0..F/32-1: gate and up of a
    feature land in the same lane of the swiglu epilogue."""
    F, K = w_gate.shape
    require(F % 64 == 0 and w_up.shape == w_gate.shape, "gate/up must be [F, K] with F % 64 == 0")
    return torch.stack([w_gate.view(F // 32, 32, K), w_up.view(F // 32, 32, K)], 1).reshape(2 * F, K).contiguous()


def gemm_qkv_rope_kv(A: torch.Tensor, W_qkv: torch.Tensor, cos_t: torch.Tensor, sin_t: torch.Tensor,
                     pos0: torch.Tensor, bl: int, q_out: torch.Tensor, pool: torch.Tensor,
                     table: torch.Tensor) -> None:
    """Fused QKV projection + NeoX RoPE + paged KV write (q to ``q_out [M, H*64]``).

    ``cos_t``/``sin_t`` are HF's [P, 64] tables (cat(freqs, freqs): column
    d + 32 equals column d); the kernel reads columns 0..31."""
    dev = A.device
    _mat(A, "A", dev)
    require_cuda(W_qkv, "W_qkv", torch.bfloat16, dev)
    M, K = A.shape
    H = pool.shape[2]
    require(tuple(W_qkv.shape) == (3 * H * 64, K), "W_qkv must be [3*H*64, K]")
    require_cuda(cos_t, "cos_t", torch.float32, dev)
    require_cuda(sin_t, "sin_t", torch.float32, dev)
    require(cos_t.shape == sin_t.shape and cos_t.dim() == 2 and cos_t.shape[1] == 64, "cos/sin must be [P, 64]")
    require_cuda(pos0, "pos0", torch.int32, dev)
    require(M % bl == 0 and pos0.numel() == M // bl, "pos0 must have M / bl entries")
    require_cuda(q_out, "q_out", torch.bfloat16, dev)
    require(tuple(q_out.shape) in ((M, H * 64), (M // bl, bl, H, 64)), "q_out shape")
    require_cuda(pool, "pool", torch.bfloat16, dev)
    require_cuda(table, "table", torch.int32, dev, contiguous=False)
    require(table.stride(1) == 1 and table.shape[0] >= M // bl, "table shape")
    check(load_library().yapd_gemm_qkv_rope_kv(
        A.data_ptr(), A.stride(0), W_qkv.data_ptr(), M, K, H, cos_t.data_ptr(), sin_t.data_ptr(), cos_t.shape[0],
        pos0.data_ptr(), bl, q_out.data_ptr(), pool.data_ptr(), pool.shape[0], table.data_ptr(), table.stride(0),
        table.shape[1], stream_ptr(dev)))


def gemm_rmsnorm_qkv_rope_kv(x: torch.Tensor, ln_w: torch.Tensor, eps: float, normed: torch.Tensor,
                             W_qkv: torch.Tensor, cos_t: torch.Tensor, sin_t: torch.Tensor, pos0: torch.Tensor,
                             bl: int, q_out: torch.Tensor, pool: torch.Tensor, table: torch.Tensor) -> None:
    """Input RMSNorm of the residual stream ``x [M, K]`` into ``normed`` (a caller workspace of the
    same shape), then :func:`gemm_qkv_rope_kv` on it (``yapd_gemm_rmsnorm_qkv_rope_kv``): two
    launches, not a fused kernel."""
    dev = x.device
    require_cuda(x, "x", torch.bfloat16, dev)
    require(x.dim() == 2, "x must be [M, K]")
    M, K = x.shape
    require_cuda(ln_w, "ln_w", torch.bfloat16, dev)
    require(ln_w.numel() == K, "ln_w must have K entries")
    require_cuda(normed, "normed", torch.bfloat16, dev)
    require(tuple(normed.shape) == (M, K), "normed must be [M, K]")
    require_cuda(W_qkv, "W_qkv", torch.bfloat16, dev)
    H = pool.shape[2]
    require(tuple(W_qkv.shape) == (3 * H * 64, K), "W_qkv must be [3*H*64, K]")
    require_cuda(cos_t, "cos_t", torch.float32, dev)
    require_cuda(sin_t, "sin_t", torch.float32, dev)
    require(cos_t.shape == sin_t.shape and cos_t.dim() == 2 and cos_t.shape[1] == 64, "cos/sin must be [P, 64]")
    require_cuda(pos0, "pos0", torch.int32, dev)
    require(M % bl == 0 and pos0.numel() == M // bl, "pos0 must have M / bl entries")
    require_cuda(q_out, "q_out", torch.bfloat16, dev)
    require(tuple(q_out.shape) in ((M, H * 64), (M // bl, bl, H, 64)), "q_out shape")
    require_cuda(pool, "pool", torch.bfloat16, dev)
    require_cuda(table, "table", torch.int32, dev, contiguous=False)
    require(table.stride(1) == 1 and table.shape[0] >= M // bl, "table shape")
    check(load_library().yapd_gemm_rmsnorm_qkv_rope_kv(
        x.data_ptr(), ln_w.data_ptr(), float(eps), normed.data_ptr(), W_qkv.data_ptr(), M, K, H, cos_t.data_ptr(),
        sin_t.data_ptr(), cos_t.shape[0], pos0.data_ptr(), bl, q_out.data_ptr(), pool.data_ptr(), pool.shape[0],
        table.data_ptr(), table.stride(0), table.shape[1], stream_ptr(dev)))


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float, out: torch.Tensor,
            delta: Optional[torch.Tensor] = None) -> None:
    """``out = rmsnorm(x) * w``; with ``delta``: ``x += delta`` (bf16, in place) first."""
    dev = x.device
    for name, t in (("x", x), ("w", w), ("out", out)):
        require_cuda(t, name, torch.bfloat16, dev)
    D = x.shape[-1]
    M = x.numel() // D
    require(out.shape == x.shape and w.numel() == D, "rmsnorm shapes")
    if delta is not None:
        require_cuda(delta, "delta", torch.bfloat16, dev)
        require(delta.shape == x.shape, "delta shape")
    check(load_library().yapd_rmsnorm(ptr(delta), x.data_ptr() if delta is not None else None,
                                      x.data_ptr() if delta is None else None, w.data_ptr(), float(eps), M, D,
                                      out.data_ptr(), stream_ptr(dev)))


def mfma_peak_probe(blocks: int, iters: int, out: torch.Tensor, random_operands: bool = True) -> float:
    """Launch the register-only MFMA calibration kernel (random or constant operands); returns its
    flop count."""
    require_cuda(out, "out", torch.float32, out.device)
    require(out.numel() >= blocks * 256, "out needs blocks * 256 floats")
    check(load_library().yapd_mfma_peak_probe(blocks, iters, int(bool(random_operands)), out.data_ptr(),
                                              stream_ptr(out.device)))
    return float(blocks) * 4 * iters * 8 * 32768


def hbm_read_probe(src: torch.Tensor, blocks: int, out: torch.Tensor) -> int:
    """Launch the streaming-read calibration kernel over all of ``src`` (contiguous, 16-byte aligned,
    a multiple of 16 bytes): workgroup b folds its contiguous share of 16-byte words, thread t of it the
    words b P + t, b P + t + 256, ... (P = the share rounded up to 256 words) by XOR into ``out[b * 256 + t]``.
    Returns the bytes read."""
    dev = src.device
    require(src.is_cuda and src.is_contiguous(), "src must be a contiguous GPU tensor")
    nbytes = src.numel() * src.element_size()
    require(nbytes % 16 == 0 and src.data_ptr() % 16 == 0, "src must be 16-byte aligned, a multiple of 16 bytes")
    require_cuda(out, "out", torch.int32, dev)
    require(out.numel() >= blocks * 256, "out needs blocks * 256 words")
    check(load_library().yapd_hbm_read_probe(src.data_ptr(), nbytes, blocks, out.data_ptr(), stream_ptr(dev)))
    return nbytes


def tick_update(*, xt: torch.Tensor, xt_blk: torch.Tensor, xt_new: torch.Tensor, k_step: torch.Tensor,
                cache_len: torch.Tensor, blk_start: torch.Tensor, is_commit: torch.Tensor, n_speech: torch.Tensor,
                hidden: torch.Tensor, shift_ctx: torch.Tensor, flags: torch.Tensor, xt_final: torch.Tensor,
                n_branch: int, K: int, mask_id: int, stop_id: int, max_len: int) -> None:
    """Continuous-batching state update after the scorer (``yapd_tick_update``) for the first
    ``xt_blk.shape[0]`` slots; every state tensor is updated in place."""
    dev = xt.device
    S, bl = xt_blk.shape
    D = hidden.shape[-1]
    for name, t in (("xt_blk", xt_blk), ("xt_new", xt_new), ("xt_final", xt_final)):
        require_cuda(t, name, torch.int64, dev)
        require(tuple(t.shape) == (S, bl), f"{name} must be [slots, bl]")
    require_cuda(xt, "xt", torch.int64, dev, contiguous=False)
    require(xt.dim() == 2 and xt.stride(1) == 1 and xt.shape[0] >= S, "xt must be [slots, n_max] row-major")
    for name, t in (("k_step", k_step), ("cache_len", cache_len), ("blk_start", blk_start), ("n_speech", n_speech)):
        require_cuda(t, name, torch.int64, dev)
        require(t.numel() >= S, f"{name} needs one entry per slot")
    require_cuda(is_commit, "is_commit", torch.uint8, dev)
    require(is_commit.numel() >= S, "is_commit needs one entry per slot")
    require_cuda(hidden, "hidden", torch.bfloat16, dev)
    require(hidden.numel() >= S * n_branch * bl * D, "hidden must hold slots * n_branch * bl rows")
    require_cuda(shift_ctx, "shift_ctx", torch.bfloat16, dev)
    require(shift_ctx.numel() >= S * n_branch * D and shift_ctx.shape[-1] == D, "shift_ctx must be [rows, 1, D]")
    require_cuda(flags, "flags", torch.int64, dev)
    require(tuple(flags.shape) == (S, 6), "flags must be [slots, 6]")
    check(load_library().yapd_tick_update(
        S, bl, n_branch, D, K, mask_id, stop_id, max_len, xt.shape[1], xt.data_ptr(), xt.stride(0),
        xt_blk.data_ptr(), xt_new.data_ptr(), k_step.data_ptr(), cache_len.data_ptr(), blk_start.data_ptr(),
        is_commit.data_ptr(), n_speech.data_ptr(), hidden.data_ptr(), shift_ctx.data_ptr(), flags.data_ptr(),
        xt_final.data_ptr(), stream_ptr(dev)))


# --------------------------------------------------------------------------- #
# streaming vocoder: chunk stitching
# --------------------------------------------------------------------------- #

def voc_stitch(wav: torch.Tensor, jobs: torch.Tensor, fade_in: torch.Tensor, fade_out: torch.Tensor,
               trim: torch.Tensor, tails_in: Optional[torch.Tensor], tails_out: Optional[torch.Tensor],
               pcm: torch.Tensor) -> None:
    """Stitch a micro-batch's chunks into int16 PCM (``yapd_voc_stitch``, include/yapd_vocoder.h).

    ``wav`` fp32 ``[rows, S]`` with a unit last stride; ``jobs`` int32
    ``[n_jobs, 12]`` on the device (the layout of the header); ``fade_in`` /
    ``fade_out`` fp32 ``[fade]``; ``trim`` fp32 ``[n_trim]``; ``tails_in`` /
    ``tails_out`` fp32 ``[n, fade]`` or None; ``pcm`` int16, flat.
    """
    lib = load_library()
    dev = wav.device
    require_cuda(wav, "wav", torch.float32, dev, contiguous=False)
    require(wav.dim() == 2 and wav.stride(1) == 1, "wav must be [rows, samples] with unit last stride")
    require_cuda(jobs, "jobs", torch.int32, dev)
    require(jobs.dim() == 2 and jobs.shape[1] == STITCH_JOB_INTS, f"jobs must be [n, {STITCH_JOB_INTS}]")
    fade = fade_in.numel()
    for t, name in ((fade_in, "fade_in"), (fade_out, "fade_out"), (trim, "trim")):
        require_cuda(t, name, torch.float32, dev)
    require(fade_out.numel() == fade, "fade_in and fade_out must have the same length")
    for t, name in ((tails_in, "tails_in"), (tails_out, "tails_out")):
        if t is not None:
            require_cuda(t, name, torch.float32, dev)
            require(t.dim() == 2 and t.shape[1] == fade, f"{name} must be [n, {fade}]")
    require_cuda(pcm, "pcm", torch.int16, dev)
    n_in = 0 if tails_in is None else tails_in.shape[0]
    n_out = 0 if tails_out is None else tails_out.shape[0]
    check(lib.yapd_voc_stitch(wav.data_ptr(), wav.stride(0), wav.shape[1], wav.shape[0], jobs.data_ptr(),
                              jobs.shape[0], fade_in.data_ptr(), fade_out.data_ptr(), fade, ptr(trim),
                              trim.numel(), ptr(tails_in), n_in, ptr(tails_out), n_out, pcm.data_ptr(), pcm.numel(),
                              stream_ptr(dev)))
