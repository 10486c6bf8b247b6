"""Affine group quantisation in the MLX layout, and the quantised GEMM (kernel (d)).

The reference's Metal engine quantises the backbone with ``mlx.nn.quantize``
(chatterbox_flash/engines/mlx.py:221-255: bits from
``CHATTERBOX_FLASH_MLX_QUANT_BITS``, group 64 by default, only layers whose
input dim is a multiple of the group).  The documented MLX formula is used:
per group of 64 input features ``scale = (max - min) / (2^bits - 1)``,
``bias = min``, ``q = round((w - bias) / scale)`` clipped to
``[0, 2^bits - 1]`` and ``w_hat = scale * q + bias``; codes are packed
LSB-first into uint32 words; scales and biases are stored as fp16.

Two routes compute ``A @ w_hat^T``, bit for bit alike: the fused kernel
(``yapd_qgemm_affine``) dequantises each W tile on its way into LDS, which
pays at few rows, where reading 4- or 8-bit codes instead of bf16 is what
counts; with a bf16 scratch buffer and at least ``DEQUANT_MIN_ROWS`` rows,
W is dequantised once (``yapd_dequant_affine``) and the bf16 GEMM runs on
it, since the fused kernel repeats the dequantisation for every tile row.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import kernels

GROUP = 64
DEQUANT_MIN_ROWS = 4096


def quantize_affine(w: torch.Tensor, bits: int, group: int = GROUP):
    """``w [out, in]`` -> (packed uint32 as int32 ``[out, in*bits/32]``, scales fp16, biases fp16)."""
    kernels.require(bits in (4, 8), "bits must be 4 or 8")
    kernels.require(w.dim() == 2 and w.shape[1] % group == 0, f"in_features must be a multiple of {group}")
    out_f, in_f = w.shape
    wg = w.float().reshape(out_f, in_f // group, group)
    wmin = wg.amin(-1)
    wmax = wg.amax(-1)
    nbins = (1 << bits) - 1
    scale = ((wmax - wmin) / nbins).clamp_min(1e-12).to(torch.float16)
    bias = wmin.to(torch.float16)
    q = torch.round((wg - bias.float()[..., None]) / scale.float()[..., None]).clamp_(0, nbins)
    q = q.to(torch.int64).reshape(out_f, in_f // (32 // bits), 32 // bits)
    shifts = torch.arange(32 // bits, device=w.device, dtype=torch.int64) * bits
    packed = (q << shifts).sum(-1)                   # < 2^32, exact in int64
    packed = torch.where(packed >= 2 ** 31, packed - 2 ** 32, packed).to(torch.int32)
    return packed.contiguous(), scale.contiguous(), bias.contiguous()


def _check_codes(packed: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, bits: int, K: int, dev) -> int:
    kernels.require(bits in (4, 8), "bits must be 4 or 8")
    N = packed.shape[0]
    kernels.require_cuda(packed, "packed", torch.int32, dev)
    kernels.require(packed.shape[1] * 32 // bits == K, "packed width does not match K")
    for name, t in (("scales", scales), ("biases", biases)):
        kernels.require_cuda(t, name, torch.float16, dev)
        kernels.require(tuple(t.shape) == (N, K // GROUP), f"{name} must be [N, K/64]")
    return N


def dequant_affine(packed: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, bits: int,
                   out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``w_hat [N, K] = bf16(scale * q + bias)`` (``yapd_dequant_affine``), the weights the fused
    kernel multiplies by."""
    dev = packed.device
    K = packed.shape[1] * 32 // bits
    N = _check_codes(packed, scales, biases, bits, K, dev)
    if out is None:
        out = torch.empty(N, K, dtype=torch.bfloat16, device=dev)
    kernels.require_cuda(out, "out", torch.bfloat16, dev)
    kernels.require(out.numel() >= N * K, "out holds fewer than N*K elements")
    kernels.check(kernels.load_library().yapd_dequant_affine(
        packed.data_ptr(), scales.data_ptr(), biases.data_ptr(), int(bits), GROUP, N, K, out.data_ptr(),
        kernels.stream_ptr(dev)))
    return out.view(-1)[: N * K].view(N, K)


def qgemm_affine(A: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, bits: int,
                 out: Optional[torch.Tensor] = None, scratch: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``out[M, N] = A[M, K] @ dequant(W)^T`` in bf16 (fp32 accumulation).  ``scratch`` (bf16, at
    least N*K elements) enables the dequantise-once route at ``DEQUANT_MIN_ROWS`` rows or more."""
    dev = A.device
    kernels.require_cuda(A, "A", torch.bfloat16, dev, contiguous=False)
    kernels.require(A.dim() == 2 and A.stride(1) == 1, "A must be row-major 2-D")
    M, K = A.shape
    N = _check_codes(packed, scales, biases, bits, K, dev)
    if out is None:
        out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    kernels.require_cuda(out, "out", torch.bfloat16, dev, contiguous=False)
    kernels.require(tuple(out.shape) == (M, N) and out.stride(1) == 1, "out must be [M, N] row-major")
    if scratch is not None and M >= DEQUANT_MIN_ROWS:
        kernels.gemm_bf16(A, dequant_affine(packed, scales, biases, bits, out=scratch), out)
        return out
    kernels.check(kernels.load_library().yapd_qgemm_affine(
        A.data_ptr(), A.stride(0), packed.data_ptr(), scales.data_ptr(), biases.data_ptr(), int(bits), GROUP,
        M, N, K, out.data_ptr(), out.stride(0), kernels.stream_ptr(dev)))
    return out


class QuantLinear:
    """A bias-free projection held as MLX-layout codes (``bits`` in {4, 8}, group 64)."""

    def __init__(self, weight: torch.Tensor, bits: int):
        self.bits = int(bits)
        self.out_features, self.in_features = weight.shape
        self.packed, self.scales, self.biases = quantize_affine(weight, self.bits)

    def __call__(self, x: torch.Tensor, out: Optional[torch.Tensor] = None,
                 scratch: Optional[torch.Tensor] = None) -> torch.Tensor:
        lead = x.shape[:-1]
        y = qgemm_affine(x.reshape(-1, self.in_features), self.packed, self.scales, self.biases, self.bits,
                         out=None if out is None else out.view(-1, self.out_features), scratch=scratch)
        return y.view(*lead, self.out_features)
