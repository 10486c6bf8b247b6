"""The HiFT vocoder's fused elementwise family on gfx950, behind the operator
API of server/kernels.py.

``load_snake_extension()`` returns an object carrying the six ops the
reference's run-time extension binds (server/kernels.py:19-26): ``snake``,
``snake_bias``, ``residual_bias``, ``mean3``, ``residual_bias_snake`` and
``branch_start`` -- same names and argument meaning, outputs allocated like
``torch::empty_like`` (server/kernels.py:77-100), a ``RuntimeError`` with the
reference's message when a check fails (server/kernels.py:69-75).  The
kernels are those of ``libyapd_t3.so`` (include/yapd_vocoder.h) and run on the
caller's current stream; a missing library raises ``ImportError``.

``install_fused_snake(module)`` rewires an S3Gen HiFT generator as
server/kernels.py:154-165 does: in every ``ResBlock`` the conv biases move into
the neighbouring ops (``convs1[i].bias`` becomes ``activations2[i].pre_bias``,
``convs2[i].bias`` becomes ``residual_bias_{i}``) and the forward becomes the
fused chain of server/kernels.py:114-121; a ``HiFTGenerator``'s decode averages
its resblocks with ``mean3`` (server/kernels.py:125-152); every ``Snake``'s
forward goes through the kernel.  It returns the number of Snake modules.

Two deliberate differences: an ``alpha_logscale`` Snake runs the kernel on
``exp(alpha)`` (the reference falls back to torch ops there, and in the fused
resblock passes the log-scale alpha of the next activation unconverted,
server/kernels.py:118), and all tensors of one call must be on one device.
The installed forwards have no torch-expression path (the reference falls
back to one for inputs its kernels do not take, server/kernels.py:110-112,
120, 142-146): a strided fp32 [B, C, T] GPU tensor is copied to a contiguous
one, any other input raises, and a generator whose decode averages other than
three resblocks is refused at install time.
"""

from __future__ import annotations

import functools
from types import MethodType
from typing import List

import torch
import torch.nn.functional as F

from . import kernels

def _bct_ok(x: torch.Tensor) -> bool:
    """What the kernels take: a contiguous 3-D fp32 GPU tensor."""
    return x.is_cuda and x.dtype == torch.float32 and x.is_contiguous() and x.dim() == 3


def _need_bct(x: torch.Tensor) -> None:
    if not _bct_ok(x):
        raise RuntimeError("contiguous fp32 CUDA BCT required")


def _need_channel(x: torch.Tensor, v: torch.Tensor, name: str) -> None:
    if not (v.is_cuda and v.dtype == torch.float32 and v.is_contiguous() and v.numel() == x.size(1)):
        raise RuntimeError(name)


def _need_same(ref: torch.Tensor, *others: torch.Tensor) -> None:
    for t in others:
        if t.device != ref.device:
            raise RuntimeError(f"tensors must be on one device ({ref.device} vs {t.device})")


class SnakeOps:
    """The operator object of server/kernels.py:103-106, backed by libyapd_t3."""

    def __init__(self) -> None:
        self._lib = kernels.load_library()

    def _bct(self, x: torch.Tensor):
        B, C, T = x.shape
        return B, C, T, kernels.stream_ptr(x.device)

    def snake(self, x: torch.Tensor, alpha: torch.Tensor) -> torch.Tensor:
        _need_bct(x)
        _need_channel(x, alpha, "alpha mismatch")
        _need_same(x, alpha)
        out = torch.empty_like(x)
        B, C, T, st = self._bct(x)
        kernels.check(self._lib.yapd_snake(x.data_ptr(), alpha.data_ptr(), None, out.data_ptr(), B, C, T, st))
        return out

    def snake_bias(self, x: torch.Tensor, alpha: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
        _need_bct(x)
        _need_channel(x, alpha, "alpha mismatch")
        _need_channel(x, bias, "bias mismatch")
        _need_same(x, alpha, bias)
        out = torch.empty_like(x)
        B, C, T, st = self._bct(x)
        kernels.check(self._lib.yapd_snake(x.data_ptr(), alpha.data_ptr(), bias.data_ptr(), out.data_ptr(), B, C, T,
                                           st))
        return out

    def residual_bias(self, x: torch.Tensor, residual: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
        _need_bct(x)
        _need_bct(residual)
        if x.shape != residual.shape:
            raise RuntimeError("residual shape mismatch")
        _need_channel(x, bias, "bias mismatch")
        _need_same(x, residual, bias)
        out = torch.empty_like(x)
        B, C, T, st = self._bct(x)
        kernels.check(self._lib.yapd_residual_bias(x.data_ptr(), residual.data_ptr(), bias.data_ptr(), out.data_ptr(),
                                                   B, C, T, st))
        return out

    def mean3(self, a: torch.Tensor, b: torch.Tensor, c: torch.Tensor) -> torch.Tensor:
        for t in (a, b, c):
            _need_bct(t)
        if not (a.shape == b.shape == c.shape):
            raise RuntimeError("mean3 shape mismatch")
        _need_same(a, b, c)
        out = torch.empty_like(a)
        kernels.check(self._lib.yapd_mean3(a.data_ptr(), b.data_ptr(), c.data_ptr(), out.data_ptr(), a.numel(),
                                           kernels.stream_ptr(a.device)))
        return out

    def residual_bias_snake(self, x: torch.Tensor, residual: torch.Tensor, bias: torch.Tensor,
                            alpha: torch.Tensor) -> List[torch.Tensor]:
        _need_bct(x)
        _need_bct(residual)
        if x.shape != residual.shape:
            raise RuntimeError("residual shape mismatch")
        _need_channel(x, bias, "bias mismatch")
        _need_channel(x, alpha, "alpha mismatch")
        _need_same(x, residual, bias, alpha)
        raw, act = torch.empty_like(x), torch.empty_like(x)
        B, C, T, st = self._bct(x)
        kernels.check(self._lib.yapd_residual_bias_snake(x.data_ptr(), residual.data_ptr(), bias.data_ptr(),
                                                         alpha.data_ptr(), raw.data_ptr(), act.data_ptr(), B, C, T,
                                                         st))
        return [raw, act]

    def branch_start(self, x: torch.Tensor, source: torch.Tensor, alpha0: torch.Tensor, alpha1: torch.Tensor,
                     alpha2: torch.Tensor) -> List[torch.Tensor]:
        _need_bct(x)
        _need_bct(source)
        if x.shape != source.shape:
            raise RuntimeError("source shape mismatch")
        for i, a in enumerate((alpha0, alpha1, alpha2)):
            _need_channel(x, a, f"alpha{i} mismatch")
        _need_same(x, source, alpha0, alpha1, alpha2)
        outs = [torch.empty_like(x) for _ in range(4)]
        B, C, T, st = self._bct(x)
        kernels.check(self._lib.yapd_branch_start(x.data_ptr(), source.data_ptr(), alpha0.data_ptr(),
                                                  alpha1.data_ptr(), alpha2.data_ptr(),
                                                  *[o.data_ptr() for o in outs], B, C, T, st))
        return outs


@functools.lru_cache(maxsize=1)
def load_snake_extension() -> SnakeOps:
    """The native ops, loaded once (server/kernels.py:103-106)."""
    return SnakeOps()


# ---------------------------------------------------------------------------
# HiFT wiring (server/kernels.py:108-165)

def _alpha(snake: torch.nn.Module) -> torch.Tensor:
    """The Snake's effective per-channel alpha as a contiguous fp32 vector."""
    a = snake.alpha.detach()
    if getattr(snake, "alpha_logscale", False):
        a = torch.exp(a)
    return a.float().contiguous()


def _kernel_input(x: torch.Tensor) -> torch.Tensor:
    """The tensor the kernels take: a strided fp32 [B, C, T] CUDA tensor is copied
    to a contiguous one; any other dtype, device or rank raises.  There is no
    torch-expression path (the reference has one, server/kernels.py:110-112)."""
    if not (x.is_cuda and x.dtype == torch.float32 and x.dim() == 3):
        raise RuntimeError("contiguous fp32 CUDA BCT required")
    return x if x.is_contiguous() else x.contiguous()


def _fused_snake_forward(snake: torch.nn.Module, x: torch.Tensor) -> torch.Tensor:
    x = _kernel_input(x)
    ops = load_snake_extension()
    bias = getattr(snake, "pre_bias", None)
    if bias is None:
        return ops.snake(x, _alpha(snake))
    return ops.snake_bias(x, _alpha(snake), bias.detach().float().contiguous())


def _residual_bias(block: torch.nn.Module, i: int, like: torch.Tensor) -> torch.Tensor:
    b = getattr(block, f"residual_bias_{i}", None)
    if b is None:  # a bias-free conv: add zeros
        return torch.zeros(like.size(1), dtype=torch.float32, device=like.device)
    return b.detach().float().contiguous()


def _fused_resblock_forward(block: torch.nn.Module, x: torch.Tensor) -> torch.Tensor:
    """HiFT ResBlock with the fused ops (server/kernels.py:114-121): the
    residual add, its bias and the next pair's first Snake are one kernel."""
    n = len(block.convs1)
    pre = None  # the next pair's first activation, when already computed
    for i in range(n):
        y = block.activations1[i](x) if pre is None else pre
        y = block.convs1[i](y)
        y = block.activations2[i](y)
        y = block.convs2[i](y)
        bias = _residual_bias(block, i, y)
        y, x = _kernel_input(y), _kernel_input(x)
        ops = load_snake_extension()
        if i + 1 < n:
            x, pre = ops.residual_bias_snake(y, x, bias, _alpha(block.activations1[i + 1]))
        else:
            x, pre = ops.residual_bias(y, x, bias), None
    return x


def _fused_hift_decode(gen: torch.nn.Module, x: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    """HiFTGenerator.decode with the resblock mean as one kernel
    (server/kernels.py:125-152)."""
    s_real, s_imag = gen._stft(s.squeeze(1))
    s_stft = torch.cat([s_real, s_imag], dim=1)
    x = gen.conv_pre(x)
    nk = gen.num_kernels
    for i in range(gen.num_upsamples):
        x = F.leaky_relu(x, gen.lrelu_slope)
        x = gen.ups[i](x)
        if i == gen.num_upsamples - 1:
            x = gen.reflection_pad(x)
        x = x + gen.source_resblocks[i](gen.source_downs[i](s_stft))
        outs = [_kernel_input(gen.resblocks[i * nk + j](x)) for j in range(nk)]
        x = load_snake_extension().mean3(*outs)
    x = gen.conv_post(F.leaky_relu(x))
    split = gen.istft_params["n_fft"] // 2 + 1
    wav = gen._istft(torch.exp(x[:, :split, :]), torch.sin(x[:, split:, :]))
    return torch.clamp(wav, -gen.audio_limit, gen.audio_limit)


def install_fused_snake(module: torch.nn.Module) -> int:
    """Route a HiFT generator's Snake / resblock / decode through the fused
    kernels (server/kernels.py:154-165); returns the number of Snake modules."""
    load_snake_extension()  # fail before the module is touched
    if type(module).__name__ == "HiFTGenerator" and getattr(module, "num_kernels", 3) != 3:
        # the fused decode averages the resblock branches with mean3
        raise ValueError(f"install_fused_snake: HiFT decode needs 3 resblock kernels, got {module.num_kernels}")
    for block in [m for m in module.modules() if type(m).__name__ == "ResBlock"]:
        for i, (c1, c2, a2) in enumerate(zip(block.convs1, block.convs2, block.activations2)):
            if c1.bias is not None:
                a2.pre_bias = c1.bias
                c1.bias = None
            if c2.bias is not None:
                setattr(block, f"residual_bias_{i}", c2.bias)
                c2.bias = None
        block.forward = MethodType(_fused_resblock_forward, block)
    if type(module).__name__ == "HiFTGenerator":
        module.decode = MethodType(_fused_hift_decode, module)
    n = 0
    for m in module.modules():
        if type(m).__name__ == "Snake":
            m.forward = MethodType(_fused_snake_forward, m)
            n += 1
    return n
