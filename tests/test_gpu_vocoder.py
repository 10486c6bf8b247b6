"""GPU parity of the HiFT vocoder's elementwise family (server/kernels.py:35-67)
against oracle.vocoder, the reference's operator API and error behaviour
(server/kernels.py:69-100), and install_fused_snake on a HiFT-shaped
generator against its own torch forward (server/kernels.py:108-165).

Tolerances: the adds and mean3 are bit-exact (float32, the reference's
order); Snake is compared with the float64 value of the activation and may
differ by sinf's error (<= 2 ulp of |sin| <= 1, so <= 2.4e-7 per sin, scaled
by 2 |sin| / (a + 1e-9) through the square) plus the rounding of the product
and the sum."""

import math

import numpy as np
import pytest
import torch
import torch.nn as nn

from oracle import vocoder as OV
from yapd_amd.vocoder import install_fused_snake, load_snake_extension

pytestmark = pytest.mark.gpu


def bct(dev, shape, g, scale=2.0, offset=0):
    """A contiguous fp32 tensor on `dev`; a storage offset of 1 float makes it only 4-byte aligned."""
    n = math.prod(shape)
    buf = torch.empty(n + offset, dtype=torch.float32, device=dev)
    t = buf[offset:].view(*shape)
    t.copy_(torch.randn(*shape, generator=g) * scale)
    return t


def chan(dev, C, g, lo=0.2, hi=3.0):
    return (torch.rand(C, generator=g) * (hi - lo) + lo).to(dev)


def assert_snake(got, ref64, alpha):
    ref = torch.from_numpy(np.asarray(ref64))
    got = got.cpu().double()
    inv = 1.0 / (alpha.cpu().double() + 1e-9)[None, :, None]
    ulp = torch.from_numpy(np.spacing(np.abs(ref.numpy()).astype(np.float32)).astype(np.float64))
    bound = 6e-7 * inv + 2 * ulp
    err = (got - ref).abs()
    assert bool((err <= bound).all()), f"max err {err.max().item():.3e}, worst excess {(err - bound).max().item():.3e}"


SHAPES = [(2, 5, 37, 0), (3, 64, 1280, 0), (1, 3, 4100, 0), (2, 4, 1024, 1), (2, 3, 6401, 0)]


@pytest.mark.parametrize("B,C,T,off", SHAPES)
def test_snake_and_snake_bias(dev, B, C, T, off):
    g = torch.Generator().manual_seed(B * 7 + T)
    x = bct(dev, (B, C, T), g, offset=off)
    a, b = chan(dev, C, g), chan(dev, C, g, -1.0, 1.0)
    ops = load_snake_extension()
    assert_snake(ops.snake(x, a), OV.snake(x.cpu().numpy(), a.cpu().numpy()), a)
    assert_snake(ops.snake_bias(x, a, b), OV.snake(x.cpu().numpy(), a.cpu().numpy(), b.cpu().numpy()), a)


@pytest.mark.parametrize("B,C,T,off", SHAPES)
def test_residual_ops(dev, B, C, T, off):
    g = torch.Generator().manual_seed(B * 11 + T)
    x, r = bct(dev, (B, C, T), g, offset=off), bct(dev, (B, C, T), g, offset=off)
    a, b = chan(dev, C, g), chan(dev, C, g, -1.0, 1.0)
    ops = load_snake_extension()
    xn, rn, an, bn = (t.cpu().numpy() for t in (x, r, a, b))
    out = ops.residual_bias(x, r, b)
    assert torch.equal(out.cpu(), torch.from_numpy(OV.residual_bias(xn, rn, bn)))
    raw, act = ops.residual_bias_snake(x, r, b, a)
    raw_ref, act_ref = OV.residual_bias_snake(xn, rn, bn, an)
    assert torch.equal(raw.cpu(), torch.from_numpy(raw_ref))
    assert_snake(act, act_ref, a)


@pytest.mark.parametrize("B,C,T,off", SHAPES)
def test_mean3_and_branch_start(dev, B, C, T, off):
    g = torch.Generator().manual_seed(B * 13 + T)
    t3 = [bct(dev, (B, C, T), g, offset=off) for _ in range(3)]
    ops = load_snake_extension()
    m = ops.mean3(*t3)
    assert torch.equal(m.cpu(), torch.from_numpy(OV.mean3(*(t.cpu().numpy() for t in t3))))
    src = bct(dev, (B, C, T), g, offset=off)
    al = [chan(dev, C, g) for _ in range(3)]
    outs = ops.branch_start(t3[0], src, *al)
    refs = OV.branch_start(t3[0].cpu().numpy(), src.cpu().numpy(), *(a.cpu().numpy() for a in al))
    assert torch.equal(outs[0].cpu(), torch.from_numpy(refs[0]))
    for o, ref, a in zip(outs[1:], refs[1:], al):
        assert_snake(o, ref, a)


def test_reference_error_messages(dev):
    ops = load_snake_extension()
    g = torch.Generator().manual_seed(0)
    x = bct(dev, (2, 4, 16), g)
    a = chan(dev, 4, g)
    with pytest.raises(RuntimeError, match="contiguous fp32 CUDA BCT required"):
        ops.snake(x.half(), a)
    with pytest.raises(RuntimeError, match="contiguous fp32 CUDA BCT required"):
        ops.snake(x.transpose(1, 2), a)
    with pytest.raises(RuntimeError, match="contiguous fp32 CUDA BCT required"):
        ops.snake(x.cpu(), a)
    with pytest.raises(RuntimeError, match="alpha mismatch"):
        ops.snake(x, chan(dev, 5, g))
    with pytest.raises(RuntimeError, match="bias mismatch"):
        ops.snake_bias(x, a, chan(dev, 3, g))
    with pytest.raises(RuntimeError, match="residual shape mismatch"):
        ops.residual_bias(x, bct(dev, (2, 4, 8), g), a)
    with pytest.raises(RuntimeError, match="mean3 shape mismatch"):
        ops.mean3(x, x, bct(dev, (2, 4, 8), g))
    with pytest.raises(RuntimeError, match="source shape mismatch"):
        ops.branch_start(x, bct(dev, (1, 4, 16), g), a, a, a)
    with pytest.raises(RuntimeError, match="alpha1 mismatch"):
        ops.branch_start(x, x, a, chan(dev, 2, g), a)


# ---------------------------------------------------------------------------
# A HiFT-shaped generator (the S3Gen HiFTGenerator's module names and decode
# chain, small sizes) whose unpatched forward is plain torch.

class Snake(nn.Module):
    def __init__(self, ch, g, alpha_logscale=False):
        super().__init__()
        a = torch.rand(ch, generator=g) * 2.0 + 0.3
        self.alpha_logscale = alpha_logscale
        self.alpha = nn.Parameter(torch.log(a) if alpha_logscale else a)
        self.no_div_by_zero = 1e-9

    def forward(self, x):
        a = self.alpha.unsqueeze(0).unsqueeze(-1)
        if self.alpha_logscale:
            a = torch.exp(a)
        return x + (1.0 / (a + self.no_div_by_zero)) * torch.sin(x * a) ** 2


class ResBlock(nn.Module):
    def __init__(self, ch, k, g, dilations=(1, 3, 5)):
        super().__init__()
        self.convs1 = nn.ModuleList([nn.Conv1d(ch, ch, k, dilation=d, padding=(k * d - d) // 2) for d in dilations])
        self.convs2 = nn.ModuleList([nn.Conv1d(ch, ch, k, padding=(k - 1) // 2) for _ in dilations])
        self.activations1 = nn.ModuleList([Snake(ch, g) for _ in dilations])
        self.activations2 = nn.ModuleList([Snake(ch, g) for _ in dilations])

    def forward(self, x):
        for c1, c2, a1, a2 in zip(self.convs1, self.convs2, self.activations1, self.activations2):
            x = c2(a2(c1(a1(x)))) + x
        return x


class HiFTGenerator(nn.Module):
    def __init__(self, g):
        super().__init__()
        self.istft_params = {"n_fft": 16, "hop_len": 4}
        self.num_kernels, self.num_upsamples, self.lrelu_slope, self.audio_limit = 3, 2, 0.1, 0.99
        self.conv_pre = nn.Conv1d(80, 64, 7, padding=3)
        self.ups = nn.ModuleList([nn.ConvTranspose1d(64, 32, 8, 4, padding=2), nn.ConvTranspose1d(32, 16, 4, 2, padding=1)])
        self.reflection_pad = nn.ReflectionPad1d((1, 0))
        self.resblocks = nn.ModuleList([ResBlock(ch, k, g) for ch in (32, 16) for k in (3, 7, 11)])
        self.source_downs = nn.ModuleList([nn.Conv1d(18, 32, 4, 2, padding=1), nn.Conv1d(18, 16, 1)])
        self.source_resblocks = nn.ModuleList([ResBlock(32, 7, g), ResBlock(16, 11, g)])
        self.conv_post = nn.Conv1d(16, 18, 7, padding=3)
        self.register_buffer("window", torch.hann_window(16), persistent=False)

    def _stft(self, x):
        spec = torch.stft(x, 16, 4, 16, window=self.window, return_complex=True)
        return spec.real, spec.imag

    def _istft(self, mag, phase):
        return torch.istft(torch.complex(mag * torch.cos(phase), mag * torch.sin(phase)), 16, 4, 16,
                           window=self.window)

    def decode(self, x, s):
        s_real, s_imag = self._stft(s.squeeze(1))
        s_stft = torch.cat([s_real, s_imag], dim=1)
        x = self.conv_pre(x)
        for i in range(self.num_upsamples):
            x = self.ups[i](nn.functional.leaky_relu(x, self.lrelu_slope))
            if i == self.num_upsamples - 1:
                x = self.reflection_pad(x)
            x = x + self.source_resblocks[i](self.source_downs[i](s_stft))
            x = sum(self.resblocks[i * 3 + j](x) for j in range(3)) / 3
        x = self.conv_post(nn.functional.leaky_relu(x))
        wav = self._istft(torch.exp(x[:, :9, :]), torch.sin(x[:, 9:, :]))
        return torch.clamp(wav, -self.audio_limit, self.audio_limit)


@torch.inference_mode()
def test_install_fused_snake_matches_the_torch_generator(dev):
    g = torch.Generator().manual_seed(5)
    gen = HiFTGenerator(g)
    for p in gen.parameters():  # audible-scale weights (conv default init keeps activations O(1))
        p.data.mul_(0.5)
    gen = gen.to(dev).eval()
    B, Tm = 3, 20  # stage lengths 80 (16-byte path) and 161 (scalar path)
    x = (torch.randn(B, 80, Tm, generator=g) * 0.5).to(dev)
    s = (torch.randn(B, 1, 32 * Tm, generator=g) * 0.1).to(dev)
    ref = gen.decode(x, s)
    n = install_fused_snake(gen)
    assert n == 8 * 3 * 2  # 8 resblocks x 3 dilations x 2 activations
    assert gen.resblocks[0].convs1[0].bias is None and gen.resblocks[0].activations2[0].pre_bias is not None
    out = gen.decode(x, s)
    assert out.shape == ref.shape
    torch.testing.assert_close(out, ref, rtol=1e-4, atol=2e-5)


@torch.inference_mode()
def test_fused_snake_module_paths(dev):
    g = torch.Generator().manual_seed(6)
    holder = nn.Module()
    holder.a = Snake(8, g, alpha_logscale=True)
    holder.b = Snake(8, g)
    holder = holder.to(dev)
    x = (torch.randn(2, 8, 64, generator=g) * 2).to(dev)
    want_a, want_b = holder.a(x), holder.b(x)
    want_t = holder.b(x.transpose(1, 2).contiguous().transpose(1, 2))
    assert install_fused_snake(holder) == 2
    torch.testing.assert_close(holder.a(x), want_a, rtol=1e-5, atol=1e-5)  # log-scale alpha through the kernel
    torch.testing.assert_close(holder.b(x), want_b, rtol=1e-5, atol=1e-5)
    # a strided input is copied to a contiguous one and runs the same kernel
    # (there is no torch-expression path)
    xt = x.transpose(1, 2).contiguous().transpose(1, 2)
    assert not xt.is_contiguous()
    assert torch.equal(holder.b(xt), holder.b(xt.contiguous()))
    torch.testing.assert_close(holder.b(xt), want_t, rtol=1e-5, atol=1e-5)
    # inputs the kernels cannot take raise instead of falling back to torch
    with pytest.raises(RuntimeError, match="contiguous fp32 CUDA BCT required"):
        holder.b(x.double())
    with pytest.raises(RuntimeError, match="contiguous fp32 CUDA BCT required"):
        holder.b(x.cpu())
    with pytest.raises(RuntimeError, match="contiguous fp32 CUDA BCT required"):
        holder.b(x[0])
