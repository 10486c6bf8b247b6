"""GPU numerics of the affine-quantised projection (d) against
dequantise-then-matmul in fp32 (the oracle's MLX-formula dequantiser)."""

import numpy as np
import pytest
import torch

from oracle import quant as Q
from yapd_amd.quant import QuantLinear, dequant_affine, qgemm_affine, quantize_affine

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bits", [4, 8])
# (16384, 1000, 1024): the large-M kernel with a partial last column tile; (1024, 1000, 64) and
# (512, 200, 128): the direct-load 128 x 128 kernel with one and two k-tiles and partial tiles
@pytest.mark.parametrize("M,N,K", [(256, 3072, 1024), (8192, 1024, 4096), (37, 200, 128), (16384, 1000, 1024),
                                   (1024, 1000, 64), (512, 200, 128)])
def test_qgemm_vs_fp32_dequant(dev, bits, M, N, K):
    g = torch.Generator().manual_seed(M + N + bits)
    w = torch.randn(N, K, generator=g) * 0.02
    a = torch.randn(M, K, generator=g).bfloat16()
    packed, s, b = quantize_affine(w.to(dev), bits)
    out = qgemm_affine(a.to(dev), packed, s, b, bits)
    w_hat = torch.from_numpy(Q.dequantize(packed.cpu().numpy().view(np.uint32), s.cpu().numpy(),
                                          b.cpu().numpy(), bits))
    ref = a.float() @ w_hat.T
    rel = ((out.float().cpu() - ref).abs().max() / ref.abs().max()).item()
    assert rel <= 1e-2, rel


def test_quant_linear_module(dev):
    g = torch.Generator().manual_seed(7)
    w = (torch.randn(1024, 1024, generator=g) * 0.02).to(dev)
    ql = QuantLinear(w, 8)
    x = torch.randn(4, 64, 1024, generator=g).bfloat16().to(dev)
    y = ql(x)
    assert y.shape == (4, 64, 1024)
    rel = ((y.float() - x.float() @ w.T).abs().max() / (x.float() @ w.T).abs().max()).item()
    assert rel <= 2e-2  # 8-bit codes: quantisation error of W itself


@pytest.mark.parametrize("bits", [4, 8])
def test_quant_rows_do_not_depend_on_batch_size(dev, bits):
    """Every row of a quantised projection is bit-identical whichever of the three kernels computes
    it -- direct-load 256 x 256 tiles (M = 16384), register-staged 128 x 128 tiles (M = 8192: two
    tiles per CU), direct-load 128 x 128 tiles (M = 1024 and 96: at most one tile per CU, 4-bit
    codes read as 8-byte chunks) -- since all dequantise W the same way and take the same MFMA
    over K in the same order."""
    N, K = 1000, 4096  # a partial last column tile
    g = torch.Generator().manual_seed(50 + bits)
    w = torch.randn(N, K, generator=g) * 0.02
    A = torch.randn(16384, K, generator=g).bfloat16().to(dev)
    packed, s, b = quantize_affine(w.to(dev), bits)
    outs = [qgemm_affine(A[:M], packed, s, b, bits).cpu() for M in (16384, 8192, 1024, 96)]
    for M, out in zip((8192, 1024, 96), outs[1:]):
        assert torch.equal(outs[0][:M], out), M


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("N,K", [(3072, 1024), (1024, 1024), (8192, 1024), (1024, 4096)])
def test_c5_projection_shapes_at_m8192(dev, bits, N, K):
    """The benched quantised projections -- QKV, o_proj, gate/up and down of the
    T3 layer at M = 256 x 32 tokens -- against dequantise-then-matmul in fp32."""
    M = 8192
    g = torch.Generator(device=dev).manual_seed(N + K + bits)
    w = torch.randn(N, K, generator=g, device=dev) * 0.02
    a = torch.randn(M, K, generator=g, device=dev).bfloat16()
    packed, s, b = quantize_affine(w, bits)
    out = qgemm_affine(a, packed, s, b, bits)
    w_hat = torch.from_numpy(Q.dequantize(packed.cpu().numpy().view(np.uint32), s.cpu().numpy(),
                                          b.cpu().numpy(), bits)).to(dev)
    ref = a.float() @ w_hat.T
    rel = ((out.float() - ref).abs().max() / ref.abs().max()).item()
    assert rel <= 1e-2, rel


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("N,K", [(3072, 1024), (1000, 4096), (64, 64)])
def test_dequant_affine_matches_the_oracle_bit_for_bit(dev, bits, N, K):
    """``yapd_dequant_affine`` = bf16(fp32(scale * q + bias)): the codes unpacked by the oracle, the
    product and sum exact in float64 and rounded once to fp32 (what the kernels' FMA does), then to
    bf16.  Scales and biases of mixed sign and magnitude, so a dropped rounding or a mul-then-add
    shows."""
    g = torch.Generator().manual_seed(N + K + bits)
    w = torch.randn(N, K, generator=g) * torch.logspace(-3, 0, K)[None, :] + torch.randn(N, 1, generator=g)
    packed, s, b = quantize_affine(w.to(dev), bits)
    out = dequant_affine(packed, s, b, bits)
    q = Q.unpack(packed.cpu().numpy().view(np.uint32), bits, K).astype(np.float64)
    s64 = np.repeat(s.cpu().numpy().astype(np.float64), 64, axis=1)
    b64 = np.repeat(b.cpu().numpy().astype(np.float64), 64, axis=1)
    ref = torch.from_numpy((s64 * q + b64).astype(np.float32)).bfloat16()
    assert torch.equal(out.cpu(), ref)


@pytest.mark.parametrize("bits", [4, 8])
# C5's four shapes at M = 8192, and a partial last column tile at M = 16384
@pytest.mark.parametrize("M,N,K", [(8192, 3072, 1024), (8192, 1024, 1024), (8192, 8192, 1024), (8192, 1024, 4096),
                                   (16384, 1000, 1024)])
def test_dequantise_once_route_equals_the_fused_kernel(dev, bits, M, N, K):
    """With a scratch buffer and at least DEQUANT_MIN_ROWS rows, ``qgemm_affine`` dequantises W once and
    runs the bf16 GEMM; the result equals the fused kernel's bit for bit (the same bf16 weights, the
    same MFMA over K in the same order)."""
    g = torch.Generator().manual_seed(M + N + K + bits)
    w = torch.randn(N, K, generator=g) * 0.02
    A = torch.randn(M, K, generator=g).bfloat16().to(dev)
    packed, s, b = quantize_affine(w.to(dev), bits)
    scratch = torch.empty(N * K + 64, dtype=torch.bfloat16, device=dev)
    fused = qgemm_affine(A, packed, s, b, bits)
    once = qgemm_affine(A, packed, s, b, bits, scratch=scratch)
    assert torch.equal(fused, once)
    assert torch.equal(scratch[: N * K].view(N, K), dequant_affine(packed, s, b, bits))
