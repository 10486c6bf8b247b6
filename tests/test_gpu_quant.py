"""GPU numerics of the affine-quantised projection (d) against
dequantise-then-matmul in fp32 (the oracle's MLX-formula dequantiser)."""

import numpy as np
import pytest
import torch

from oracle import quant as Q
from yapd_amd.quant import QuantLinear, qgemm_affine, quantize_affine

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bits", [4, 8])
# (16384, 1000, 1024): the large-M kernel with a partial last column tile
@pytest.mark.parametrize("M,N,K", [(256, 3072, 1024), (8192, 1024, 4096), (37, 200, 128), (16384, 1000, 1024)])
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
