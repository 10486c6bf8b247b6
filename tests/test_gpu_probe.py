"""The measurement harness's calibration kernels: the streaming-read probe
reads every 16-byte word exactly once (each thread's XOR fold equals the fold
of the words its grid-stride walk covers) and the MFMA probe runs."""

import numpy as np
import pytest
import torch

from yapd_amd import kernels

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n16,blocks", [(5000, 2), (1 << 16, 16), (3, 1)])
def test_read_probe_covers_every_word_once(dev, n16, blocks):
    rng = np.random.default_rng(n16)
    words = rng.integers(0, 2 ** 32, size=(n16, 4), dtype=np.uint64).astype(np.uint32)
    src = torch.from_numpy(words.view(np.int32)).to(dev)
    out = torch.full((blocks * 256,), -1, dtype=torch.int32, device=dev)
    assert kernels.hbm_read_probe(src, blocks, out) == n16 * 16
    torch.cuda.synchronize()
    per = (-(-n16 // blocks) + 255) // 256 * 256  # each workgroup's contiguous share, in words
    folded = np.bitwise_xor.reduce(words, axis=1)  # the four lanes of a word
    want = np.zeros(blocks * 256, dtype=np.uint32)
    for b in range(blocks):
        share = folded[b * per:min(n16, (b + 1) * per)]
        for t in range(min(256, len(share))):
            want[b * 256 + t] = np.bitwise_xor.reduce(share[t::256])
    np.testing.assert_array_equal(out.cpu().numpy().view(np.uint32), want)


def test_mfma_probe_runs(dev):
    out = torch.empty(4 * 256, dtype=torch.float32, device=dev)
    assert kernels.mfma_peak_probe(4, 10, out) == 4 * 4 * 10 * 8 * 32768
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
