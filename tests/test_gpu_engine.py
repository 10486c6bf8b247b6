"""End-to-end parity of ``HipEngine`` against the oracle's torch-SDPA
restatement (engines/torch_sdpa.py:145-341 semantics, per-row cache starts):
prefix prefill, block forward (eager and graph replay), token-shifted head.

Tolerances (hidden states and logits are checked against the fp32 oracle):
bf16 hidden states within max(2e-2, 1.5 x the bf16 oracle's own max-abs
error) -- bf16 arithmetic alone puts the reference's bf16 path about 0.024
away from fp32 on one layer (a bf16 ulp is 0.0156 in [2, 4)), so a flat
2e-2 would fail the reference itself; logits within max(1e-2, 1.5 x the bf16
oracle's) relative error (max-abs error / max-abs logit)."""

import numpy as np
import pytest
import torch

from oracle import llama as OL
from yapd_amd import kernels
from yapd_amd.engines.hip import HipEngine
from yapd_amd.synthetic import make_t3, uniform_lengths

pytestmark = pytest.mark.gpu


def oracle_backbones(model, max_pos):
    bb16 = OL.backbone_from_model(model, max_pos=max_pos, dtype=torch.bfloat16)
    bb32 = OL.backbone_from_model(model, max_pos=max_pos, dtype=torch.float32)
    return bb16, bb32


def max_abs(a, b):
    return (a.float().cpu() - b.float().cpu()).abs().max().item()


def hidden_ok(out, ref16, ref32, label):
    """GPU vs fp32 within max(2e-2, 1.5 x (bf16 oracle vs fp32))."""
    e_gpu, e_ref = max_abs(out, ref32), max_abs(ref16, ref32)
    print(f"{label}: max-abs vs fp32 oracle GPU {e_gpu:.4g}, bf16 oracle {e_ref:.4g}; GPU vs bf16 {max_abs(out, ref16):.4g}")
    return e_gpu <= max(2e-2, 1.5 * e_ref)


@pytest.fixture(scope="module")
def one_layer(dev):
    return make_t3(n_layers=1, seed=0, norm_jitter=True, device=dev)


def test_one_layer_prefix_and_block(dev):
    # Hidden 1024, 16x64 heads, FFN 4096, eps 1e-5, RoPE theta 10000; prefix of
    # 256 tokens (identity page table), block of 32 masked positions, N(0,1)
    # states, linear weights N(0, 0.02), norm gains 1.
    model = make_t3(n_layers=1, seed=0, device=dev)
    B, lp, bl = 1, 256, 32
    g = torch.Generator().manual_seed(0)
    prefix = torch.randn(B, lp, 1024, generator=g).bfloat16()
    block = torch.randn(B, bl, 1024, generator=g).bfloat16()
    eng = HipEngine(model, 512, torch.bfloat16, batch_size=B)
    sos = eng.prefix_forward(prefix.to(dev))
    hid = eng.block_forward(block.to(dev), lp)
    bb16, bb32 = oracle_backbones(model, 512)
    outs = {}
    for name, bb in (("bf16", bb16), ("fp32", bb32)):
        cache = OL.KVCache.empty(1, B, 512, 16, 64, bb.dtype)
        s = OL.prefix_forward(bb, [prefix[0]], cache)
        h = OL.block_forward(bb, block, cache, [lp])
        outs[name] = (s, h)
    assert hidden_ok(hid, outs["bf16"][1], outs["fp32"][1], "1-layer block hidden")
    assert hidden_ok(sos, outs["bf16"][0], outs["fp32"][0], "1-layer prefix SOS hidden")


def test_other_model_dims(dev):
    # hidden 512 (one 512-wide RMSNorm chunk), 8 heads (two four-head attention
    # workgroups, QKV N = 1536), FFN 1536; two ragged rows
    D, H, Fd = 512, 8, 1536
    model = make_t3(n_layers=1, hidden=D, heads=H, ffn=Fd, seed=4, norm_jitter=True, device=dev)
    B, bl, lps = 2, 16, [90, 200]
    g = torch.Generator().manual_seed(4)
    prefixes = [torch.randn(1, lp, D, generator=g).bfloat16() for lp in lps]
    block = torch.randn(B, bl, D, generator=g).bfloat16()
    eng = HipEngine(model, 512, torch.bfloat16, batch_size=B)
    sos = eng.prefix_forward([p.to(dev) for p in prefixes])
    hid = eng.block_forward(block.to(dev), lps)
    bb16, bb32 = oracle_backbones(model, 512)
    refs = {}
    for name, bb in (("bf16", bb16), ("fp32", bb32)):
        cache = OL.KVCache.empty(1, B, 512, H, 64, bb.dtype)
        s_ref = OL.prefix_forward(bb, [p[0].to(bb.dtype) for p in prefixes], cache)
        refs[name] = (s_ref, OL.block_forward(bb, block.to(bb.dtype), cache, lps))
    assert hidden_ok(sos, refs["bf16"][0], refs["fp32"][0], "512-wide SOS hidden")
    assert hidden_ok(hid, refs["bf16"][1], refs["fp32"][1], "512-wide block hidden")


def test_ragged_starts_shuffled_pages_graph_and_head(dev, one_layer):
    model = one_layer
    B, bl = 3, 32
    lps = [100, 177, 256]
    g = torch.Generator().manual_seed(1)
    prefixes = [torch.randn(1, lp, 1024, generator=g).bfloat16() for lp in lps]
    block = torch.randn(B, bl, 1024, generator=g).bfloat16()
    eng = HipEngine(model, 512, torch.bfloat16, batch_size=B, page_table_seed=7)
    sos = eng.prefix_forward([p.to(dev) for p in prefixes])
    assert eng.cache_lens == lps
    hid = eng.block_forward(block.to(dev), lps)
    bb16, bb32 = oracle_backbones(model, 512)
    refs = {}
    for name, bb in (("bf16", bb16), ("fp32", bb32)):
        cache = OL.KVCache.empty(1, B, 512, 16, 64, bb.dtype)
        s_ref = OL.prefix_forward(bb, [p[0].to(bb.dtype) for p in prefixes], cache)
        refs[name] = (s_ref, OL.block_forward(bb, block.to(bb.dtype), cache, lps))
    assert hidden_ok(sos, refs["bf16"][0], refs["fp32"][0], "ragged SOS hidden")
    assert hidden_ok(hid, refs["bf16"][1], refs["fp32"][1], "ragged block hidden")
    # graph replay == eager, logits vs the oracle's shifted head
    eng.capture_cuda_graph(bl, speech_head=model.speech_head)
    eng.set_shift_ctx(sos)
    hid_g, logits = eng.block_forward_graph(block.to(dev), lps)
    assert torch.equal(hid_g.cpu(), hid.cpu())
    lg_ref = OL.speech_head_shift(hid.float().cpu(), sos.float().cpu(), model.speech_head.weight.float().cpu())
    rel = max_abs(logits, lg_ref) / lg_ref.abs().max().item()
    assert rel <= 1e-2  # same hidden in, fp32 head: only the bf16 GEMM output rounding
    # a second replay at the next block start re-plans in place
    lps2 = [x + bl for x in lps]
    eng.advance_cache(bl)
    hid_g2, _ = eng.block_forward_graph(block.to(dev), lps2)
    hid_e2 = eng.block_forward(block.to(dev), lps2)
    assert torch.equal(hid_g2.cpu(), hid_e2.cpu())


@pytest.mark.parametrize("lps", [[100, 177, 256], [100, 1100, 1300]])  # rows > 1024 keys are split
def test_graph_replay_with_and_without_split_rows(dev, one_layer, lps):
    """The engine captures its step with and without the split-KV merge launch
    and replays the one the current plan needs; both equal the eager path."""
    model = one_layer
    B, bl = 3, 32
    g = torch.Generator().manual_seed(2)
    prefixes = [torch.randn(1, lp, 1024, generator=g).bfloat16().to(dev) for lp in lps]
    block = torch.randn(B, bl, 1024, generator=g).bfloat16().to(dev)
    eng = HipEngine(model, 2048, torch.bfloat16, batch_size=B)
    sos = eng.prefix_forward(prefixes)
    hid = eng.block_forward(block, lps).cpu()
    eng.capture_cuda_graph(bl, speech_head=model.speech_head)
    eng.set_shift_ctx(sos)
    hid_g, _ = eng.block_forward_graph(block, lps)
    assert (eng._g_plan.n_merge_live > 0) == (max(lps) + bl > 1024)
    assert torch.equal(hid_g.cpu(), hid)
    for rep in range(2):  # more replays, with the eager forward (the program's own work) between them
        assert torch.equal(eng.block_forward(block, lps).cpu(), hid), rep
        torch.cuda.synchronize()
        hid_g, _ = eng.block_forward_graph(block, lps)
        assert torch.equal(hid_g.cpu(), hid), rep


def test_thirty_layers_block_step(dev):
    # 30 layers, 16 CFG pairs = 32 rows, prefixes U[150, 600] (pairs share a
    # length), shuffled page table, block 32, speech head V = 8194.
    model = make_t3(n_layers=30, seed=1, device=dev)
    pairs, bl = 16, 32
    lens = uniform_lengths(pairs, 150, 600, seed=2)
    lps = [L for L in lens for _ in range(2)]
    B = 2 * pairs
    eng = HipEngine(model, 700, torch.bfloat16, batch_size=B, page_table_seed=3)
    bb16, bb32 = oracle_backbones(model, 700)
    c16 = OL.KVCache.empty(30, B, 700, 16, 64, torch.bfloat16)
    c32 = OL.KVCache.empty(30, B, 700, 16, 64, torch.float32)
    gd = torch.Generator().manual_seed(4)
    tab = eng.kv.table
    for li in range(30):
        for r in range(B):
            k = torch.randn(lps[r], 16, 64, generator=gd).bfloat16()
            v = torch.randn(lps[r], 16, 64, generator=gd).bfloat16()
            c16.k[li][r][: lps[r]] = k
            c16.v[li][r][: lps[r]] = v
            c32.k[li][r][: lps[r]] = k.float()
            c32.v[li][r][: lps[r]] = v.float()
            kernels.kv_write(k.to(dev), v.to(dev), eng.kv.pools[li], tab[r: r + 1],
                             torch.zeros(1, dtype=torch.int32, device=dev), lps[r])
    eng.cache_len = 0
    eng._cache_lens = list(lps)
    block = torch.randn(B, bl, 1024, generator=gd).bfloat16()
    ctx = torch.randn(B, 1, 1024, generator=gd).bfloat16()
    eng.capture_cuda_graph(bl, speech_head=model.speech_head)
    eng.set_shift_ctx(ctx.to(dev))
    hid, logits = eng.block_forward_graph(block.to(dev), lps)
    h16 = OL.block_forward(bb16, block, c16, lps)
    h32 = OL.block_forward(bb32, block.float(), c32, lps)
    e_gpu, e_ref = max_abs(hid, h32), max_abs(h16, h32)
    print(f"30-layer: hidden max-abs GPU-vs-fp32 {e_gpu:.4g}, bf16-oracle-vs-fp32 {e_ref:.4g}, "
          f"GPU-vs-bf16 {max_abs(hid, h16):.4g}")
    assert e_gpu <= max(2e-2, 1.5 * e_ref)
    W = model.speech_head.weight.float().cpu()
    lg32 = OL.speech_head_shift(h32, ctx.float(), W)
    rel = max_abs(logits, lg32) / lg32.abs().max().item()
    rel_ref = max_abs(OL.speech_head_shift(h16.float(), ctx.float(), W), lg32) / lg32.abs().max().item()
    print(f"30-layer: logits rel err GPU {rel:.4g}, bf16 oracle {rel_ref:.4g}")
    assert rel <= max(1e-2, 1.5 * rel_ref)


def test_engine_rejects_bad_inputs(dev, one_layer):
    with pytest.raises(ValueError):
        HipEngine(one_layer, 512, torch.float16)
    eng = HipEngine(one_layer, 128, torch.bfloat16, batch_size=2)
    with pytest.raises(ValueError):
        eng.block_forward(torch.zeros(3, 16, 1024, dtype=torch.bfloat16, device=dev), 0)
    with pytest.raises(ValueError):
        eng.block_forward(torch.zeros(2, 16, 1024, dtype=torch.bfloat16, device=dev), 120)
    assert eng.can_reuse(100, torch.bfloat16, batch_size=2) and not eng.can_reuse(200, torch.bfloat16, batch_size=2)


def test_recapture_at_another_block_size_keeps_the_prefix(dev, one_layer):
    """capture_cuda_graph at bl = 16, then at bl = 32 with unchanged cache
    starts: the second graph must be re-planned for the new block size (its
    keys cover the prefix), so its replay equals the eager block forward."""
    model = one_layer
    B, lps = 2, [100, 140]
    g = torch.Generator().manual_seed(6)
    prefixes = [torch.randn(1, lp, 1024, generator=g).bfloat16().to(dev) for lp in lps]
    eng = HipEngine(model, 512, torch.bfloat16, batch_size=B)
    sos = eng.prefix_forward(prefixes)
    for bl in (16, 32):
        block = torch.randn(B, bl, 1024, generator=g).bfloat16().to(dev)
        eng.capture_cuda_graph(bl, speech_head=model.speech_head)
        eng.set_shift_ctx(sos)
        assert eng._g_plan.kv_len.tolist() == [lp + bl for lp in lps]
        hid_g, _ = eng.block_forward_graph(block, lps)
        hid_g = hid_g.clone()
        hid_e = eng.block_forward(block, lps)
        assert torch.equal(hid_g, hid_e), f"bl={bl}"
