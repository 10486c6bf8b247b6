"""Pins the backbone oracle against ``transformers.LlamaModel`` driven the way
engines/torch_sdpa.py drives it: causal prefix with a DynamicCache, then the
block with position ids ``cs..cs+bl`` and a zero additive mask over
``[0, cs+bl)`` (torch_sdpa.py:299-307, 324-341)."""

from types import SimpleNamespace

import pytest
import torch
from transformers import DynamicCache, LlamaConfig, LlamaModel

from oracle import llama as O


def tiny_model(dtype=torch.float32, rope=None, layers=2, seed=0):
    torch.manual_seed(seed)
    kw = dict(hidden_size=64, intermediate_size=128, num_hidden_layers=layers, num_attention_heads=4,
              num_key_value_heads=4, head_dim=16, rms_norm_eps=1e-5, vocab_size=8,
              max_position_embeddings=4096, attn_implementation="sdpa")
    if rope is None:
        kw["rope_theta"] = 10000.0
    else:
        kw["rope_parameters"] = rope
    m = LlamaModel(LlamaConfig(**kw)).eval()
    with torch.no_grad():
        for lyr in m.layers:  # non-trivial norm gains so the weight multiply is exercised
            lyr.input_layernorm.weight.uniform_(0.5, 1.5)
            lyr.post_attention_layernorm.weight.uniform_(0.5, 1.5)
        m.norm.weight.uniform_(0.5, 1.5)
    return m.to(dtype)


def hf_prefix_then_block(m, prefix, block, cs):
    B, lp, _ = prefix.shape
    bl = block.shape[1]
    cache = DynamicCache()
    out = m(inputs_embeds=prefix, position_ids=torch.arange(lp).expand(B, -1), past_key_values=cache,
            use_cache=True)
    cache = out.past_key_values
    cache.crop(cs)
    mask = torch.zeros(1, 1, bl, cs + bl, dtype=prefix.dtype)
    out2 = m(inputs_embeds=block, position_ids=torch.arange(cs, cs + bl).expand(B, -1),
             past_key_values=cache, attention_mask=mask, use_cache=True)
    return out.last_hidden_state, out2.last_hidden_state


@pytest.mark.parametrize("rope", [None, {"rope_type": "llama3", "rope_theta": 500000.0, "factor": 8.0,
                                         "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                                         "original_max_position_embeddings": 8192}])
def test_uniform_prefix_and_block_fp32(rope):
    m = tiny_model(rope=rope)
    g = torch.Generator().manual_seed(1)
    B, lp, bl = 3, 37, 16
    prefix = torch.randn(B, lp, 64, generator=g)
    block = torch.randn(B, bl, 64, generator=g)
    with torch.no_grad():
        pre_hf, blk_hf = hf_prefix_then_block(m, prefix, block, lp)
        bb = O.backbone_from_model(SimpleNamespace(tfmr=m), max_pos=512)
        cache = O.KVCache.empty(len(bb.layers), B, 512, 4, 16, torch.float32)
        sos = O.prefix_forward(bb, [prefix[b] for b in range(B)], cache)
        hid = O.block_forward(bb, block, cache, [lp] * B)
    torch.testing.assert_close(sos[:, 0], pre_hf[:, lp - 1], rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(hid, blk_hf, rtol=1e-5, atol=1e-5)


def test_ragged_rows_match_per_row_hf():
    m = tiny_model()
    g = torch.Generator().manual_seed(2)
    lps = [20, 33, 47]
    bl = 8
    prefixes = [torch.randn(lp, 64, generator=g) for lp in lps]
    block = torch.randn(len(lps), bl, 64, generator=g)
    with torch.no_grad():
        bb = O.backbone_from_model(SimpleNamespace(tfmr=m), max_pos=256)
        cache = O.KVCache.empty(len(bb.layers), len(lps), 256, 4, 16, torch.float32)
        sos = O.prefix_forward(bb, prefixes, cache)
        hid = O.block_forward(bb, block, cache, lps)
        for r, lp in enumerate(lps):
            pre_hf, blk_hf = hf_prefix_then_block(m, prefixes[r][None], block[r: r + 1], lp)
            torch.testing.assert_close(sos[r, 0], pre_hf[0, lp - 1], rtol=1e-5, atol=1e-5)
            torch.testing.assert_close(hid[r], blk_hf[0], rtol=1e-5, atol=1e-5)


def test_tentative_rewrite_then_next_block():
    # Denoise steps rewrite the block KV at the same cache start; a commit
    # forward then the next block at cs+bl sees the committed tokens.
    m = tiny_model()
    g = torch.Generator().manual_seed(3)
    B, lp, bl = 2, 21, 8
    prefix = torch.randn(B, lp, 64, generator=g)
    b1a, b1b, b2 = (torch.randn(B, bl, 64, generator=g) for _ in range(3))
    with torch.no_grad():
        bb = O.backbone_from_model(SimpleNamespace(tfmr=m), max_pos=128)
        cache = O.KVCache.empty(len(bb.layers), B, 128, 4, 16, torch.float32)
        O.prefix_forward(bb, [prefix[b] for b in range(B)], cache)
        O.block_forward(bb, b1a, cache, [lp] * B)           # tentative step
        O.block_forward(bb, b1b, cache, [lp] * B)           # commit of the final tokens
        hid2 = O.block_forward(bb, b2, cache, [lp + bl] * B)
        # HF: one prefill over prefix + committed block is NOT the same (the block
        # is bidirectional), so build the HF cache the engine way.
        hc = DynamicCache()
        out = m(inputs_embeds=prefix, position_ids=torch.arange(lp).expand(B, -1), past_key_values=hc,
                use_cache=True)
        hc = out.past_key_values
        z = lambda n: torch.zeros(1, 1, bl, n)
        out = m(inputs_embeds=b1b, position_ids=torch.arange(lp, lp + bl).expand(B, -1),
                past_key_values=hc, attention_mask=z(lp + bl), use_cache=True)
        hc = out.past_key_values
        out = m(inputs_embeds=b2, position_ids=torch.arange(lp + bl, lp + 2 * bl).expand(B, -1),
                past_key_values=hc, attention_mask=z(lp + 2 * bl), use_cache=True)
    torch.testing.assert_close(hid2, out.last_hidden_state, rtol=1e-5, atol=1e-5)


def test_bf16_tracks_hf_bf16():
    m = tiny_model(dtype=torch.bfloat16)
    g = torch.Generator().manual_seed(4)
    B, lp, bl = 2, 30, 16
    prefix = torch.randn(B, lp, 64, generator=g).bfloat16()
    block = torch.randn(B, bl, 64, generator=g).bfloat16()
    with torch.no_grad():
        _, blk_hf = hf_prefix_then_block(m, prefix, block, lp)
        bb = O.backbone_from_model(SimpleNamespace(tfmr=m), max_pos=128)
        cache = O.KVCache.empty(len(bb.layers), B, 128, 4, 16, torch.bfloat16)
        O.prefix_forward(bb, [prefix[b] for b in range(B)], cache)
        hid = O.block_forward(bb, block, cache, [lp] * B)
    assert (hid.float() - blk_hf.float()).abs().max().item() <= 3e-2


def test_speech_head_token_shift():
    g = torch.Generator().manual_seed(5)
    hidden = torch.randn(2, 4, 8, generator=g)
    ctx = torch.randn(2, 1, 8, generator=g)
    W = torch.randn(11, 8, generator=g)
    lg = O.speech_head_shift(hidden, ctx, W)
    assert lg.shape == (2, 4, 11)
    torch.testing.assert_close(lg[:, 0], ctx[:, 0] @ W.T)
    for j in range(1, 4):
        torch.testing.assert_close(lg[:, j], hidden[:, j - 1] @ W.T)


def test_rms_norm_matches_hf_module():
    from transformers.models.llama.modeling_llama import LlamaRMSNorm
    n = LlamaRMSNorm(64, eps=1e-5)
    with torch.no_grad():
        n.weight.uniform_(0.5, 1.5)
    x = torch.randn(5, 64).bfloat16()
    n = n.bfloat16()
    assert torch.equal(O.rms_norm(x, n.weight, 1e-5), n(x))
