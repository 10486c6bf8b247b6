"""The graph embedder (``yapd_amd.embed.SpeechEmbedder``) against the model's
own ``_embed_speech_tokens`` (chatterbox_flash/model.py:397-402), bit for bit,
on the CPU: with and without a learned position embedding, for bf16 and
fp32 models (the add happens in the model dtype, then one cast to bf16)."""

import pytest
import torch

from yapd_amd.embed import SpeechEmbedder
from yapd_amd.synthetic import MASK_ID, make_t3


@pytest.mark.parametrize("learned", [False, True])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_embedder_equals_embed_speech_tokens(learned, dtype):
    model = make_t3(n_layers=1, hidden=512, heads=8, ffn=512, max_positions=64, seed=3, dtype=dtype,
                    learned_pos_emb=learned)
    rows, bl = 5, 16
    g = torch.Generator().manual_seed(0)
    toks = torch.randint(0, MASK_ID + 1, (rows, bl), generator=g)
    toks[0] = MASK_ID
    emb = SpeechEmbedder(model, bl, torch.device("cpu"))
    out = torch.empty(rows * bl, 512, dtype=torch.bfloat16)
    emb(toks.view(-1), out)
    with torch.no_grad():
        ref = model._embed_speech_tokens(toks).to(torch.bfloat16)
    assert torch.equal(out.view(rows, bl, 512), ref)
    if learned:
        # the position term is really there: positions 0..bl-1 of the block
        plain = model.speech_emb(toks).to(torch.bfloat16)
        assert not torch.equal(out.view(rows, bl, 512), plain)
        with torch.no_grad():
            slab = model.speech_pos_emb.emb.weight[:bl]
        assert torch.equal(out.view(rows, bl, 512)[2], (model.speech_emb(toks[2]) + slab).to(torch.bfloat16))


def test_embedder_refuses_token_dependent_positions():
    model = make_t3(n_layers=1, hidden=512, heads=8, ffn=512, max_positions=64, seed=3, learned_pos_emb=True)
    model.speech_pos_emb.forward = lambda t: model.speech_pos_emb.emb(t % 64)
    with pytest.raises(ValueError, match="depends on the token values"):
        SpeechEmbedder(model, 16, torch.device("cpu"))
