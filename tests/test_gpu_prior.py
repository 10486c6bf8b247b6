"""The unconditional block prior (model.py:408-475) on the native engine
against HF LlamaModel driven the same way (causal forward of [SOS, MASK x bs]
at positions 0..bs, head on positions 0..bs-1, fp32 softmax, mean) in fp32 on
the CPU.  Tolerance: the bf16 engine's hidden differs from fp32 by ~3e-2
max-abs, which moves logits of scale ~1 by ~1e-2 and probabilities by < 1 %
relative (measured: L1 ~1e-3, worst relative 0.5 %); the test bounds the L1
distance of the two priors by 5e-3 and the worst relative error by 3e-2."""

import copy

import pytest
import torch

from yapd_amd.prior import uncond_block_prior
from yapd_amd.synthetic import make_t3

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bs", [32, 16])
def test_uncond_block_prior_matches_hf_fp32(dev, bs):
    model = make_t3(n_layers=2, seed=7, norm_jitter=True, device=dev)
    sos, mask = 6561, 8194
    prior = uncond_block_prior(model, bs, sos, mask).cpu()
    tf32 = copy.deepcopy(model.tfmr).float().cpu()
    toks = torch.tensor([sos] + [mask] * bs)
    emb = model.speech_emb.weight.detach().cpu().float()[toks].unsqueeze(0)
    with torch.no_grad():
        h = tf32(inputs_embeds=emb, position_ids=torch.arange(bs + 1).unsqueeze(0), use_cache=False).last_hidden_state
        logits = h[0, :bs] @ model.speech_head.weight.detach().cpu().float().T
    ref = torch.softmax(logits, dim=-1).mean(dim=0)
    assert prior.shape == ref.shape and abs(prior.sum().item() - 1.0) < 1e-4
    l1 = (prior - ref).abs().sum().item()
    rel = ((prior - ref).abs() / ref).max().item()
    print(f"bs={bs}: L1 {l1:.3e}, max relative {rel:.3e}")
    assert l1 <= 5e-3 and rel <= 3e-2


def test_embed_callable_follows_the_reference_call(dev):
    model = make_t3(n_layers=1, seed=8, device=dev)
    table = model.speech_emb.weight.detach()
    seen = []

    def embed(tok_seq):  # model.py:448-449 passes [1, n] token ids and gets [1, n, D]
        seen.append(tuple(tok_seq.shape))
        return table[tok_seq]

    a = uncond_block_prior(model, 8, 6561, 8194, embed=embed)
    b = uncond_block_prior(model, 8, 6561, 8194)
    assert seen == [(1, 9)] and torch.equal(a, b)


def test_block_size_limit(dev):
    model = make_t3(n_layers=1, seed=7, device=dev)
    with pytest.raises(ValueError, match="block_size"):
        uncond_block_prior(model, 64, 6561, 8194)
