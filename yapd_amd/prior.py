"""Unconditional block prior (the PMI denominator) on the native engine.

chatterbox_flash/model.py:408-475 (``_compute_uncond_block_prior``): one
causal forward of ``[SOS, MASK x bs]`` at positions 0..bs with no
conditioning, the speech head on the hidden of positions 0..bs-1 (the token
shift: SOS -> mask 0, mask k-1 -> mask k), softmax in fp32, mean over the bs
positions.  The forward is one causal chunk of a one-row HipEngine (so
bs <= 63), the head one ``yapd_gemm_bf16`` (bf16 logits, as the reference's
bf16 ``speech_head``); the softmax and the mean over bs x V values stay in
torch.  The reference caches the result per (block size, SOS, MASK, dtype,
device); callers keep the returned tensor likewise.
"""

from __future__ import annotations

from typing import Callable, Optional

import torch

from . import kernels
from .engines.hip import HipEngine


def uncond_block_prior(model, block_size: int, sos_id: int, mask_id: int, *,
                       embed: Optional[Callable[[torch.Tensor], torch.Tensor]] = None) -> torch.Tensor:
    """The ``(V,)`` fp32 prior of model.py:408-475.  ``embed`` maps a ``[1, n]`` token tensor to
    ``[1, n, D]`` input embeddings, as ``_embed_speech_tokens`` (model.py:397-402, called so at
    :448-449); default: the model's own ``_embed_speech_tokens`` (which adds the learned
    position embedding when the model has one), else rows of ``model.speech_emb``."""
    bs = int(block_size)
    if not 1 <= bs <= 63:
        raise ValueError(f"block_size must be in [1, 63] (one causal chunk of 1 + block_size); got {bs}")
    head_w = model.speech_head.weight.detach().to(torch.bfloat16).contiguous()
    if getattr(model.speech_head, "bias", None) is not None:
        raise ValueError("the speech head must be bias-free (T3's is)")
    dev = head_w.device
    toks = torch.tensor([int(sos_id)] + [int(mask_id)] * bs, dtype=torch.long, device=dev)
    if embed is None:
        embed = getattr(model, "_embed_speech_tokens", None) or (lambda t: model.speech_emb(t))
    with torch.no_grad():
        emb = embed(toks.unsqueeze(0))[0]
    eng = HipEngine(model, 64, torch.bfloat16, batch_size=1)
    hidden = eng.causal_forward(emb.to(torch.bfloat16))
    logits = torch.empty(bs, head_w.shape[0], dtype=torch.bfloat16, device=dev)
    kernels.gemm_bf16(hidden[:bs].contiguous(), head_w, logits)
    return torch.softmax(logits.float(), dim=-1).mean(dim=0)
