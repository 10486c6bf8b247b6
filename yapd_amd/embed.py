"""Block embedding of speech tokens for the captured step graphs.

The reference embeds a block with ``model._embed_speech_tokens(xt_blk)``
(chatterbox_flash/model.py:397-402, called at :833 and
server/engine.py:499): the rows of ``speech_emb``, plus
``speech_pos_emb(xt_blk)`` when ``hp.input_pos_emb == "learned"``, in the
model's dtype, then cast to the engine dtype.  ``SpeechEmbedder`` does the
same inside a graph without host work: one ``index_select`` of the table and,
for a learned position embedding, an add of a ``[bl, D]`` slab computed once
by calling the model's own ``speech_pos_emb`` on a ``[1, bl]`` token tensor.
The slab must not depend on the token values (chatterbox's module returns the
rows of positions ``0..n-1``); that is checked at construction, and a module
whose output does depend on them is refused.
"""

from __future__ import annotations

import torch


class SpeechEmbedder:
    def __init__(self, model, block_size: int, device: torch.device, out_dtype=torch.bfloat16):
        self.bl = int(block_size)
        self.table = model.speech_emb.weight.detach().to(device).contiguous()
        self.out_dtype = out_dtype
        self.slab = None
        hp = getattr(model, "hp", None)
        if getattr(hp, "input_pos_emb", None) == "learned":
            pe = model.speech_pos_emb
            with torch.no_grad():
                z = torch.zeros(1, self.bl, dtype=torch.long, device=device)
                a = pe(z)
                b = pe(torch.ones_like(z))
            if not torch.equal(a, b):
                raise ValueError("speech_pos_emb output depends on the token values; the graph embedder "
                                 "needs a per-position slab")
            self.slab = a.reshape(self.bl, -1).to(self.table.dtype).contiguous()

    def __call__(self, toks: torch.Tensor, out: torch.Tensor) -> None:
        """``out [n*bl, D] = _embed_speech_tokens(toks.view(n, bl))`` cast to ``out_dtype``."""
        if self.slab is None and self.table.dtype == out.dtype:
            torch.index_select(self.table, 0, toks, out=out)
            return
        e = torch.index_select(self.table, 0, toks)
        if self.slab is not None:
            e.view(-1, self.bl, e.shape[-1]).add_(self.slab)
        out.copy_(e)
