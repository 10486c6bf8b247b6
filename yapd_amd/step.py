"""One block-diffusion decode step on the GPU, captured as a single HIP graph.

The vectorised step of server/engine.py:491-593 (and the per-step body of
chatterbox_flash/model.py:823-900) for CFG pairs in generate()'s stacked
row order ``[cond x Bp | null x Bp]`` (model.py:761-767, 859-860):

  1. embed the block tokens of every pair into both of its rows
     (``_embed_speech_tokens``, model.py:397-402, server/engine.py:497-500);
  2. 30-layer backbone + final norm + token-shifted speech head
     (HipEngine, engines/flashinfer.py:1312-1461);
  3. CFG combine + PMI + quantile unmask (kernel (c), server/engine.py:532-593).

No host synchronisation inside the step; outputs are views of persistent
buffers overwritten by the next replay.
"""

from __future__ import annotations

from typing import Dict, List, Optional

import torch

from .embed import SpeechEmbedder
from .engines.hip import HipEngine
from .scoring import BlockScorer, ScoreResult


class DecodeStep:
    def __init__(self, engine: HipEngine, model, *, n_pairs: int, block_size: int, log_prior: torch.Tensor,
                 mask_id: int, stop_id: int, num_steps: int = 10, time_shift_tau: float = 0.1,
                 omnivoice_t_shift: float = 0.5, cfg_scale: float = 1.0):
        if engine.batch_size != 2 * n_pairs:
            raise ValueError("engine batch must be 2 * n_pairs (cond and null rows)")
        self.engine = engine
        self.n_pairs = n_pairs
        self.bl = block_size
        self.dev = engine._device
        self.embed = SpeechEmbedder(model, block_size, self.dev)
        self.speech_head = model.speech_head
        self.scorer = BlockScorer(n_pairs=n_pairs, block_size=block_size, log_prior=log_prior, mask_id=mask_id,
                                  stop_id=stop_id, num_steps=num_steps, time_shift_tau=time_shift_tau,
                                  omnivoice_t_shift=omnivoice_t_shift, cfg_scale=cfg_scale, device=self.dev)
        self.xt = torch.full((n_pairs, block_size), mask_id, dtype=torch.int64, device=self.dev)
        self.k_step = torch.zeros(n_pairs, dtype=torch.int64, device=self.dev)
        self._graphs: Dict[bool, torch.cuda.CUDAGraph] = {}  # keyed by "plan splits a row"
        self.result: Optional[ScoreResult] = None

    def _body(self, merge: bool = True) -> None:
        eng = self.engine
        buf = eng._buffers(eng.batch_size, self.bl)
        toks = torch.cat([self.xt, self.xt], 0).view(-1)
        self.embed(toks, buf.emb)
        eng._run(buf, eng._g_plan, eng._g_plan.kv_len, head_w=eng._head_w, shift_ctx=eng._g_shift_ctx,
                 logits=eng._g_logits, merge=merge)
        self.result = self.scorer(eng._g_logits, self.xt, self.k_step, layout="stacked")

    def capture(self, cache_starts: List[int], shift_ctx: torch.Tensor) -> None:
        """Capture the step for these per-row cache starts (re-plan later with ``set_cache_starts``)."""
        eng = self.engine
        eng._cache_lens = list(cache_starts)
        eng.capture_cuda_graph(self.bl, speech_head=self.speech_head)
        eng.set_shift_ctx(shift_ctx)
        self.set_cache_starts(cache_starts)
        self._body()  # warm-up outside the graph
        torch.cuda.synchronize(self.dev)
        # with and without the split-KV merge launch; each replay takes the one
        # its current attention plan needs
        for merge in (True, False):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self._body(merge)
            self._graphs[merge] = g

    def set_cache_starts(self, cache_starts: List[int]) -> None:
        self.engine._update_graph_inputs(list(cache_starts))

    def replay(self) -> ScoreResult:
        self._graphs[self.engine._g_plan.n_merge_live > 0].replay()
        return self.result
