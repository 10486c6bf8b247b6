"""Seeded synthetic workloads for the T3 block step (no checkpoints needed).

Every draw uses a CPU ``torch.Generator`` (or a seeded numpy Generator) in a
fixed order and is then moved to the target device, so inputs are identical
on every machine.  Used by the tests and ``bench.py``; the real model's
weights are not available offline.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import List, Optional

import numpy as np
import torch

from .scoring import omnivoice_unmask_schedule

SPEECH_VOCAB = 8194      # speech_head outputs (model.py:340-352)
MASK_ID = 8194           # = V, the extra embedding row
SOS_ID = 6561            # start_speech_token
STOP_ID = 6562           # stop_speech_token
CODEC_V = 6561           # ids < 6561 are codec tokens


@dataclass
class ScoringInputs:
    logits: torch.Tensor      # bf16 [rows, bl, V] (rows = 2*pairs with CFG)
    log_prior: torch.Tensor   # fp32 [V]
    xt: torch.Tensor          # int64 [pairs, bl]
    k_step: torch.Tensor      # int64 [pairs]
    peaks: torch.Tensor       # int64 [pairs, bl] planted argmax ids
    layout: str


def scoring_inputs(*, n_pairs: int, bl: int = 32, vocab: int = SPEECH_VOCAB, seed: int = 0,
                   layout: str = "interleaved", logit_std: float = 3.0, peak: float = 12.0,
                   dirichlet_alpha: float = 0.1, num_steps: int = 10, k_max: int = 8,
                   t_shift: float = 0.5, mask_id: int = MASK_ID, cfg: bool = True,
                   row_pitch: Optional[int] = None, device="cpu") -> ScoringInputs:
    """The CFG + PMI scoring workload: bf16 logits ~ N(0, std) with one planted
    peak per position (the same id in the cond and null rows), a
    Dirichlet(alpha) prior, per-pair step ``k ~ U{0..k_max-1}`` and a block
    whose masked count follows the OmniVoice schedule after ``k`` steps.

    ``row_pitch`` > vocab pads each logit row (a view of ``[..., :vocab]`` is returned).
    """
    g = torch.Generator().manual_seed(seed)
    rows = 2 * n_pairs if cfg else n_pairs
    pitch = row_pitch or vocab
    base = torch.randn(rows, bl, vocab, generator=g) * logit_std
    peaks = torch.randint(0, vocab, (n_pairs, bl), generator=g)
    if cfg:
        if layout == "interleaved":
            cond_rows = torch.arange(n_pairs) * 2
            null_rows = cond_rows + 1
        elif layout == "stacked":
            cond_rows = torch.arange(n_pairs)
            null_rows = cond_rows + n_pairs
        else:
            raise ValueError(layout)
        for rows_idx in (cond_rows, null_rows):
            base[rows_idx[:, None], torch.arange(bl)[None, :], peaks] += peak
    else:
        base[torch.arange(n_pairs)[:, None], torch.arange(bl)[None, :], peaks] += peak
    buf = torch.zeros(rows, bl, pitch, dtype=torch.bfloat16)
    buf[..., :vocab] = base.to(torch.bfloat16)
    rng = np.random.default_rng(seed)
    prior = torch.from_numpy(rng.dirichlet(np.full(vocab, dirichlet_alpha))).float()
    log_prior = prior.clamp_min(1e-8).log()
    k_step = torch.randint(0, k_max, (n_pairs,), generator=g)
    sched = omnivoice_unmask_schedule(bl, num_steps, t_shift)
    xt = torch.randint(0, CODEC_V, (n_pairs, bl), generator=g)
    for p in range(n_pairs):
        n_masked = bl - sum(sched[: int(k_step[p])])
        perm = torch.randperm(bl, generator=g)[:n_masked]
        xt[p, perm] = mask_id
    logits = buf.to(device)[..., :vocab]
    return ScoringInputs(logits, log_prior.to(device), xt.to(device), k_step.to(device),
                         peaks.to(device), layout)


def split_cond_null(logits: torch.Tensor, n_pairs: int, layout: str):
    """Cond/null logit views ``[pairs, bl, V]`` for either CFG row layout."""
    if layout == "interleaved":
        return logits[0::2], logits[1::2]
    return logits[:n_pairs], logits[n_pairs: 2 * n_pairs]


def uniform_lengths(n: int, lo: int, hi: int, seed: int) -> List[int]:
    g = torch.Generator().manual_seed(seed)
    return torch.randint(lo, hi + 1, (n,), generator=g).tolist()


def log_uniform_lengths(n: int, lo: int, hi: int, seed: int) -> List[int]:
    g = torch.Generator().manual_seed(seed)
    u = torch.rand(n, generator=g, dtype=torch.float64)
    return [int(round(math.exp(math.log(lo) + float(x) * (math.log(hi) - math.log(lo))))) for x in u]
