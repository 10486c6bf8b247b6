"""CPU restatement of the continuous-batching tick bookkeeping (test
infrastructure only).

Follows FlashEngine._step_gpu of server/engine.py: the shift-context update
of committing rows (:522-527), the xt write-back of denoise rows (:586-589),
``n_mask_after`` / ``hit_eos`` over the final block (:591-592), the k_step
advance (:593), the commit advance with its clamps (:595-606), the next
commit decision (:607-611) and the flags row (:613-620).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class SlotState:
    """Per-slot state of server/engine.py:338-345 (first ``n`` slots live)."""
    xt: torch.Tensor          # [S, n_max] int64
    blk_start: torch.Tensor   # [S] int64
    k_step: torch.Tensor      # [S] int64
    cache_len: torch.Tensor   # [S] int64
    n_speech: torch.Tensor    # [S] int64
    is_commit: torch.Tensor   # [S] bool
    shift_ctx: torch.Tensor   # [S * n_branch, 1, D]

    def clone(self) -> "SlotState":
        return SlotState(*(t.clone() for t in (self.xt, self.blk_start, self.k_step, self.cache_len, self.n_speech,
                                               self.is_commit, self.shift_ctx)))


def block_tokens(st: SlotState, n: int, bl: int) -> torch.Tensor:
    """xt_blk = xt[s, blk_start[s] + j] for the first n slots (server/engine.py:497-498)."""
    idx = st.blk_start[:n, None] + torch.arange(bl)
    return st.xt[:n].gather(1, idx)


def tick_update(st: SlotState, n: int, xt_blk: torch.Tensor, xt_new: torch.Tensor, hidden: torch.Tensor, *,
                n_branch: int, K: int, mask_id: int, stop_id: int, max_len: int):
    """Apply one tick's bookkeeping to ``st`` in place; returns (flags [n, 6], xt_final [n, bl]).

    ``xt_new`` is the scorer's block after unmasking; ``hidden`` the final-normed
    block hidden ``[n * n_branch, bl, D]``.
    """
    bl = xt_blk.shape[1]
    n_max = st.xt.shape[1]
    commit_rows = st.is_commit[:n].clone()
    denoise_rows = ~commit_rows
    # shift context of committing rows = the block's last hidden row
    last_h = hidden[:, bl - 1: bl]
    cm2 = commit_rows.repeat_interleave(n_branch) if n_branch == 2 else commit_rows
    st.shift_ctx[:n * n_branch] = torch.where(cm2[:, None, None], last_h, st.shift_ctx[:n * n_branch])
    # only denoise rows take the scorer's block
    xt_final = torch.where(denoise_rows[:, None], xt_new, xt_blk)
    blk_idx = st.blk_start[:n, None] + torch.arange(bl)
    st.xt[:n] = st.xt[:n].scatter(1, blk_idx, xt_final)
    n_mask_after = (xt_final == mask_id).sum(1)
    hit_eos = (xt_final == stop_id).any(1)
    ks = st.k_step[:n]
    st.k_step[:n] = torch.where(denoise_rows, ks + 1, ks)
    adv = commit_rows
    st.cache_len[:n] = torch.where(adv, (st.cache_len[:n] + bl).clamp(max=max_len - bl), st.cache_len[:n])
    st.blk_start[:n] = torch.where(adv, (st.blk_start[:n] + bl).clamp(max=n_max - bl), st.blk_start[:n])
    st.k_step[:n] = torch.where(adv, torch.zeros_like(ks), st.k_step[:n])
    st.is_commit[:n] = torch.where(adv, torch.zeros_like(adv), st.is_commit[:n])
    to_commit = denoise_rows & ~hit_eos & ((n_mask_after == 0) | (st.k_step[:n] >= K))
    st.is_commit[:n] = st.is_commit[:n] | to_commit
    flags = torch.stack([commit_rows.long(), n_mask_after, hit_eos.long(), st.k_step[:n], st.blk_start[:n],
                         st.n_speech[:n]], dim=1)
    return flags, xt_final
