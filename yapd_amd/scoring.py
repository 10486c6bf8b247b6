"""Host side of the CFG + PMI + quantile unmask step (kernel (c)).

``omnivoice_unmask_schedule`` and ``quantile_table`` are the host-computed
tables of chatterbox_flash/model.py:133-177 and server/engine.py:355-358;
:class:`BlockScorer` owns the per-step device buffers and launches the
fused scoring kernel, replacing the vectorised scorer of
server/engine.py:532-593 and the per-row loop of
chatterbox_flash/model.py:856-900.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional

import torch

from . import kernels


def omnivoice_unmask_schedule(n_total_mask: int, num_steps: int, t_shift: float) -> List[int]:
    """Per-step unmask counts under the OmniVoice ``r_n`` curve (model.py:133-177).

    Cumulative fraction after step ``s`` is ``tau*x/(1+(tau-1)*x)`` at
    ``x = s/K``; counts are cumulative roundings (Python ``round``), capped by
    what remains, and the last step closes the block.
    """
    K = max(1, int(num_steps))
    N = max(0, int(n_total_mask))
    if N == 0:
        return [0] * K
    if K == 1:
        return [N]
    tau = float(t_shift)
    if tau <= 0:
        even = [N // K] * K
        even[-1] += N - sum(even)
        return even
    cum_target = [tau * (s / K) / (1.0 + (tau - 1.0) * (s / K)) for s in range(K + 1)]
    out: List[int] = []
    taken = 0
    for s in range(K):
        remaining = N - taken
        if s == K - 1:
            cnt = remaining
        else:
            cnt = min(max(0, int(round(N * cum_target[s + 1])) - taken), remaining)
        out.append(cnt)
        taken += cnt
    return out


def quantile_table(time_shift_tau: float, num_steps: int) -> List[float]:
    """``q_k = max(0, 1 - tau*(k+1)/K)`` (server/engine.py:357, model.py:293)."""
    return [max(0.0, 1.0 - time_shift_tau * (k + 1) / num_steps) for k in range(num_steps)]


@dataclass
class ScoreResult:
    sampled: torch.Tensor       # [pairs, bl] int64  (argmax / Gumbel-max token)
    pmi: torch.Tensor           # [pairs, bl] fp32   (CFG-combined PMI)
    unmask: torch.Tensor        # [pairs, bl] uint8
    xt: torch.Tensor            # [pairs, bl] int64  (tokens after this step)
    n_mask_after: torch.Tensor  # [pairs] int32
    hit_eos: torch.Tensor       # [pairs] uint8


class BlockScorer:
    """Persistent buffers + launcher for one block size and batch.

    ``layout`` gives where a pair's rows sit in the logits batch:
    ``"stacked"`` is ``[cond x B | null x B]`` (model.py:859-860),
    ``"interleaved"`` is ``(cond_i, null_i)`` (server/engine.py:534).  With
    ``cfg_scale == 0`` there is one row per pair (no null branch).
    Outputs are views of persistent buffers, overwritten by the next call.
    """

    def __init__(self, *, n_pairs: int, block_size: int, log_prior: torch.Tensor, mask_id: int,
                 stop_id: int, num_steps: int = 10, time_shift_tau: float = 0.1,
                 omnivoice_t_shift: float = 0.5, cfg_scale: float = 1.0,
                 device: Optional[torch.device] = None):
        dev = torch.device(device) if device is not None else log_prior.device
        self.device = dev
        self.n_pairs = int(n_pairs)
        self.bl = int(block_size)
        self.K = int(num_steps)
        self.tau = float(time_shift_tau)
        self.cfg = float(cfg_scale)
        self.mask_id = int(mask_id)
        self.stop_id = int(stop_id)
        kernels.require(1 <= self.bl <= 64, "block_size must be in [1, 64]")
        self.sched_list = omnivoice_unmask_schedule(self.bl, self.K, omnivoice_t_shift)
        self.sched = torch.tensor(self.sched_list, dtype=torch.int32, device=dev)
        self.q_t = torch.tensor(quantile_table(self.tau, self.K), dtype=torch.float32, device=dev)
        self.log_prior = log_prior.to(device=dev, dtype=torch.float32).contiguous()
        P, bl = self.n_pairs, self.bl
        self.out = dict(
            sampled=torch.empty(P, bl, dtype=torch.int64, device=dev),
            pmi=torch.empty(P, bl, dtype=torch.float32, device=dev),
            unmask=torch.empty(P, bl, dtype=torch.uint8, device=dev),
            xt_out=torch.empty(P, bl, dtype=torch.int64, device=dev),
            n_mask_after=torch.empty(P, dtype=torch.int32, device=dev),
            hit_eos=torch.empty(P, dtype=torch.uint8, device=dev),
        )

    @staticmethod
    def log_prior_from_prior(prior: torch.Tensor) -> torch.Tensor:
        """``log(clamp(prior, 1e-8))`` in fp32 (server/engine.py:362-366)."""
        return prior.float().clamp_min(1e-8).log()

    def __call__(self, logits: torch.Tensor, xt_blk: torch.Tensor, k_step: torch.Tensor, *,
                 layout: str = "stacked", active: Optional[torch.Tensor] = None,
                 temperature: float = 0.0, position_noise: bool = False, seed: int = 0,
                 rng_offset: int = 0, n_pairs: Optional[int] = None) -> ScoreResult:
        """Score the first ``n_pairs`` pairs (default: all); outputs are ``[n_pairs, ...]`` views."""
        P = self.n_pairs if n_pairs is None else int(n_pairs)
        kernels.require(1 <= P <= self.n_pairs, f"n_pairs must be in [1, {self.n_pairs}]")
        if self.cfg > 0:
            if layout == "stacked":
                row0, step, null_off = 0, 1, P
            elif layout == "interleaved":
                row0, step, null_off = 0, 2, 1
            else:
                raise ValueError(f"layout must be 'stacked' or 'interleaved', got {layout!r}")
        else:
            row0, step, null_off = 0, 1, None
        kernels.score_cfg_pmi_unmask(
            logits, n_pairs=P, cond_row0=row0, pair_row_step=step, null_row_offset=null_off,
            log_prior=self.log_prior, xt_blk=xt_blk, k_step=k_step, sched=self.sched, q_tab=self.q_t,
            cfg_w=self.cfg, quantile_on=self.tau > 0, mask_id=self.mask_id, stop_id=self.stop_id,
            out={k: v[:P] for k, v in self.out.items()}, active=active, temperature=temperature,
            pos_gumbel=position_noise, seed=seed, rng_offset=rng_offset)
        o = {k: v[:P] for k, v in self.out.items()}
        return ScoreResult(o["sampled"], o["pmi"], o["unmask"], o["xt_out"], o["n_mask_after"], o["hit_eos"])
