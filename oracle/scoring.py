"""Oracle: CFG + prior-calibrated PMI + quantile unmask scoring.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

:func:`score_step` restates the vectorised scorer of server/engine.py:532-593
in the same fp32 op order (the server upcasts logits with ``.float()`` at
server/engine.py:520).  One deliberate choice is recorded: the descending
rank uses a *stable* sort (lowest position first on exact ties); the
reference's ``argsort`` is unstable, so any tie order is equally faithful.

:func:`model_rule_unmask` restates the per-row rule of
chatterbox_flash/model.py:282-311 (``torch.quantile`` + ``topk``) so tests can
assert both reference variants reach the same decisions on the fixtures.

:func:`philox4x32` restates the published Philox4x32-10 counter-based
generator (Salmon, Moraes, Dror, Shaw: "Parallel random numbers: as easy as
1, 2, 3", SC'11); the GPU scorer draws its Gumbel noise from the same
stream, so the stochastic path can be replayed on the CPU.
"""

from __future__ import annotations

from typing import Dict, Optional

import numpy as np
import torch
import torch.nn.functional as F

LOG_EPS = 1e-8  # chatterbox_flash/calibration.py:19, server/engine.py:556


def cfg_guided(logits_c: torch.Tensor, logits_u: Optional[torch.Tensor], w: float) -> torch.Tensor:
    """``lsc + w*(lsc - lsu)`` on log-softmax (cfg_guidance.py:22-47, server/engine.py:536-539)."""
    if logits_u is None:
        return logits_c
    lsc = F.log_softmax(logits_c, dim=-1)
    lsu = F.log_softmax(logits_u, dim=-1)
    return lsc + w * (lsc - lsu)


def score_step(
    logits_c: torch.Tensor,           # [B, bl, V] fp32 (cond rows)
    logits_u: Optional[torch.Tensor],  # [B, bl, V] fp32 (null rows) or None
    xt_blk: torch.Tensor,             # [B, bl] int64
    k_step: torch.Tensor,             # [B] int64
    log_prior: torch.Tensor,          # [V] fp32 = log(clamp(prior, 1e-8))
    sched_t: torch.Tensor,            # [K] int64
    q_t: torch.Tensor,                # [K] fp32
    *,
    K: int,
    cfg: float,
    tau: float,
    mask_id: int,
    stop_id: int,
    temperature: float = 0.0,
    gumbel_tok: Optional[torch.Tensor] = None,   # [B, bl, V] fp32 when temperature > 0
    pos_noise: Optional[torch.Tensor] = None,    # [B, bl] fp32 added on masked positions
    active: Optional[torch.Tensor] = None,       # [B] bool; inactive rows keep xt
    sampled: Optional[torch.Tensor] = None,      # [B, bl] int64: use these tokens instead of the argmax
) -> Dict[str, torch.Tensor]:
    """server/engine.py:532-593 (fp32), returning every intermediate decision.

    ``sampled`` replaces the token choice, so the decisions that follow a
    given (e.g. tied) choice can be recomputed."""
    B, bl, V = logits_c.shape
    lc = logits_c.float()
    lu = None if logits_u is None else logits_u.float()
    if lu is not None:
        lsc = F.log_softmax(lc, dim=-1)
        lsu = F.log_softmax(lu, dim=-1)
        guided = lsc + cfg * (lsc - lsu)
        probs_c = lc.softmax(-1)
        probs_u = lu.softmax(-1)
    else:
        guided = lc
        probs_c = lc.softmax(-1)
        probs_u = None

    if sampled is not None:
        sampled = sampled.long()
    elif temperature > 0:
        assert gumbel_tok is not None
        sampled = (guided / temperature + gumbel_tok).argmax(-1)
    else:
        sampled = guided.argmax(-1)

    is_mask = xt_blk == mask_id
    lp_c = probs_c.gather(2, sampled.unsqueeze(-1)).squeeze(-1).clamp_min(LOG_EPS).log()
    pmi = lp_c - log_prior[sampled]
    if probs_u is not None:
        lp_u = probs_u.gather(2, sampled.unsqueeze(-1)).squeeze(-1).clamp_min(LOG_EPS).log()
        pmi_u = lp_u - log_prior[sampled]
        pmi = (1.0 + cfg) * pmi - cfg * pmi_u
    if pos_noise is not None:
        pmi = torch.where(is_mask, pmi + pos_noise, pmi)

    rule = unmask_rule(pmi, is_mask, k_step, sched_t, q_t, K=K, tau=tau)
    do_unmask = rule["do_unmask"]
    if active is not None:
        do_unmask = do_unmask & active[:, None]

    xt_new = torch.where(do_unmask, sampled, xt_blk)
    return dict(
        sampled=sampled,
        pmi=pmi,
        is_mask=is_mask,
        m=rule["m"],
        tau_k=rule["tau_k"],
        n_quant=rule["n_quant"],
        n_unmask=rule["n_unmask"],
        do_unmask=do_unmask,
        xt_new=xt_new,
        n_mask_after=(xt_new == mask_id).sum(1),
        hit_eos=(xt_new == stop_id).any(1),
        guided=guided,
    )


def unmask_rule(pmi: torch.Tensor, is_mask: torch.Tensor, k_step: torch.Tensor,
                sched_t: torch.Tensor, q_t: torch.Tensor, *, K: int, tau: float) -> Dict[str, torch.Tensor]:
    """Quantile count + top-n selection of server/engine.py:563-584 (fp32)."""
    B, bl = pmi.shape
    m = is_mask.sum(1)
    ks = k_step
    kc = ks.clamp(max=K - 1)
    asc = torch.where(is_mask, pmi, torch.inf).sort(1).values
    p = q_t[kc] * (m - 1).clamp_min(0).float()
    lo = p.floor().long().clamp_min(0)
    hi = p.ceil().long().clamp_min(0)
    v_lo = asc.gather(1, lo[:, None]).squeeze(1)
    v_hi = asc.gather(1, hi[:, None]).squeeze(1)
    tau_k = v_lo + (p - lo.float()) * (v_hi - v_lo)
    n_quant = ((pmi >= tau_k[:, None]) & is_mask).sum(1)
    if tau <= 0:
        n_quant = torch.zeros_like(n_quant)
    n_sched = torch.minimum(sched_t[kc], m)
    n_unmask = torch.minimum(torch.maximum(n_sched, n_quant), m)
    n_unmask = torch.where(ks >= K - 1, m, n_unmask)
    n_unmask = torch.where(m == 0, torch.zeros_like(n_unmask), n_unmask)
    keyed = torch.where(is_mask, pmi, -torch.inf)
    order = torch.sort(keyed, dim=1, descending=True, stable=True).indices
    rank = torch.empty_like(order)
    rank.scatter_(1, order, torch.arange(bl).expand(B, -1).contiguous())
    do_unmask = is_mask & (rank < n_unmask[:, None])
    return dict(m=m, tau_k=tau_k, n_quant=n_quant, n_unmask=n_unmask, do_unmask=do_unmask)


def model_rule_unmask(
    pmi_row: torch.Tensor, is_mask_row: torch.Tensor, *, k: int, K: int,
    n_sched_k: int, tau: float,
) -> torch.Tensor:
    """The per-row rule of chatterbox_flash/model.py:282-311 (``torch.quantile`` + ``topk``)."""
    bl = pmi_row.numel()
    ar = torch.arange(bl)
    if k == K - 1:
        return is_mask_row.clone()
    masked_idx = ar[is_mask_row]
    m_cur = int(masked_idx.numel())
    do = torch.zeros(bl, dtype=torch.bool)
    if m_cur > 0:
        pmi_m = pmi_row[masked_idx]
        n_sched = max(0, min(int(n_sched_k), m_cur))
        if tau > 0.0:
            q_shifted = max(0.0, 1.0 - tau * (k + 1) / K)
            tau_k = torch.quantile(pmi_m.float(), q_shifted).to(dtype=pmi_m.dtype)
            n_quant = int((pmi_m >= tau_k).sum().item())
        else:
            n_quant = 0
        n_unmask = min(max(n_sched, n_quant), m_cur)
        if n_unmask >= m_cur:
            do[masked_idx] = True
        elif n_unmask > 0:
            _, topi = pmi_m.topk(n_unmask)
            do[masked_idx[topi]] = True
    return do


# --------------------------------------------------------------------------- #
# Philox4x32-10 and the Gumbel stream of the GPU scorer
# --------------------------------------------------------------------------- #

_PHILOX_M0 = np.uint64(0xD2511F53)
_PHILOX_M1 = np.uint64(0xCD9E8D57)
_PHILOX_W0 = np.uint32(0x9E3779B9)
_PHILOX_W1 = np.uint32(0xBB67AE85)


def philox4x32(c0, c1, c2, c3, k0, k1, rounds: int = 10):
    """Vectorised Philox4x32 (SC'11); all inputs uint32 arrays or scalars."""
    c0 = np.asarray(c0, dtype=np.uint32).copy()
    c1 = np.asarray(c1, dtype=np.uint32).copy()
    c2 = np.asarray(c2, dtype=np.uint32).copy()
    c3 = np.asarray(c3, dtype=np.uint32).copy()
    k0 = np.uint32(k0)
    k1 = np.uint32(k1)
    with np.errstate(over="ignore"):
        for _ in range(rounds):
            p0 = c0.astype(np.uint64) * _PHILOX_M0
            p1 = c2.astype(np.uint64) * _PHILOX_M1
            hi0 = (p0 >> np.uint64(32)).astype(np.uint32)
            lo0 = (p0 & np.uint64(0xFFFFFFFF)).astype(np.uint32)
            hi1 = (p1 >> np.uint64(32)).astype(np.uint32)
            lo1 = (p1 & np.uint64(0xFFFFFFFF)).astype(np.uint32)
            c0, c1, c2, c3 = hi1 ^ c1 ^ k0, lo1, hi0 ^ c3 ^ k1, lo0
            k0 = np.uint32(k0 + _PHILOX_W0)
            k1 = np.uint32(k1 + _PHILOX_W1)
    return c0, c1, c2, c3


def uniform_from_u32(x: np.ndarray) -> np.ndarray:
    """Map a u32 to the open interval (0, 1): ``((x >> 9) + 0.5) * 2^-23`` in fp32 (exact, max 1 - 2^-24)."""
    return ((x >> np.uint32(9)).astype(np.float32) + np.float32(0.5)) * np.float32(2.0 ** -23)


def gumbel_token_noise(B: int, bl: int, V: int, seed: int, offset: int) -> torch.Tensor:
    """Gumbel(0,1) noise ``-log(-log(u))`` for every (pair, position, vocab id).

    Counter layout shared with the GPU scorer: ``c0 = v // 4``,
    ``c1 = pair*bl + position``, ``c2, c3 = offset lo/hi``; key = seed lo/hi;
    vocab id ``v`` takes output word ``v % 4``.
    """
    v = np.arange(V, dtype=np.int64)
    item = np.arange(B * bl, dtype=np.int64)
    c0 = np.broadcast_to((v // 4).astype(np.uint32)[None, :], (B * bl, V))
    c1 = np.broadcast_to(item.astype(np.uint32)[:, None], (B * bl, V))
    c2 = np.full((B * bl, V), offset & 0xFFFFFFFF, dtype=np.uint32)
    c3 = np.full((B * bl, V), (offset >> 32) & 0xFFFFFFFF, dtype=np.uint32)
    r = philox4x32(c0, c1, c2, c3, seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF)
    words = np.stack(r, axis=-1)  # [items, V, 4]
    sel = words[np.arange(B * bl)[:, None], np.arange(V)[None, :], (np.arange(V) % 4)[None, :]]
    u = uniform_from_u32(sel)
    g = -np.log(-np.log(u.astype(np.float64))).astype(np.float32)
    return torch.from_numpy(g.reshape(B, bl, V))


def gumbel_position_noise(B: int, bl: int, seed: int, offset: int) -> torch.Tensor:
    """Gumbel(0,1) position noise per (pair, position): counter ``(0xffffffff, item, offset)``, word 0."""
    item = np.arange(B * bl, dtype=np.uint32)
    r = philox4x32(np.full(B * bl, 0xFFFFFFFF, dtype=np.uint32), item,
                   np.full(B * bl, offset & 0xFFFFFFFF, dtype=np.uint32),
                   np.full(B * bl, (offset >> 32) & 0xFFFFFFFF, dtype=np.uint32),
                   seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF)
    u = uniform_from_u32(r[0])
    g = -np.log(-np.log(u.astype(np.float64))).astype(np.float32)
    return torch.from_numpy(g.reshape(B, bl))
