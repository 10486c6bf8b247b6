"""Oracle: host-side unmask schedules.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Pinned in tests/test_oracle_schedule.py by the closed form of the OmniVoice
curve, hand-computed tables and the degenerate branches.
"""

from __future__ import annotations

from typing import List


def omnivoice_unmask_schedule(n_total_mask: int, num_steps: int, t_shift: float) -> List[int]:
    """Per-step unmask counts, restating chatterbox_flash/model.py:133-177.

    ``t_s = tau*s/(1 + (tau-1)*s)`` at ``s = step/K``; counts are the cumulative
    rounding of ``N*t_{s+1}`` (Python ``round``: half to even), capped at what
    is left, and the last step takes the remainder.
    """
    K = max(1, int(num_steps))
    N = max(0, int(n_total_mask))
    if N == 0:
        return [0] * K
    if K == 1:
        return [N]
    tau = float(t_shift)
    if tau <= 0:
        base = N // K
        out = [base] * K
        out[-1] += N - sum(out)
        return out
    frac = [tau * (s / K) / (1.0 + (tau - 1.0) * (s / K)) for s in range(K + 1)]
    counts: List[int] = []
    done = 0
    left = N
    for s in range(K):
        if s == K - 1:
            num = left
        else:
            num = min(max(0, int(round(N * frac[s + 1])) - done), left)
        counts.append(num)
        done += num
        left -= num
    return counts


def quantile_fractions(time_shift_tau: float, num_steps: int) -> List[float]:
    """``q_k = max(0, 1 - tau*(k+1)/K)`` (server/engine.py:357-358, model.py:293).

    Returned as Python floats; callers convert to fp32 exactly as the
    reference does with ``torch.tensor(q, dtype=torch.float32)``.
    """
    K = int(num_steps)
    return [max(0.0, 1.0 - float(time_shift_tau) * (k + 1) / K) for k in range(K)]
