"""Pins the schedule oracle (model.py:133-177, server/engine.py:357) by hand
tables, the closed form of the OmniVoice curve and its degenerate branches;
and checks the product's host tables against it."""

import math

import pytest

from oracle.schedule import omnivoice_unmask_schedule as oracle_sched
from oracle.schedule import quantile_fractions
from yapd_amd.scoring import omnivoice_unmask_schedule as prod_sched
from yapd_amd.scoring import quantile_table


# Hand-computed: t(s) = 0.5 s / (1 - 0.5 s); N*t rounded cumulatively.
HAND = {
    (16, 10, 0.5): [1, 1, 1, 1, 1, 2, 2, 2, 2, 3],
    (32, 10, 0.5): [2, 2, 2, 2, 3, 3, 3, 4, 5, 6],
    # tau' = 1 is the linear curve; 10*[.25,.5,.75] = 2.5, 5, 7.5 -> Python's
    # round-half-even gives 2, 5, 8.
    (10, 4, 1.0): [2, 3, 3, 2],
    (16, 10, 1.0): [2, 1, 2, 1, 2, 2, 1, 2, 1, 2],
    # degenerate branches (model.py:150-162)
    (16, 10, 0.0): [1, 1, 1, 1, 1, 1, 1, 1, 1, 7],
    (16, 10, -1.0): [1, 1, 1, 1, 1, 1, 1, 1, 1, 7],
    (16, 1, 0.5): [16],
    (0, 5, 0.5): [0, 0, 0, 0, 0],
    (3, 10, 0.5): [0, 0, 1, 0, 0, 0, 1, 0, 0, 1],
}


@pytest.mark.parametrize("args,want", sorted(HAND.items()))
def test_hand_tables(args, want):
    assert oracle_sched(*args) == want
    assert prod_sched(*args) == want


def test_closed_form_cumulative():
    # cumulative counts before the last step equal round(N * r_n(s/K)) when the
    # curve is increasing (no capping): the closed form of the schedule.
    for N in (8, 16, 32, 48, 64):
        for K in (2, 5, 10, 16):
            for t in (0.25, 0.5, 2.0, 5.0):
                c = oracle_sched(N, K, t)
                assert len(c) == K and sum(c) == N and min(c) >= 0
                cum = 0
                for s in range(K - 1):
                    cum += c[s]
                    x = (s + 1) / K
                    assert cum == round(N * t * x / (1 + (t - 1) * x))


def test_product_matches_oracle_sweep():
    for N in range(0, 65):
        for K in (1, 2, 3, 7, 10):
            for t in (-0.5, 0.0, 0.1, 0.5, 1.0, 3.0):
                assert prod_sched(N, K, t) == oracle_sched(N, K, t)


def test_quantile_table():
    q = quantile_fractions(0.1, 10)
    assert q[0] == pytest.approx(0.99) and q[-1] == pytest.approx(0.9)
    q3 = quantile_fractions(3.0, 10)
    assert q3[:3] == pytest.approx([0.7, 0.4, 0.1]) and q3[3:] == [0.0] * 7
    assert quantile_table(3.0, 10) == q3
    assert all(not math.isnan(x) for x in q3)
