"""Pins the scoring oracle (server/engine.py:532-593, model.py:185-311,
calibration.py, cfg_guidance.py) by closed forms, special cases, brute
force on tiny inputs, agreement of the two reference rule variants, and the
Random123 known-answer vectors of Philox4x32-10."""

import numpy as np
import pytest
import torch

from oracle import scoring as S
from oracle.schedule import omnivoice_unmask_schedule, quantile_fractions

# Random123 kat_vectors for philox4x32_10: (ctr, key) -> out
PHILOX_KAT = [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("ctr,key,want", PHILOX_KAT)
def test_philox_kat(ctr, key, want):
    got = S.philox4x32(*ctr, *key)
    assert tuple(int(x) for x in got) == want


def test_uniform_open_interval():
    u = S.uniform_from_u32(np.array([0, 0xFFFFFFFF, 0x80000000], dtype=np.uint32))
    assert u[0] > 0 and u[1] < 1 and u[2] == np.float32(0.5 + 2 ** -24)


def test_cfg_closed_form():
    g = torch.Generator().manual_seed(1)
    lc = torch.randn(3, 50, generator=g)
    lu = torch.randn(3, 50, generator=g)
    for w in (0.0, 0.5, 1.0, 2.0):
        guided = S.cfg_guided(lc, lu, w)
        # softmax(guided) is proportional to pc^(1+w) * pu^(-w)
        pc, pu = lc.softmax(-1).double(), lu.softmax(-1).double()
        want = pc ** (1 + w) * pu ** (-w)
        want = want / want.sum(-1, keepdim=True)
        torch.testing.assert_close(guided.double().softmax(-1), want, rtol=1e-5, atol=1e-9)
    assert torch.equal(S.cfg_guided(lc, None, 1.0), lc)


def _setup(B, bl, V, seed):
    g = torch.Generator().manual_seed(seed)
    lc = torch.randn(B, bl, V, generator=g) * 3
    lu = torch.randn(B, bl, V, generator=g) * 3
    prior = torch.distributions.Dirichlet(torch.full((V,), 0.1)).sample()
    return lc, lu, prior.clamp_min(1e-8).log()


def test_pmi_closed_form():
    # PMI of the argmax token: (1+w)(log pc - log prior) - w(log pu - log prior)
    lc, lu, lp = _setup(2, 4, 7, 0)
    K = 10
    sched = torch.tensor(omnivoice_unmask_schedule(4, K, 0.5))
    q = torch.tensor(quantile_fractions(0.1, K), dtype=torch.float32)
    xt = torch.full((2, 4), 99)
    r = S.score_step(lc, lu, xt, torch.zeros(2, dtype=torch.long), lp, sched, q, K=K, cfg=0.5, tau=0.1,
                     mask_id=99, stop_id=98)
    for b in range(2):
        for j in range(4):
            x = int(r["sampled"][b, j])
            guided = [(1.5 * torch.log_softmax(lc[b, j].double(), -1) - 0.5 * torch.log_softmax(lu[b, j].double(), -1))[v]
                      for v in range(7)]
            assert x == int(np.argmax([float(v) for v in guided]))
            pc = float(torch.softmax(lc[b, j].double(), -1)[x])
            pu = float(torch.softmax(lu[b, j].double(), -1)[x])
            want = 1.5 * (np.log(max(pc, 1e-8)) - float(lp[x])) - 0.5 * (np.log(max(pu, 1e-8)) - float(lp[x]))
            assert float(r["pmi"][b, j]) == pytest.approx(want, rel=1e-5, abs=1e-5)


def test_prior_clamp():
    # a prior entry below 1e-8 is clamped before the log (server/engine.py:365-366)
    prior = torch.tensor([0.5, 0.5 - 1e-12, 1e-12, 0.0])
    lp = prior.clamp_min(1e-8).log()
    assert float(lp[2]) == pytest.approx(np.log(1e-8)) and float(lp[3]) == pytest.approx(np.log(1e-8))


def _rule(pmi_rows, mask_rows, ks, K=10, tau=0.1, bl=None, t_shift=0.5):
    pmi = torch.tensor(pmi_rows, dtype=torch.float32)
    msk = torch.tensor(mask_rows, dtype=torch.bool)
    bl = pmi.shape[1]
    sched = torch.tensor(omnivoice_unmask_schedule(bl, K, t_shift))
    q = torch.tensor(quantile_fractions(tau, K), dtype=torch.float32)
    return S.unmask_rule(pmi, msk, torch.tensor(ks), sched, q, K=K, tau=tau)


def test_rule_special_cases():
    # m = 0: nothing to unmask, n = 0
    r = _rule([[1.0, 2.0, 3.0, 4.0]], [[False] * 4], [0])
    assert int(r["n_unmask"][0]) == 0 and not r["do_unmask"].any()
    # m = 1 with q > 0: tau_k is that single value, n_quant = 1
    r = _rule([[1.0, 2.0, 3.0, 4.0]], [[False, True, False, False]], [0])
    assert int(r["n_quant"][0]) == 1 and r["do_unmask"].tolist() == [[False, True, False, False]]
    # q = 0 (tau*(k+1)/K >= 1): tau_k = min over masked, so every masked position counts
    r = _rule([[5.0, -1.0, 3.0, 2.0]], [[True] * 4], [2], tau=5.0)
    assert float(r["tau_k"][0]) == -1.0 and int(r["n_quant"][0]) == 4 and r["do_unmask"].all()
    # k >= K-1 closes the block
    r = _rule([[5.0, -1.0, 3.0, 2.0]], [[True] * 4], [9])
    assert int(r["n_unmask"][0]) == 4
    # tau <= 0 disables the quantile: exactly n_sched (top by pmi)
    r = _rule([[0.5, 4.0, 3.0, 2.0, 1.0, 0.0, -1.0, 6.0]], [[True] * 8], [0], tau=0.0, K=4, t_shift=1.0)
    assert int(r["n_quant"][0]) == 0 and int(r["n_unmask"][0]) == 2
    assert r["do_unmask"][0].nonzero().flatten().tolist() == [1, 7]
    # exact ties: lowest position first
    r = _rule([[1.0, 1.0, 1.0, 1.0]], [[True] * 4], [0], tau=0.0, K=4, t_shift=1.0)
    assert r["do_unmask"][0].tolist() == [True, False, False, False]


def _brute(pmi, msk, k, K, tau, t_shift):
    """Independent restatement with Python lists and numpy fp32 scalars."""
    bl = len(pmi)
    f32 = np.float32
    sched = omnivoice_unmask_schedule(bl, K, t_shift)
    idx = [i for i in range(bl) if msk[i]]
    m = len(idx)
    if m == 0:
        return [False] * bl
    vals = sorted(f32(pmi[i]) for i in idx)
    kc = min(k, K - 1)
    p = f32(quantile_fractions(tau, K)[kc]) * f32(max(m - 1, 0))
    lo, hi = int(np.floor(p)), int(np.ceil(p))
    tk = f32(vals[lo] + f32(f32(p - f32(lo)) * f32(vals[hi] - vals[lo])))
    nq = sum(1 for i in idx if f32(pmi[i]) >= tk) if tau > 0 else 0
    n = min(max(min(sched[kc], m), nq), m)
    if k >= K - 1:
        n = m
    chosen = sorted(idx, key=lambda i: (-f32(pmi[i]), i))[:n]
    return [i in chosen for i in range(bl)]


def test_rule_brute_force_and_model_variant():
    rng = np.random.default_rng(7)
    for trial in range(400):
        bl = int(rng.integers(1, 33))
        K = int(rng.integers(1, 12))
        tau = float(rng.choice([0.0, 0.1, 0.5, 3.0]))
        t_shift = float(rng.choice([0.5, 1.0, 2.0]))
        k = int(rng.integers(0, K + 1))
        pmi = rng.normal(size=bl).astype(np.float32)
        msk = rng.random(bl) < 0.7
        r = _rule([pmi.tolist()], [msk.tolist()], [k], K=K, tau=tau, t_shift=t_shift)
        got = r["do_unmask"][0].tolist()
        assert got == _brute(pmi.tolist(), msk.tolist(), k, K, tau, t_shift)
        # model.py's per-row variant (torch.quantile + topk) agrees (no ties here)
        sched = omnivoice_unmask_schedule(bl, K, t_shift)
        kk = min(k, K - 1)
        if k <= K - 1:
            mv = S.model_rule_unmask(torch.from_numpy(pmi), torch.from_numpy(msk), k=kk, K=K,
                                     n_sched_k=sched[kk], tau=tau)
            assert mv.tolist() == got


def test_score_step_decisions_match_rule():
    lc, lu, lp = _setup(4, 16, 64, 3)
    K = 10
    sched = torch.tensor(omnivoice_unmask_schedule(16, K, 0.5))
    q = torch.tensor(quantile_fractions(0.1, K), dtype=torch.float32)
    xt = torch.full((4, 16), 99)
    xt[:, ::3] = 5
    ks = torch.tensor([0, 3, 8, 9])
    r = S.score_step(lc, lu, xt, ks, lp, sched, q, K=K, cfg=1.0, tau=0.1, mask_id=99, stop_id=5)
    assert torch.equal(r["xt_new"], torch.where(r["do_unmask"], r["sampled"], xt))
    assert r["hit_eos"].all()  # stop id 5 was already present
    assert torch.equal(r["n_mask_after"], (r["xt_new"] == 99).sum(1))
    assert int(r["n_mask_after"][3]) == 0  # k = K-1 closes the block


def test_gumbel_streams_distribution():
    g = S.gumbel_token_noise(2, 4, 1000, seed=123, offset=5)
    assert g.shape == (2, 4, 1000)
    # Gumbel(0,1): mean = Euler-Mascheroni, var = pi^2/6
    assert float(g.mean()) == pytest.approx(0.5772, abs=0.03)
    assert float(g.var()) == pytest.approx(np.pi ** 2 / 6, rel=0.05)
    g2 = S.gumbel_token_noise(2, 4, 1000, seed=123, offset=6)
    assert not torch.equal(g, g2)
    pn = S.gumbel_position_noise(4, 8, seed=1, offset=0)
    assert pn.shape == (4, 8) and torch.isfinite(pn).all()
