"""GPU parity of the scoring kernel (c) against the oracle
(server/engine.py:532-593): argmax tokens, unmask decisions, new block
tokens and per-pair flags must be bit-exact; PMI within fp32 rounding."""

import pytest
import torch

from oracle import scoring as S
from oracle.schedule import omnivoice_unmask_schedule, quantile_fractions
from yapd_amd.scoring import BlockScorer
from yapd_amd.synthetic import MASK_ID, STOP_ID, scoring_inputs, split_cond_null

pytestmark = pytest.mark.gpu


def run_both(dev, *, n_pairs, bl, V, seed, layout="interleaved", cfg=0.5, tau=3.0, K=10, t_shift=0.5,
             pitch=None, temperature=0.0, pos_noise=False, active=None, k_max=8):
    inp = scoring_inputs(n_pairs=n_pairs, bl=bl, vocab=V, seed=seed, layout=layout, cfg=cfg > 0,
                         row_pitch=pitch, num_steps=K, k_max=k_max, t_shift=t_shift)
    logits_dev = torch.empty(inp.logits.shape[0], bl, pitch or V, dtype=torch.bfloat16, device=dev)
    logits_dev[..., :V] = inp.logits.to(dev)
    logits_dev = logits_dev[..., :V]
    scorer = BlockScorer(n_pairs=n_pairs, block_size=bl, log_prior=inp.log_prior.to(dev), mask_id=MASK_ID,
                         stop_id=STOP_ID, num_steps=K, time_shift_tau=tau, omnivoice_t_shift=t_shift,
                         cfg_scale=cfg, device=dev)
    seed_rng, off = 1234 + seed, 77
    act_dev = None if active is None else active.to(device=dev, dtype=torch.uint8)
    res = scorer(logits_dev, inp.xt.to(dev), inp.k_step.to(dev), layout=layout, active=act_dev,
                 temperature=temperature, position_noise=pos_noise, seed=seed_rng, rng_offset=off)
    torch.cuda.synchronize()
    if cfg > 0:
        lc, lu = split_cond_null(inp.logits.float(), n_pairs, layout)
    else:
        lc, lu = inp.logits.float(), None
    sched = torch.tensor(omnivoice_unmask_schedule(bl, K, t_shift))
    q = torch.tensor(quantile_fractions(tau, K), dtype=torch.float32)
    gt = S.gumbel_token_noise(n_pairs, bl, V, seed_rng, off) if temperature > 0 else None
    pn = S.gumbel_position_noise(n_pairs, bl, seed_rng, off) if pos_noise else None
    def oracle(sampled=None):
        return S.score_step(lc.contiguous(), None if lu is None else lu.contiguous(), inp.xt, inp.k_step,
                            inp.log_prior, sched, q, K=K, cfg=cfg, tau=tau, mask_id=MASK_ID, stop_id=STOP_ID,
                            temperature=temperature, gumbel_tok=gt, pos_noise=pn, active=active, sampled=sampled)
    ref = oracle()
    if cfg > 0 and temperature == 0:
        ref = settle_exact_ties(res.sampled.cpu(), ref, lc, lu, cfg, oracle)
    return res, ref, inp


def settle_exact_ties(tok, ref, lc, lu, cfg, oracle):
    """The guided argmax of bf16 logits can be an exact tie: (1+w)*lc - w*lu is
    then equal, in exact arithmetic, for two tokens.  The kernel takes the lowest
    index among exact maxima (torch.argmax's rule on exact values); the oracle's
    fp32 lsc + w*(lsc - lsu) breaks the tie by the rounding of its log-sum-exp,
    which no other implementation reproduces.  Where the two differ, both tokens
    must be exact maxima with the kernel's the lowest; the decisions are then
    compared against the oracle run on the kernel's tokens."""
    diff = tok != ref["sampled"]
    if not diff.any():
        return ref
    g = (1.0 + cfg) * lc.double() - cfg * lu.double()  # exact for bf16 inputs and w = 0.5
    gmax = g.max(-1).values
    lowest = (g == gmax[..., None]).double().argmax(-1)
    assert torch.equal(tok[diff], lowest[diff]), "kernel token is not the lowest exact maximum"
    assert torch.equal(g.gather(-1, ref["sampled"][..., None]).squeeze(-1)[diff], gmax[diff]), \
        "oracle and kernel tokens differ away from an exact tie"
    assert diff.sum() <= max(1, diff.numel() // 1000), "too many exact ties for random logits"
    return oracle(sampled=tok)


def settle_confidence_near_ties(res, ref, k_step, sched, q, *, K, tau, mask_id, stop_id, max_frac=2 / 256):
    """The unmask rule ranks fp32 confidences and counts those at or above an interpolated quantile
    (server/engine.py:563-584).  Kernel and oracle confidences agree only to rounding (their softmax
    denominators are summed in different orders), so where two masked confidences of a pair, or a
    confidence and the pair's quantile threshold, lie within that rounding of each other, the
    decision can go either way in any implementation.  A model whose positions share one token
    makes such near-ties common.  Where the kernel's and the oracle's decisions differ: the oracle's
    rule run on the kernel's own confidences must reproduce the kernel's decisions exactly, every
    differing pair must hold a near-tie no wider than twice its largest confidence difference, at
    most ``max_frac`` of the pairs (2 of 256, at least one) may differ, and their confidences must
    agree with the oracle's to
    the 2e-5 tolerance of ``assert_exact``.  Returns the oracle's decisions on the kernel's confidences."""
    unm = res.unmask.cpu().bool()
    if torch.equal(unm, ref["do_unmask"]):
        return ref, 0
    pmi_k = res.pmi.cpu().float()
    rule = S.unmask_rule(pmi_k, ref["is_mask"], k_step, sched, q, K=K, tau=tau)
    assert torch.equal(unm, rule["do_unmask"]), "kernel decisions differ from the rule on its own confidences"
    pairs = (unm != ref["do_unmask"]).any(1).nonzero().flatten().tolist()
    assert len(pairs) <= max(1, int(max_frac * unm.shape[0])), f"{len(pairs)} pairs decided differently"
    for b in pairs:
        mk = ref["is_mask"][b]
        pr, pk = ref["pmi"][b][mk].double(), pmi_k[b][mk].double()
        eps = (pr - pk).abs().max().item()
        assert eps <= 2e-5 + 2e-5 * pr.abs().max().item(), f"pair {b}: confidences differ by {eps:.3g}"
        srt = pr.sort().values
        # distance to the threshold, leaving out the confidence it equals when the quantile index is
        # whole (that comparison moves with it); exact ties show up in the adjacent gaps
        d = (pr - ref["tau_k"][b].double()).abs()
        d = d[d > 0]
        gap = d.min().item() if d.numel() else float("inf")
        if srt.numel() > 1:
            gap = min(gap, (srt[1:] - srt[:-1]).min().item())
        assert gap <= 2 * eps, f"pair {b}: decisions differ without a near-tie (gap {gap:.3g}, eps {eps:.3g})"
    out = dict(ref)
    out["do_unmask"] = rule["do_unmask"]
    out["xt_new"] = torch.where(rule["do_unmask"], ref["sampled"], torch.where(ref["is_mask"], mask_id, out["xt_new"]))
    out["n_mask_after"] = (out["xt_new"] == mask_id).sum(1)
    out["hit_eos"] = (out["xt_new"] == stop_id).any(1)
    return out, len(pairs)


def assert_exact(res, ref):
    assert torch.equal(res.sampled.cpu(), ref["sampled"])
    torch.testing.assert_close(res.pmi.cpu(), ref["pmi"], rtol=2e-5, atol=2e-5)
    assert torch.equal(res.unmask.cpu().bool(), ref["do_unmask"])
    assert torch.equal(res.xt.cpu(), ref["xt_new"])
    assert torch.equal(res.n_mask_after.cpu().long(), ref["n_mask_after"])
    assert torch.equal(res.hit_eos.cpu().bool(), ref["hit_eos"])


@pytest.mark.parametrize("layout", ["interleaved", "stacked"])
@pytest.mark.parametrize("n_pairs,bl,V,tau,pitch", [(4, 16, 1000, 0.1, None), (8, 32, 8194, 3.0, None),
                                                    (3, 7, 8193, 0.1, 8194), (2, 64, 513, 0.5, 514),
                                                    (1, 1, 3, 0.1, 4), (1, 2, 64, 3.0, None),  # tail-only rows
                                                    (3, 40, 2050, 3.0, None)])  # ranks over > 32 positions
def test_matches_oracle(dev, layout, n_pairs, bl, V, tau, pitch):
    res, ref, _ = run_both(dev, n_pairs=n_pairs, bl=bl, V=V, seed=n_pairs + bl, layout=layout, tau=tau,
                           pitch=pitch)
    assert_exact(res, ref)


def test_odd_row_pitch_is_rejected(dev):
    # rows must start 4-byte aligned (even pitch); the check fires before any launch
    with pytest.raises(ValueError, match="even"):
        run_both(dev, n_pairs=2, bl=4, V=33, seed=1)


def test_no_cfg_single_branch(dev):
    res, ref, _ = run_both(dev, n_pairs=5, bl=16, V=2050, seed=3, cfg=0.0, tau=0.1)
    assert_exact(res, ref)


def test_padded_pitch_and_quantile_off(dev):
    res, ref, _ = run_both(dev, n_pairs=6, bl=32, V=8194, seed=11, pitch=8200, tau=0.0)
    assert_exact(res, ref)


def test_closing_step_and_active_mask(dev):
    active = torch.tensor([True, False, True, True, False, True])
    res, ref, inp = run_both(dev, n_pairs=6, bl=16, V=4096, seed=5, active=active, k_max=10)
    assert_exact(res, ref)
    keep = ~active
    assert torch.equal(res.xt.cpu()[keep], inp.xt[keep])


def test_repeated_calls_reset_tickets(dev):
    for seed in (21, 22, 23):
        res, ref, _ = run_both(dev, n_pairs=16, bl=32, V=8194, seed=seed)
        assert_exact(res, ref)


def test_full_scoring_shape(dev):
    # 256 CFG pairs (512 rows) x 32 positions x 8194 vocab, w = 0.5, tau = 3.0
    res, ref, _ = run_both(dev, n_pairs=256, bl=32, V=8194, seed=0)
    assert_exact(res, ref)
    torch.testing.assert_close(res.pmi.cpu(), ref["pmi"], rtol=2e-5, atol=2e-5)


@pytest.mark.parametrize("n_pairs,bl,V,cfg", [(96, 32, 8194, 0.5), (40, 32, 8192, 0.5), (33, 32, 8704, 0.5),
                                               (40, 32, 8194, 0.0)])
def test_pass_and_tail_structure(dev, n_pairs, bl, V, cfg):
    # A wave streams a row in passes of 1024 dwords, then a per-lane tail:
    # V = 8194 is four passes and one tail dword, V = 8192 four passes and no
    # tail, V = 8704 four passes and four tail dwords per lane; cfg = 0 runs
    # the single-branch kernel.
    res, ref, _ = run_both(dev, n_pairs=n_pairs, bl=bl, V=V, seed=V + n_pairs, cfg=cfg, layout="stacked")
    assert_exact(res, ref)


def test_sampling_replays_streams_at_scale(dev):
    res, ref, _ = run_both(dev, n_pairs=64, bl=32, V=8194, seed=4, temperature=0.6, pos_noise=True, tau=3.0)
    agree = (res.sampled.cpu() == ref["sampled"]).float().mean().item()
    assert agree >= 0.98
    same_tok = res.sampled.cpu() == ref["sampled"]
    torch.testing.assert_close(res.pmi.cpu()[same_tok], ref["pmi"][same_tok], rtol=1e-4, atol=1e-4)


def test_stochastic_streams_replay(dev):
    # Gumbel-max sampling and position noise from the shared Philox stream: the
    # oracle replays them; only ulp-level near-ties of exp/log may differ.
    res, ref, _ = run_both(dev, n_pairs=4, bl=16, V=1000, seed=9, temperature=0.6, pos_noise=True, tau=0.1)
    agree = (res.sampled.cpu() == ref["sampled"]).float().mean().item()
    assert agree >= 0.98
    same_tok = res.sampled.cpu() == ref["sampled"]
    torch.testing.assert_close(res.pmi.cpu()[same_tok], ref["pmi"][same_tok], rtol=1e-4, atol=1e-4)
