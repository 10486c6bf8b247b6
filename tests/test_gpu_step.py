"""``DecodeStep`` -- the benched block-diffusion step (embed -> backbone +
token-shifted head -> CFG/PMI/quantile unmask, one HIP graph) -- at the bench
shape: 256 CFG pairs in generate()'s stacked row order (512 rows), block 32,
w = 0.5, tau = 3.0, K = 10, prefixes U[150, 600] prefilled through the engine
on a shuffled page table (server/engine.py:491-593, model.py:823-900).  Two
decoder layers keep the CPU oracle to seconds; the 30-layer backbone is
checked on 32 rows in test_gpu_engine.py.  The model has a learned speech
position embedding, so the embedded rows carry it.

Checked per replay:
  (i)   the embedded rows equal ``_embed_speech_tokens(xt)`` (model.py:397-402)
        in both halves of the batch, bit for bit;
  (ii)  hidden states and logits of a row sample against the oracle
        (max(2e-2, 1.5 x the bf16 oracle's own error) vs fp32);
  (iii) sampled tokens, unmask mask, new tokens, n_mask_after and hit_eos equal
        ``oracle.scoring.score_step`` run on the GPU's own logits, bit for bit
        (exact ties of the guided score, and confidences that tie to within
        their fp32 rounding, settled as in test_gpu_score.py);
  (iv)  graph replay equals the eager path (``block_forward`` +
        ``gemm_head_shift`` + a separate ``BlockScorer``) bit for bit, once
        with cache starts that split no row (graph without the merge launch)
        and once with a row long enough for the planner to split (merge graph).
"""

import pytest
import torch

from oracle import llama as OL
from oracle import scoring as OS
from oracle.schedule import omnivoice_unmask_schedule, quantile_fractions
from test_gpu_score import settle_confidence_near_ties, settle_exact_ties
from yapd_amd import kernels
from yapd_amd.engines.hip import HipEngine
from yapd_amd.scoring import BlockScorer
from yapd_amd.step import DecodeStep
from yapd_amd.synthetic import CODEC_V, MASK_ID, STOP_ID, make_t3, uniform_lengths

pytestmark = pytest.mark.gpu

PAIRS, BL, W, TAU, K, T_SHIFT = 256, 32, 0.5, 3.0, 10, 0.5
ROWS = 2 * PAIRS
SAMPLE = (0, 77, 255)  # pairs whose cond and null rows go through the CPU oracle


def block_tokens(seed, pairs=PAIRS, bl=BL):
    """Per pair a step index k ~ U{0..7} and a block whose masked count follows the
    OmniVoice schedule after k steps; a few unmasked positions hold STOP."""
    g = torch.Generator().manual_seed(seed)
    k_step = torch.randint(0, 8, (pairs,), generator=g)
    sched = omnivoice_unmask_schedule(bl, K, T_SHIFT)
    xt = torch.randint(0, CODEC_V, (pairs, bl), generator=g)
    for p in range(pairs):
        n_masked = bl - sum(sched[: int(k_step[p])])
        xt[p, torch.randperm(bl, generator=g)[:n_masked]] = MASK_ID
    stop_rows = torch.randint(0, pairs, (8,), generator=g)
    for p in stop_rows.tolist():
        free = (xt[p] != MASK_ID).nonzero().flatten()
        if len(free):
            xt[p, free[0]] = STOP_ID
    return xt, k_step


@pytest.fixture(scope="module")
def world(dev):
    model = make_t3(n_layers=2, seed=11, norm_jitter=True, learned_pos_emb=True, max_positions=2048, device=dev)
    lens = uniform_lengths(PAIRS, 150, 600, seed=12)
    lps = lens + lens  # stacked: cond rows 0..255, null rows 256..511 share their pair's length
    gd = torch.Generator(device=dev).manual_seed(13)
    prefixes = [(torch.randn(lp, 1024, generator=gd, device=dev) * 0.5).to(torch.bfloat16) for lp in lps]
    eng = HipEngine(model, 2464, torch.bfloat16, batch_size=ROWS, page_table_seed=14)
    sos = eng.prefix_forward(prefixes)
    g = torch.Generator().manual_seed(15)
    prior = torch.distributions.Dirichlet(torch.full((8194,), 0.1)).sample()
    log_prior = prior.clamp_min(1e-8).log()
    step = DecodeStep(eng, model, n_pairs=PAIRS, block_size=BL, log_prior=log_prior.to(dev), mask_id=MASK_ID,
                      stop_id=STOP_ID, num_steps=K, time_shift_tau=TAU, omnivoice_t_shift=T_SHIFT, cfg_scale=W)
    xt, k_step = block_tokens(16)
    step.xt.copy_(xt)
    step.k_step.copy_(k_step)
    step.capture(list(lps), sos)
    return dict(model=model, eng=eng, step=step, lps=lps, prefixes=prefixes, sos=sos, log_prior=log_prior,
                xt=xt, k_step=k_step)


def embedded_reference(model, xt):
    with torch.no_grad():
        return model._embed_speech_tokens(xt).to(torch.bfloat16)


def eager_step(w, starts):
    """block_forward + gemm_head_shift + a separate BlockScorer on the step's inputs."""
    eng, model, step = w["eng"], w["model"], w["step"]
    pairs, bl = w.get("pairs", PAIRS), w.get("bl", BL)
    emb = embedded_reference(model, torch.cat([step.xt, step.xt], 0))
    hid = eng.block_forward(emb, starts)
    V = model.speech_head.weight.shape[0]
    logits_buf = torch.zeros(2 * pairs, bl, (V + 7) // 8 * 8, dtype=torch.bfloat16, device=hid.device)
    logits = logits_buf[..., :V]
    kernels.gemm_head_shift(hid, eng._g_shift_ctx, eng._head_w, logits)
    scorer = BlockScorer(n_pairs=pairs, block_size=bl, log_prior=w["log_prior"].to(hid.device), mask_id=MASK_ID,
                         stop_id=STOP_ID, num_steps=K, time_shift_tau=TAU, omnivoice_t_shift=T_SHIFT, cfg_scale=W,
                         device=hid.device)
    res = scorer(logits, step.xt, step.k_step, layout="stacked")
    torch.cuda.synchronize()
    return hid, logits, res


def decisions_vs_oracle(res, logits, w):
    pairs, bl = w.get("pairs", PAIRS), w.get("bl", BL)
    lf = logits.float().cpu()
    lc, lu = lf[:pairs].contiguous(), lf[pairs:].contiguous()
    sched = torch.tensor(omnivoice_unmask_schedule(bl, K, T_SHIFT))
    q = torch.tensor(quantile_fractions(TAU, K), dtype=torch.float32)
    xt, ks = w["step"].xt.cpu(), w["step"].k_step.cpu()

    def oracle(sampled=None):
        return OS.score_step(lc, lu, xt, ks, w["log_prior"], sched, q, K=K, cfg=W, tau=TAU, mask_id=MASK_ID,
                             stop_id=STOP_ID, sampled=sampled)
    ref = settle_exact_ties(res.sampled.cpu(), oracle(), lc, lu, W, oracle)
    assert torch.equal(res.sampled.cpu(), ref["sampled"])
    torch.testing.assert_close(res.pmi.cpu(), ref["pmi"], rtol=2e-5, atol=2e-5)
    ref, n_near = settle_confidence_near_ties(res, ref, ks, sched, q, K=K, tau=TAU, mask_id=MASK_ID,
                                              stop_id=STOP_ID)
    print(f"decisions: {n_near} of {pairs} pairs settled at confidence near-ties")
    assert torch.equal(res.unmask.cpu().bool(), ref["do_unmask"])
    assert torch.equal(res.xt.cpu(), ref["xt_new"])
    assert torch.equal(res.n_mask_after.cpu().long(), ref["n_mask_after"])
    assert torch.equal(res.hit_eos.cpu().bool(), ref["hit_eos"])
    return ref


def test_step_replay_no_split_matches_eager_and_oracle(world):
    w = world
    step, eng, model = w["step"], w["eng"], w["model"]
    starts = list(w["lps"])
    step.set_cache_starts(starts)
    assert eng._g_plan.n_merge_live == 0  # rows <= 632 keys: no split, graph without the merge launch
    res = step.replay()
    torch.cuda.synchronize()
    buf = eng._buffers(ROWS, BL)
    # (i) embedded rows, both halves
    emb_ref = embedded_reference(model, w["xt"].to(buf.emb.device)).view(PAIRS * BL, -1)
    emb = buf.emb.view(ROWS * BL, -1)
    assert torch.equal(emb[: PAIRS * BL], emb_ref) and torch.equal(emb[PAIRS * BL:], emb_ref)
    hid_g = buf.hidden.view(ROWS, BL, -1).clone()
    logits_g = eng._g_logits.clone()
    out_g = {k: getattr(res, k).clone() for k in ("sampled", "pmi", "unmask", "xt", "n_mask_after", "hit_eos")}
    n_unmasked = int(out_g["unmask"].sum())
    assert n_unmasked > 0 and int(out_g["hit_eos"].sum()) > 0  # the rule unmasked something; EOS seen
    # (iii) decisions on the GPU's own logits
    decisions_vs_oracle(res, logits_g, w)
    # (iv) eager path, bit for bit
    hid_e, logits_e, res_e = eager_step(w, starts)
    assert torch.equal(hid_g, hid_e)
    assert torch.equal(logits_g, logits_e)
    for k, v in out_g.items():
        assert torch.equal(v, getattr(res_e, k)), k
    # (ii) a row sample against the oracle (prefill + block), bf16 and fp32
    rows = [p for p in SAMPLE] + [PAIRS + p for p in SAMPLE]
    emb_rows = emb.view(ROWS, BL, -1)[rows].cpu()
    W_head = model.speech_head.weight.float().cpu()
    refs = {}
    for name, dt in (("bf16", torch.bfloat16), ("fp32", torch.float32)):
        bb = OL.backbone_from_model(model, max_pos=1120, dtype=dt)
        cache = OL.KVCache.empty(2, len(rows), 1120, 16, 64, dt)
        s_ref = OL.prefix_forward(bb, [w["prefixes"][r].cpu().to(dt) for r in rows], cache)
        h_ref = OL.block_forward(bb, emb_rows.to(dt), cache, [starts[r] for r in rows])
        refs[name] = (h_ref, OL.speech_head_shift(h_ref.float(), s_ref.float(), W_head))
    h16, lg16 = refs["bf16"]
    h32, lg32 = refs["fp32"]
    hid_s = hid_g[rows].float().cpu()
    e_gpu, e_ref = (hid_s - h32).abs().max().item(), (h16.float() - h32).abs().max().item()
    print(f"step rows {rows}: hidden max-abs vs fp32 GPU {e_gpu:.4g}, bf16 oracle {e_ref:.4g}")
    assert e_gpu <= max(2e-2, 1.5 * e_ref)
    scale = lg32.abs().max().item()
    rel = (logits_g[rows].float().cpu() - lg32).abs().max().item() / scale
    rel_ref = (lg16 - lg32).abs().max().item() / scale
    print(f"step rows: logits rel err GPU {rel:.4g}, bf16 oracle {rel_ref:.4g}")
    assert rel <= max(1e-2, 1.5 * rel_ref)


def test_step_replay_with_split_row_matches_eager(world):
    w = world
    step, eng = w["step"], w["eng"]
    starts = list(w["lps"])
    # pair 0: 2432 keys, split by the bench's planner (~192 items of at least 1024 keys: here ~37 chunks
    # of 32 keys per item, so a row needs more than ~1184 keys); positions past the prefix hold zeros
    starts[0] = starts[PAIRS] = 2400
    step.set_cache_starts(starts)
    assert eng._g_plan.n_merge_live > 0  # the merge graph replays
    res = step.replay()
    torch.cuda.synchronize()
    hid_g = eng._buffers(ROWS, BL).hidden.view(ROWS, BL, -1).clone()
    logits_g = eng._g_logits.clone()
    out_g = {k: getattr(res, k).clone() for k in ("sampled", "pmi", "unmask", "xt", "n_mask_after", "hit_eos")}
    assert torch.isfinite(hid_g.float()).all()
    decisions_vs_oracle(res, logits_g, w)
    hid_e, logits_e, res_e = eager_step(w, starts)
    assert torch.equal(hid_g, hid_e)
    assert torch.equal(logits_g, logits_e)
    for k, v in out_g.items():
        assert torch.equal(v, getattr(res_e, k)), k
    # back to the unsplit starts: the graph without the merge launch again
    step.set_cache_starts(list(w["lps"]))
    assert eng._g_plan.n_merge_live == 0


def test_step_replays_repeat_with_eager_work_between(world):
    """Three replays of the step graph with the eager step (the program's own work) and a device
    synchronisation between them: every replay equals the eager result bit for bit."""
    w = world
    step, eng = w["step"], w["eng"]
    starts = list(w["lps"])
    step.set_cache_starts(starts)
    for rep in range(3):
        res = step.replay()
        torch.cuda.synchronize()
        hid_g = eng._buffers(ROWS, BL).hidden.view(ROWS, BL, -1).clone()
        logits_g = eng._g_logits.clone()
        out_g = {k: getattr(res, k).clone() for k in ("sampled", "pmi", "unmask", "xt", "n_mask_after", "hit_eos")}
        hid_e, logits_e, res_e = eager_step(w, starts)
        assert torch.equal(hid_g, hid_e), rep
        assert torch.equal(logits_g, logits_e), rep
        for k, v in out_g.items():
            assert torch.equal(v, getattr(res_e, k)), (rep, k)
