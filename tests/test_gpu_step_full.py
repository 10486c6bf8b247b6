"""``DecodeStep`` at the benched configuration, full depth: the 30-layer T3
backbone (D 1024, 16 heads, FFN 4096, speech head V = 8194), 256 CFG pairs in
generate()'s stacked row order (512 rows), block 32, prefixes U[150, 600]
prefilled through the engine on a shuffled page table, w = 0.5, tau = 3.0,
K = 10 (server/engine.py:491-593, model.py:823-900).  The smaller-depth
module test_gpu_step.py checks every row sample it draws against the CPU
oracle; at 30 layers and 512 rows the checks are the size-independent ones
plus one pair through the oracle:

  (i)   graph replay equals the eager path (``block_forward`` +
        ``gemm_head_shift`` + a separate ``BlockScorer``) bit for bit, on
        three replays with the eager step between them;
  (ii)  sampled tokens, unmask mask, new tokens, n_mask_after and hit_eos equal
        ``oracle.scoring.score_step`` on the GPU's own logits, bit for bit; a
        pair whose confidences tie to within fp32 rounding and is decided
        differently there is settled by the oracle's rule on the GPU's own
        confidences (``settle_confidence_near_ties``, at most 2 of 256 pairs);
        the model's jittered norm gains and learned position embedding keep
        the block's positions from sharing one token;
  (iii) the shortest-prefix pair's cond and null rows (prefill + block through
        all 30 layers, then the token-shifted head) against the fp32 oracle,
        within max(2e-2, 1.5 x the bf16 oracle's own error) for hidden states
        and max(1e-2, 1.5 x the bf16 oracle's) relative error for logits.
"""

import pytest
import torch

from oracle import llama as OL
from test_gpu_step import BL, PAIRS, ROWS, decisions_vs_oracle, eager_step
from yapd_amd.engines.hip import HipEngine
from yapd_amd.step import DecodeStep
from yapd_amd.synthetic import MASK_ID, STOP_ID, make_t3, scoring_inputs, uniform_lengths

pytestmark = pytest.mark.gpu

LAYERS, D, V = 30, 1024, 8194


@pytest.fixture(scope="module")
def world(dev):
    # jittered norm gains and a learned position embedding keep the block's positions apart
    # (a plain random model puts one token at most positions, so confidences often near-tie)
    model = make_t3(n_layers=LAYERS, seed=21, norm_jitter=True, learned_pos_emb=True, device=dev)
    lens = uniform_lengths(PAIRS, 150, 600, seed=22)
    lps = lens + lens
    eng = HipEngine(model, max(lps) + 2 * BL, torch.bfloat16, batch_size=ROWS, page_table_seed=23)
    g = torch.Generator().manual_seed(24)
    prefixes = [torch.randn(lp, D, generator=g).to(torch.bfloat16) for lp in lens]
    sos = eng.prefix_forward([p.to(dev) for p in prefixes + prefixes])
    sc = scoring_inputs(n_pairs=PAIRS, bl=BL, vocab=V, seed=25, layout="stacked")
    step = DecodeStep(eng, model, n_pairs=PAIRS, block_size=BL, log_prior=sc.log_prior.to(dev), mask_id=MASK_ID,
                      stop_id=STOP_ID, num_steps=10, time_shift_tau=3.0, omnivoice_t_shift=0.5, cfg_scale=0.5)
    step.xt.copy_(sc.xt.to(dev))
    step.k_step.copy_(sc.k_step.to(dev))
    step.capture(list(lps), sos)
    torch.cuda.synchronize()
    return dict(model=model, eng=eng, step=step, lps=lps, lens=lens, prefixes=prefixes,
                log_prior=sc.log_prior.float())


def test_thirty_layer_step_replays_match_eager_and_the_oracle(world):
    w = world
    step, eng, model = w["step"], w["eng"], w["model"]
    starts = list(w["lps"])
    step.set_cache_starts(starts)
    for rep in range(3):
        res = step.replay()
        torch.cuda.synchronize()
        hid_g = eng._buffers(ROWS, BL).hidden.view(ROWS, BL, -1).clone()
        logits_g = eng._g_logits.clone()
        out_g = {k: getattr(res, k).clone() for k in ("sampled", "pmi", "unmask", "xt", "n_mask_after", "hit_eos")}
        assert torch.isfinite(hid_g.float()).all()
        if rep == 0:
            assert int(out_g["unmask"].sum()) > 0
            decisions_vs_oracle(res, logits_g, w)
        hid_e, logits_e, res_e = eager_step(w, starts)
        assert torch.equal(hid_g, hid_e), rep
        assert torch.equal(logits_g, logits_e), rep
        for k, v in out_g.items():
            assert torch.equal(v, getattr(res_e, k)), (rep, k)

    # (iii) the shortest-prefix pair through the oracle, all 30 layers
    p = min(range(PAIRS), key=lambda i: w["lens"][i])
    rows = [p, PAIRS + p]
    L = w["lens"][p]
    max_pos = L + BL
    emb_rows = eng._buffers(ROWS, BL).emb.view(ROWS, BL, -1)[rows].cpu()
    W_head = model.speech_head.weight.float().cpu()
    refs = {}
    for name, dt in (("bf16", torch.bfloat16), ("fp32", torch.float32)):
        bb = OL.backbone_from_model(model, max_pos=max_pos, dtype=dt)
        cache = OL.KVCache.empty(LAYERS, 2, max_pos, 16, 64, dt)
        s_ref = OL.prefix_forward(bb, [w["prefixes"][p].to(dt)] * 2, cache)
        h_ref = OL.block_forward(bb, emb_rows.to(dt), cache, [L, L])
        refs[name] = (h_ref, OL.speech_head_shift(h_ref.float(), s_ref.float(), W_head))
    h16, lg16 = refs["bf16"]
    h32, lg32 = refs["fp32"]
    e_gpu = (hid_g[rows].float().cpu() - h32).abs().max().item()
    e_ref = (h16.float() - h32).abs().max().item()
    print(f"30-layer step, pair {p} (prefix {L}): hidden max-abs vs fp32 GPU {e_gpu:.4g}, bf16 oracle {e_ref:.4g}")
    assert e_gpu <= max(2e-2, 1.5 * e_ref)
    scale = lg32.abs().max().item()
    rel = (logits_g[rows].float().cpu() - lg32).abs().max().item() / scale
    rel_ref = (lg16 - lg32).abs().max().item() / scale
    print(f"30-layer step: logits rel err GPU {rel:.4g}, bf16 oracle {rel_ref:.4g}")
    assert rel <= max(1e-2, 1.5 * rel_ref)
