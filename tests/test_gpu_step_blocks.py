"""``DecodeStep`` at the other block sizes: 16 (the server's default) and 64 (the largest the
attention kernel takes), so the step graph's attention runs one and four 16-query tiles per wave
(the benched block 32 runs two).  Two decoder layers, 32 CFG pairs in generate()'s stacked row
order, prefixes U[100, 300] prefilled through the engine on a shuffled page table
(server/engine.py:491-593, model.py:823-900).  Per block size: graph replay equals the eager path
(``block_forward`` + ``gemm_head_shift`` + a separate ``BlockScorer``) bit for bit -- hidden
states, logits and every decision output -- and the decisions equal ``oracle.scoring.score_step``
on the GPU's own logits (ties settled as in test_gpu_score.py).
"""

import pytest
import torch

from test_gpu_step import K, T_SHIFT, TAU, W, block_tokens, decisions_vs_oracle, eager_step
from yapd_amd.engines.hip import HipEngine
from yapd_amd.step import DecodeStep
from yapd_amd.synthetic import MASK_ID, STOP_ID, make_t3, uniform_lengths

pytestmark = pytest.mark.gpu

PAIRS = 32
OUTPUTS = ("sampled", "pmi", "unmask", "xt", "n_mask_after", "hit_eos")


@pytest.mark.parametrize("bl", [16, 64])
def test_step_replay_matches_eager_and_oracle_at_block(dev, bl):
    model = make_t3(n_layers=2, seed=31, norm_jitter=True, device=dev)
    lens = uniform_lengths(PAIRS, 100, 300, seed=32)
    lps = lens + lens
    eng = HipEngine(model, max(lps) + 2 * bl, torch.bfloat16, batch_size=2 * PAIRS, page_table_seed=33)
    gd = torch.Generator(device=dev).manual_seed(34)
    prefixes = [(torch.randn(lp, 1024, generator=gd, device=dev) * 0.5).to(torch.bfloat16) for lp in lens]
    sos = eng.prefix_forward(prefixes + prefixes)
    with torch.random.fork_rng(devices=[]):
        torch.manual_seed(35)
        prior = torch.distributions.Dirichlet(torch.full((8194,), 0.1)).sample()
    log_prior = prior.clamp_min(1e-8).log()
    step = DecodeStep(eng, model, n_pairs=PAIRS, block_size=bl, log_prior=log_prior.to(dev), mask_id=MASK_ID,
                      stop_id=STOP_ID, num_steps=K, time_shift_tau=TAU, omnivoice_t_shift=T_SHIFT, cfg_scale=W)
    xt, k_step = block_tokens(36, PAIRS, bl)
    step.xt.copy_(xt)
    step.k_step.copy_(k_step)
    step.capture(list(lps), sos)
    w = dict(model=model, eng=eng, step=step, log_prior=log_prior, pairs=PAIRS, bl=bl)
    starts = list(lps)
    step.set_cache_starts(starts)
    res = step.replay()
    torch.cuda.synchronize()
    rows = 2 * PAIRS
    hid_g = eng._buffers(rows, bl).hidden.view(rows, bl, -1).clone()
    logits_g = eng._g_logits.clone()
    out_g = {k: getattr(res, k).clone() for k in OUTPUTS}
    assert torch.isfinite(hid_g.float()).all()
    assert int(out_g["unmask"].sum()) > 0
    decisions_vs_oracle(res, logits_g, w)
    hid_e, logits_e, res_e = eager_step(w, starts)
    assert torch.equal(hid_g, hid_e)
    assert torch.equal(logits_g, logits_e)
    for k, v in out_g.items():
        assert torch.equal(v, getattr(res_e, k)), k
