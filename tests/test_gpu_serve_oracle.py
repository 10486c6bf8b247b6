"""Continuous batching checked against the oracle tick by tick
(server/engine.py:406-487 admission and retirement, :491-622 the step).

Six requests go through three slots of ``HipFlashEngine`` (2 layers, CFG
0.5, argmax decoding, a learned speech position embedding), so requests are
admitted into slots freed by earlier ones (ragged prefill of only the new
rows, ``prefix_forward_rows``) and leave by swap-with-last.  Every tick is
teacher-forced from the GPU's own state before the step -- each live slot's
request, block tokens, cache length, denoise step and shift context -- and:

* the oracle runs the block forward of each live request's cond and null rows
  on its own KV cache (prefilled by ``oracle.llama.prefix_forward`` from the
  request's prefix, grown by the same blocks), and the GPU's live-row logits
  must be within max(1e-2, 1.5 x the bf16 oracle's) relative error of the
  fp32 oracle's;
* the scorer's tokens, unmask mask and new block equal ``oracle.scoring``
  run on the GPU's own logits in the server's interleaved row order, bit for
  bit (exact ties settled as in test_gpu_score.py);
* flags, final block and next state equal ``oracle.serve.tick_update`` on the
  GPU's pre-tick state.
"""

import pytest
import torch

from oracle import llama as OL
from oracle import scoring as OS
from oracle.schedule import omnivoice_unmask_schedule, quantile_fractions
from oracle.serve import SlotState, tick_update as oracle_tick
from test_gpu_score import settle_exact_ties
from yapd_amd.serve import HipFlashEngine, Request
from yapd_amd.synthetic import MASK_ID, SOS_ID, STOP_ID, make_t3

pytestmark = pytest.mark.gpu

BS, K, W, TAU, T_SHIFT, L_MAX = 16, 6, 0.5, 0.1, 0.5, 96 + 96 + 16


def requests(model, dev):
    g = torch.Generator().manual_seed(9)
    sos = model._embed_speech_tokens(torch.tensor([[SOS_ID]], device=dev))[0, 0].detach()
    out = []
    for i, (lp, ns) in enumerate([(23, 32), (61, 48), (40, 64), (17, 32), (70, 48), (33, 64)]):
        pre = (torch.randn(lp, 1024, generator=g) * 0.5).to(dev, torch.bfloat16)
        pre[-1] = sos.to(torch.bfloat16)
        out.append(Request(rid=i, prefix=pre, n_speech=ns))
    return out


class OracleRequest:
    """The oracle's KV caches (bf16 and fp32) for one request's cond and null rows."""

    def __init__(self, req, bbs):
        pre = req.prefix.cpu()
        null = torch.zeros_like(pre)
        null[-1] = pre[-1]
        self.caches = {}
        for dt, bb in bbs.items():
            c = OL.KVCache.empty(len(bb.layers), 2, L_MAX, 16, 64, dt)
            OL.prefix_forward(bb, [pre.to(dt), null.to(dt)], c)
            self.caches[dt] = c


def test_ticks_match_oracle(dev):
    model = make_t3(n_layers=2, seed=5, learned_pos_emb=True, max_positions=512, device=dev)
    V = model.speech_head.weight.shape[0]
    log_prior = torch.log_softmax(torch.randn(V, generator=torch.Generator().manual_seed(1)), 0)
    eng = HipFlashEngine(model, log_prior=log_prior, mask_id=MASK_ID, stop_id=STOP_ID, codec_vocab=SOS_ID,
                         max_active=3, max_prefix_tokens=96, max_speech_tokens=96, num_steps=K, temperature=0.0,
                         position_temperature=0.0, time_shift_tau=TAU, cfg_scale=W, block_size=BS,
                         page_table_seed=3)
    bbs = {dt: OL.backbone_from_model(model, max_pos=L_MAX, dtype=dt) for dt in (torch.bfloat16, torch.float32)}
    W_head = model.speech_head.weight.float().cpu()
    sched = torch.tensor(omnivoice_unmask_schedule(BS, K, T_SHIFT))
    q_t = torch.tensor(quantile_fractions(TAU, K), dtype=torch.float32)
    oracles = {}
    seen = dict(ticks=0, admit_after_first=0, moved=0, commit_ticks=0, worst_rel=0.0)
    slot_of = {}
    original_step = eng._step_gpu

    def checked_step(A):
        nb = eng.nb
        R = A * nb
        live = list(eng.active[:A])
        for s, r in enumerate(live):
            if r.rid not in oracles:
                oracles[r.rid] = OracleRequest(r, bbs)
                if seen["ticks"] > 0:
                    seen["admit_after_first"] += 1
            if r.rid in slot_of and slot_of[r.rid] != s:
                seen["moved"] += 1  # swap-with-last moved this request to another slot
            slot_of[r.rid] = s
        pre = SlotState(xt=eng.xt.cpu(), blk_start=eng.blk_start.cpu(), k_step=eng.k_step.cpu(),
                        cache_len=eng.cache_len.cpu(), n_speech=eng.n_speech.cpu(),
                        is_commit=eng.is_commit.cpu().bool(), shift_ctx=eng.shift_ctx.cpu())
        xt_blk = pre.xt[:A].gather(1, pre.blk_start[:A, None] + torch.arange(BS))
        original_step(A)
        torch.cuda.synchronize()
        seen["ticks"] += 1
        seen["commit_ticks"] += int(pre.is_commit[:A].sum())
        logits = eng.logits[:R].float().cpu()  # interleaved (cond_i, null_i)
        res = eng.scorer.out
        # (1) logits of every live row against the oracle at that row's cache length
        with torch.no_grad():
            emb = model._embed_speech_tokens(xt_blk.to(dev)).to(torch.bfloat16).cpu()
        for s, r in enumerate(live):
            cs = int(pre.cache_len[s])
            ctx = pre.shift_ctx[s * nb:(s + 1) * nb].float()
            lg = {}
            for dt, bb in bbs.items():
                h = OL.block_forward(bb, emb[s:s + 1].expand(2, -1, -1).to(dt), oracles[r.rid].caches[dt], [cs, cs])
                lg[dt] = OL.speech_head_shift(h.float(), ctx, W_head)
            scale = lg[torch.float32].abs().max().item()
            rel = (logits[s * nb:(s + 1) * nb] - lg[torch.float32]).abs().max().item() / scale
            rel16 = (lg[torch.bfloat16] - lg[torch.float32]).abs().max().item() / scale
            seen["worst_rel"] = max(seen["worst_rel"], rel)
            assert rel <= max(1e-2, 1.5 * rel16), f"tick {seen['ticks']} slot {s} rid {r.rid}: {rel:.4g} vs {rel16:.4g}"
        # (2) the scorer's decisions on the GPU's own logits
        lc, lu = logits[0::2].contiguous(), logits[1::2].contiguous()
        ks = pre.k_step[:A]

        def oracle(sampled=None):
            return OS.score_step(lc, lu, xt_blk, ks, log_prior, sched, q_t, K=K, cfg=W, tau=TAU, mask_id=MASK_ID,
                                 stop_id=STOP_ID, sampled=sampled)
        sampled = res["sampled"][:A].cpu()
        ref = settle_exact_ties(sampled, oracle(), lc, lu, W, oracle)
        assert torch.equal(sampled, ref["sampled"])
        assert torch.equal(res["unmask"][:A].cpu().bool(), ref["do_unmask"])
        assert torch.equal(res["xt_out"][:A].cpu(), ref["xt_new"])
        # (3) the bookkeeping on the GPU's pre-tick state
        hidden = eng.eng._buffers(R, BS).hidden.view(R, BS, -1).cpu()
        flags, xt_final = oracle_tick(pre, A, xt_blk, res["xt_out"][:A].cpu(), hidden, n_branch=nb, K=K,
                                      mask_id=MASK_ID, stop_id=STOP_ID, max_len=eng.L)
        assert torch.equal(eng.flags[:A].cpu(), flags)
        assert torch.equal(eng.xt_final[:A].cpu(), xt_final)
        for name in ("xt", "blk_start", "k_step", "cache_len"):
            assert torch.equal(getattr(eng, name)[:A].cpu(), getattr(pre, name)[:A]), name
        assert torch.equal(eng.shift_ctx[:R].cpu(), pre.shift_ctx[:R])

    eng._step_gpu = checked_step
    reqs = requests(model, dev)
    for r in reqs:
        eng.submit(r)
    eng.run_until_idle(max_ticks=2000)
    print(f"serve oracle: {seen}")
    assert all(r.t3_done for r in reqs)
    assert seen["admit_after_first"] >= 3 and seen["moved"] >= 1 and seen["commit_ticks"] >= 6
    assert any(len(r.committed) > 0 for r in reqs)
