"""Continuous batching on the GPU (server/engine.py FlashEngine semantics).

* the native tick bookkeeping equals the oracle bit for bit on random states;
* batch invariance: with argmax decoding a request's committed tokens do not
  depend on what it is batched with, so requests queued through a small slot
  pool (admission, swap-with-last retirement, asynchronous read-back) commit
  exactly what each commits alone.
"""

import pytest
import torch

from oracle.serve import SlotState, block_tokens, tick_update as oracle_tick
from yapd_amd import kernels
from yapd_amd.serve import HipFlashEngine, Request
from yapd_amd.synthetic import MASK_ID, SOS_ID, STOP_ID, make_t3

pytestmark = pytest.mark.gpu


def test_tick_update_matches_oracle(dev):
    g = torch.Generator().manual_seed(0)
    S, bl, D, nb, K, nmax, L = 37, 16, 1024, 2, 10, 96, 400
    xt = torch.randint(0, 50, (S, nmax), generator=g)
    xt[torch.rand(S, nmax, generator=g) < 0.5] = MASK_ID
    st = SlotState(
        xt=xt,
        blk_start=torch.randint(0, nmax // bl, (S,), generator=g) * bl,
        k_step=torch.randint(0, K, (S,), generator=g),
        cache_len=torch.randint(20, L - bl + 1, (S,), generator=g),
        n_speech=torch.randint(1, nmax // bl, (S,), generator=g) * bl,
        is_commit=torch.rand(S, generator=g) < 0.3,
        shift_ctx=torch.randn(S * nb, 1, D, generator=g).bfloat16(),
    )
    xt_blk = block_tokens(st, S, bl)
    xt_new = torch.where(torch.rand(S, bl, generator=g) < 0.7, torch.randint(0, 50, (S, bl), generator=g), xt_blk)
    xt_new[torch.rand(S, bl, generator=g) < 0.02] = STOP_ID
    xt_new[3] = 7  # a fully unmasked block
    hidden = torch.randn(S * nb, bl, D, generator=g).bfloat16()

    d = {k: v.to(dev) for k, v in dict(xt=st.xt, blk_start=st.blk_start, k_step=st.k_step, cache_len=st.cache_len,
                                      n_speech=st.n_speech, shift_ctx=st.shift_ctx).items()}
    is_commit = st.is_commit.to(torch.uint8).to(dev)
    flags = torch.empty(S, 6, dtype=torch.int64, device=dev)
    xt_final = torch.empty(S, bl, dtype=torch.int64, device=dev)
    kernels.tick_update(xt=d["xt"], xt_blk=xt_blk.to(dev), xt_new=xt_new.to(dev), k_step=d["k_step"],
                        cache_len=d["cache_len"], blk_start=d["blk_start"], is_commit=is_commit,
                        n_speech=d["n_speech"], hidden=hidden.to(dev).view(-1, D), shift_ctx=d["shift_ctx"],
                        flags=flags, xt_final=xt_final, n_branch=nb, K=K, mask_id=MASK_ID, stop_id=STOP_ID,
                        max_len=L)
    ref_flags, ref_final = oracle_tick(st, S, xt_blk, xt_new, hidden, n_branch=nb, K=K, mask_id=MASK_ID,
                                       stop_id=STOP_ID, max_len=L)
    torch.cuda.synchronize()
    assert torch.equal(flags.cpu(), ref_flags)
    assert torch.equal(xt_final.cpu(), ref_final)
    for name in ("xt", "blk_start", "k_step", "cache_len", "shift_ctx"):
        assert torch.equal(d[name].cpu(), getattr(st, name)), name
    assert torch.equal(is_commit.cpu().bool(), st.is_commit)
    assert ref_flags[:, 0].sum() > 0 and (ref_flags[:, 0] == 0).sum() > 0  # both row kinds exercised


def _requests(model, dev, seed):
    g = torch.Generator().manual_seed(seed)
    sos = model.speech_emb.weight[SOS_ID].detach()
    reqs = []
    for i, (lp, ns) in enumerate([(23, 32), (61, 48), (40, 64), (17, 32), (70, 48), (33, 64)]):
        pre = (torch.randn(lp, 1024, generator=g) * 0.5).to(dev, torch.bfloat16)
        pre[-1] = sos
        reqs.append(Request(rid=i, prefix=pre, n_speech=ns))
    return reqs


def _engine(model, log_prior, max_active):
    return HipFlashEngine(model, log_prior=log_prior, mask_id=MASK_ID, stop_id=STOP_ID, codec_vocab=SOS_ID,
                          max_active=max_active, max_prefix_tokens=96, max_speech_tokens=96, num_steps=6,
                          temperature=0.0, position_temperature=0.0, time_shift_tau=0.1, cfg_scale=0.5,
                          block_size=16, page_table_seed=3)


def test_continuous_batching_is_batch_invariant(dev):
    model = make_t3(n_layers=2, seed=5, device=dev)
    V = model.speech_head.weight.shape[0]
    log_prior = torch.log_softmax(torch.randn(V, generator=torch.Generator().manual_seed(1)), 0)
    eng = _engine(model, log_prior, max_active=3)
    batched = _requests(model, dev, seed=9)
    for r in batched:
        eng.submit(r)
    eng.run_until_idle(max_ticks=2000)
    assert len(eng.finished) == len(batched) and all(r.t3_done for r in batched)
    for r in batched:
        assert len(r.committed) <= r.n_speech
        assert all(0 <= t < SOS_ID for t in r.committed)
    assert any(len(r.committed) > 0 for r in batched)

    for r in _requests(model, dev, seed=9):
        solo = _engine(model, log_prior, max_active=1)
        solo.submit(r)
        solo.run_until_idle(max_ticks=500)
        twin = batched[r.rid]
        assert r.committed == twin.committed, f"request {r.rid}: alone {r.committed[:8]} vs batched {twin.committed[:8]}"


def test_sampling_mode_drains(dev):
    model = make_t3(n_layers=1, seed=6, device=dev)
    V = model.speech_head.weight.shape[0]
    log_prior = torch.log_softmax(torch.randn(V, generator=torch.Generator().manual_seed(2)), 0)
    eng = HipFlashEngine(model, log_prior=log_prior, mask_id=MASK_ID, stop_id=STOP_ID, codec_vocab=SOS_ID,
                         max_active=4, max_prefix_tokens=96, max_speech_tokens=96, num_steps=10,
                         temperature=0.6, position_temperature=5.0, time_shift_tau=0.1, cfg_scale=1.0)
    reqs = _requests(model, dev, seed=11)
    for r in reqs:
        eng.submit(r)
    eng.run_until_idle(max_ticks=3000)
    assert all(r.t3_done for r in reqs)
    s = eng.stats()
    assert s["active"] == 0 and s["finished"] == len(reqs) and s["commit_blocks"] >= 1
