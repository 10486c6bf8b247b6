"""Packed prefix prefill (``yapd_t3_prefill_packed``): a step runs segments of up to 64
consecutive tokens of the prefixes back to back -- several segments of one prefix when they fit
the step's token budget -- where a padded chunk loop computes every active row's chunk in 64
tokens and a row's last, partial chunk in full.  Run against the padded form -- the same prefixes in 64-token chunks through the dense block
forward with ``causal=1``, pad tokens zero (engines/flashinfer.py:prefix_forward :678-854) --
the SOS hidden and every prefix position's K and V must be equal bit for bit: a GEMM row, an
attention query and a norm row do not depend on the rows computed beside them.  Prefix lengths
cover a single token, a chunk minus / exactly / plus one, several chunks, and rows above 1024
keys (split attention items with the merge; their lengths are whole chunks, so that both forms
plan the same key splits -- a different split would change the merge's rounding, not the math)."""

import numpy as np
import pytest
import torch

import yapd_amd.engines.hip as engine_hip
from yapd_amd.engines.hip import PREFILL_CHUNK, HipEngine
from yapd_amd.paged import PAGE_SIZE
from yapd_amd.synthetic import make_t3

pytestmark = pytest.mark.gpu

D = 1024


def padded_prefill(eng, embs, dev):
    """The padded chunk loop: every active row computes a full 64-token chunk."""
    n = len(embs)
    lps = [int(e.shape[0]) for e in embs]
    padded = torch.nn.utils.rnn.pad_sequence(embs, batch_first=True)
    sos = torch.empty(n, 1, D, dtype=torch.bfloat16, device=dev)
    for c0 in range(0, max(lps), PREFILL_CHUNK):
        bl = min(PREFILL_CHUNK, max(lps) - c0)
        active = [r for r in range(n) if lps[r] > c0]
        na = len(active)
        buf = eng._buffers(na, bl)
        idx = torch.tensor(active, dtype=torch.long, device=dev)
        buf.emb.view(na, bl, D).copy_(padded[idx, c0: c0 + bl])
        table = None if na == n else eng._kv.table[idx]
        buf.pos0.fill_(c0)
        plan = eng._plan([c0 + bl] * na, bl)
        eng._run(buf, plan, plan.kv_len, causal=True, table=table)
        hid = buf.hidden.view(na, bl, D)
        for i, r in enumerate(active):
            if c0 <= lps[r] - 1 < c0 + bl:
                sos[r, 0] = hid[i, lps[r] - 1 - c0]
    return sos


def prefix_kv(eng, lps, layer):
    """K [pos, H, 64] and V [pos, H, 64] of every row's prefix positions, from the pool."""
    pool = eng._kv.pools[layer]
    H = pool.shape[2]
    ks, vs = [], []
    for r, lp in enumerate(lps):
        pos = np.arange(lp)
        pages = torch.as_tensor(eng._kv.table_host[r, pos // PAGE_SIZE], dtype=torch.long, device=pool.device)
        slots = torch.as_tensor(pos % PAGE_SIZE, dtype=torch.long, device=pool.device)
        tok = torch.arange(lp, device=pool.device)
        k = pool[pages, 0].view(lp, H, PAGE_SIZE, 64)[tok, :, slots]
        v = pool[pages, 1].view(lp, H, 64, PAGE_SIZE)[tok, :, :, slots]
        ks.append(k)
        vs.append(v)
    return torch.cat(ks), torch.cat(vs)


@pytest.mark.parametrize("lps,budget", [([1, 63, 64, 65, 130, 200, 17, 128], 16384),
                                        ([1, 63, 64, 65, 130, 200, 17, 128], 150),  # prefixes across steps
                                        ([1088, 40, 1280, 700], 16384), ([1088, 40, 1280, 700], 1000)])
def test_packed_prefill_equals_padded_chunks(dev, lps, budget, monkeypatch):
    monkeypatch.setattr(engine_hip, "PREFILL_TOKENS", budget)
    model = make_t3(n_layers=2, seed=61, device=dev)
    cap = max(lps) + PREFILL_CHUNK
    kw = dict(batch_size=len(lps), page_table_seed=62)
    eng_p, eng_d = HipEngine(model, cap, torch.bfloat16, **kw), HipEngine(model, cap, torch.bfloat16, **kw)
    g = torch.Generator().manual_seed(63)
    embs = [torch.randn(lp, D, generator=g).bfloat16().to(dev) for lp in lps]
    sos_p = eng_p.prefix_forward(embs)
    sos_d = padded_prefill(eng_d, embs, dev)
    torch.cuda.synchronize()
    assert torch.isfinite(sos_p.float()).all()
    assert torch.equal(sos_p, sos_d)
    assert eng_p.cache_lens == lps
    for layer in range(2):
        kp, vp = prefix_kv(eng_p, lps, layer)
        kd, vd = prefix_kv(eng_d, lps, layer)
        assert torch.equal(kp, kd), layer
        assert torch.equal(vp, vd), layer


def test_packed_prefill_of_a_row_subset(dev):
    """prefix_forward_rows (serving admissions) packs only the admitted rows; the other rows'
    KV pages are untouched."""
    model = make_t3(n_layers=1, seed=64, device=dev)
    lps = [90, 33, 160, 64]
    eng = HipEngine(model, 256, torch.bfloat16, batch_size=6, page_table_seed=65)
    g = torch.Generator().manual_seed(66)
    embs = [torch.randn(lp, D, generator=g).bfloat16().to(dev) for lp in lps]
    other = [eng._kv.table_host[r] for r in (0, 5)]
    before = [eng._kv.pools[0][torch.as_tensor(t, dtype=torch.long, device=dev)].clone() for t in other]
    sos = eng.prefix_forward_rows(1, embs)
    ref = HipEngine(model, 256, torch.bfloat16, batch_size=len(lps), page_table_seed=67)
    sos_ref = padded_prefill(ref, embs, dev)
    torch.cuda.synchronize()
    assert torch.equal(sos, sos_ref)
    for t, b in zip(other, before):
        assert torch.equal(eng._kv.pools[0][torch.as_tensor(t, dtype=torch.long, device=dev)], b)


def test_prefixes_filling_the_row_capacity(dev):
    """A prefix as long as the engine's max_seq_len (the row's last page partly used) and a
    one-token prefix beside it: same SOS and prefix KV as the padded form."""
    model = make_t3(n_layers=1, seed=68, device=dev)
    lps = [200, 1, 199]
    kw = dict(batch_size=len(lps), page_table_seed=69)
    eng_p, eng_d = HipEngine(model, 200, torch.bfloat16, **kw), HipEngine(model, 200, torch.bfloat16, **kw)
    g = torch.Generator().manual_seed(70)
    embs = [torch.randn(lp, D, generator=g).bfloat16().to(dev) for lp in lps]
    sos_p = eng_p.prefix_forward(embs)
    sos_d = padded_prefill(eng_d, embs, dev)
    torch.cuda.synchronize()
    assert torch.equal(sos_p, sos_d)
    kp, vp = prefix_kv(eng_p, lps, 0)
    kd, vd = prefix_kv(eng_d, lps, 0)
    assert torch.equal(kp, kd) and torch.equal(vp, vd)
    with pytest.raises(ValueError):
        eng_p.prefix_forward([e[:1] for e in embs[:2]] + [torch.zeros(201, D, dtype=torch.bfloat16, device=dev)])
