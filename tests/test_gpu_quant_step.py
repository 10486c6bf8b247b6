"""The quantised backbone: ``HipEngine(quant_bits=4 | 8)`` runs every layer
projection on affine group-quantised weights in the MLX layout, as the
reference's Metal engine does with ``CHATTERBOX_FLASH_MLX_QUANT_BITS``
(chatterbox_flash/engines/mlx.py:171, 221-255).  Every route dequantises W as
``w = bf16(fma(scale, q, bias))`` and runs the bf16 kernels' MFMA loop and
epilogues on it -- the fused kernels tile by tile into LDS, the
dequantise-once route (4096 rows or more, with the engine's scratch) into a
bf16 copy of the layer's weights -- so:

  (i)  a quantised engine equals a bf16 engine built on the dequantised
       weights bit for bit -- the prefill's SOS hidden, and per graph replay of
       the benched step (256 CFG pairs, block 32, 4 layers) the hidden states,
       logits and every decision -- for 4-bit and 8-bit codes;
  (ii) the full 30-layer step on 4-bit weights at the benched configuration:
       decisions against ``oracle.scoring`` on the GPU's own logits, and the
       shortest-prefix pair's hidden states and logits against the fp32 oracle
       on the dequantised weights, within the bounds of the bf16 step
       (max(2e-2, 1.5 x the bf16 oracle's own error), max(1e-2, ...) relative).

The dequantised reference weights are computed here from the product's own
codes: ``scale * q + bias`` exactly in float64, rounded once to fp32 (what the
FMA does) and then to bf16.
"""

import pytest
import torch

from oracle import llama as OL
from test_gpu_step import BL, PAIRS, ROWS, decisions_vs_oracle
from yapd_amd.engines.hip import HipEngine
from yapd_amd.quant import quantize_affine
from yapd_amd.step import DecodeStep
from yapd_amd.synthetic import MASK_ID, STOP_ID, make_t3, scoring_inputs, uniform_lengths

pytestmark = pytest.mark.gpu

D, V = 1024, 8194


def dequantized(w: torch.Tensor, bits: int) -> torch.Tensor:
    """The weight the quantised kernels multiply with: bf16(fp32(scale * q + bias))."""
    packed, s, b = quantize_affine(w, bits)
    per = 32 // bits
    words = packed.to(torch.int64) & 0xFFFFFFFF
    shifts = torch.arange(per, device=w.device, dtype=torch.int64) * bits
    q = ((words[..., None] >> shifts) & ((1 << bits) - 1)).reshape(w.shape[0], -1)
    s64 = s.double().repeat_interleave(64, dim=1)
    b64 = b.double().repeat_interleave(64, dim=1)
    return (s64 * q.double() + b64).float().bfloat16()


def dequantize_model_(model, bits: int) -> None:
    with torch.no_grad():
        for lyr in model.tfmr.layers:
            for lin in (lyr.self_attn.q_proj, lyr.self_attn.k_proj, lyr.self_attn.v_proj, lyr.self_attn.o_proj,
                        lyr.mlp.gate_proj, lyr.mlp.up_proj, lyr.mlp.down_proj):
                lin.weight.copy_(dequantized(lin.weight, bits))


def build(dev, model, lens, bits, seed, fused=False):
    pairs = len(lens)
    lps = lens + lens
    eng = HipEngine(model, max(lps) + 2 * BL, torch.bfloat16, batch_size=2 * pairs, page_table_seed=seed,
                    quant_bits=bits)
    if fused:  # no dequantisation scratch: the fused quantised kernels at every row count
        eng._wdq = None
    g = torch.Generator().manual_seed(seed + 1)
    prefixes = [torch.randn(lp, D, generator=g).to(torch.bfloat16) for lp in lens]
    sos = eng.prefix_forward([p.to(dev) for p in prefixes + prefixes])
    sc = scoring_inputs(n_pairs=pairs, bl=BL, vocab=V, seed=seed + 2, layout="stacked")
    step = DecodeStep(eng, model, n_pairs=pairs, block_size=BL, log_prior=sc.log_prior.to(dev), mask_id=MASK_ID,
                      stop_id=STOP_ID, num_steps=10, time_shift_tau=3.0, omnivoice_t_shift=0.5, cfg_scale=0.5)
    step.xt.copy_(sc.xt.to(dev))
    step.k_step.copy_(sc.k_step.to(dev))
    step.capture(list(lps), sos)
    torch.cuda.synchronize()
    return dict(model=model, eng=eng, step=step, lps=lps, lens=lens, prefixes=prefixes, sos=sos.clone(),
                log_prior=sc.log_prior.float(), pairs=pairs, bl=BL)


def replay(w):
    res = w["step"].replay()
    torch.cuda.synchronize()
    eng, rows = w["eng"], 2 * w["pairs"]
    out = {k: getattr(res, k).clone() for k in ("sampled", "pmi", "unmask", "xt", "n_mask_after", "hit_eos")}
    return eng._buffers(rows, BL).hidden.view(rows, BL, -1).clone(), eng._g_logits.clone(), out, res


# At 4096 rows or more (64 and 256 pairs, and the prefill's packed steps of
# 16384 tokens) the engine dequantises each layer's weights once into its
# scratch and runs the bf16 kernels; with fused=True (no scratch) and at 16
# pairs (1024 rows) the fused kernels run: at 256 pairs every projection on
# 256 x 256 direct-load tiles; at 16 pairs QKV, o and down on direct-load
# 128 x 128 tiles and gate/up register-staged.
@pytest.mark.parametrize("bits,pairs,fused", [(4, 256, False), (8, 256, False), (4, 64, False), (8, 16, False),
                                              (4, 256, True), (8, 64, True)])
def test_quantised_engine_equals_bf16_engine_on_dequantised_weights(dev, bits, pairs, fused):
    lens = uniform_lengths(pairs, 150, 600, seed=61)
    model_q = make_t3(n_layers=4, seed=60, norm_jitter=True, learned_pos_emb=True, device=dev)
    model_e = make_t3(n_layers=4, seed=60, norm_jitter=True, learned_pos_emb=True, device=dev)
    dequantize_model_(model_e, bits)
    wq = build(dev, model_q, lens, bits, seed=62, fused=fused)
    we = build(dev, model_e, lens, 0, seed=62)
    assert wq["eng"].quant_bits == bits and we["eng"].quant_bits == 0
    assert torch.equal(wq["sos"], we["sos"])
    for rep in range(2):
        hq, lq, oq, _ = replay(wq)
        he, le, oe, _ = replay(we)
        assert torch.isfinite(hq.float()).all()
        assert torch.equal(hq, he), rep
        assert torch.equal(lq, le), rep
        for k in oq:
            assert torch.equal(oq[k], oe[k]), (rep, k)
    assert int(oq["unmask"].sum()) > 0


def test_thirty_layer_step_on_4bit_weights_against_the_oracle(dev):
    layers = 30
    lens = uniform_lengths(PAIRS, 150, 600, seed=71)
    model_q = make_t3(n_layers=layers, seed=70, norm_jitter=True, learned_pos_emb=True, device=dev)
    w = build(dev, model_q, lens, 4, seed=72)
    hid, logits, _, res = replay(w)
    assert torch.isfinite(hid.float()).all()
    decisions_vs_oracle(res, logits, w)
    # the reference model: the same weights, dequantised
    model_e = make_t3(n_layers=layers, seed=70, norm_jitter=True, learned_pos_emb=True, device=dev)
    dequantize_model_(model_e, 4)
    eng = w["eng"]
    p = min(range(PAIRS), key=lambda i: lens[i])
    rows = [p, PAIRS + p]
    L = lens[p]
    max_pos = L + BL
    emb_rows = eng._buffers(ROWS, BL).emb.view(ROWS, BL, -1)[rows].cpu()
    W_head = model_e.speech_head.weight.float().cpu()
    refs = {}
    for name, dt in (("bf16", torch.bfloat16), ("fp32", torch.float32)):
        bb = OL.backbone_from_model(model_e, max_pos=max_pos, dtype=dt)
        cache = OL.KVCache.empty(layers, 2, max_pos, 16, 64, dt)
        s_ref = OL.prefix_forward(bb, [w["prefixes"][p].to(dt)] * 2, cache)
        h_ref = OL.block_forward(bb, emb_rows.to(dt), cache, [L, L])
        refs[name] = (h_ref, OL.speech_head_shift(h_ref.float(), s_ref.float(), W_head))
    h16, lg16 = refs["bf16"]
    h32, lg32 = refs["fp32"]
    e_gpu = (hid[rows].float().cpu() - h32).abs().max().item()
    e_ref = (h16.float() - h32).abs().max().item()
    print(f"4-bit 30-layer step, pair {p} (prefix {L}): hidden max-abs vs fp32 GPU {e_gpu:.4g}, "
          f"bf16 oracle {e_ref:.4g}")
    assert e_gpu <= max(2e-2, 1.5 * e_ref)
    scale = lg32.abs().max().item()
    rel = (logits[rows].float().cpu() - lg32).abs().max().item() / scale
    rel_ref = (lg16 - lg32).abs().max().item() / scale
    print(f"4-bit 30-layer step: logits rel err GPU {rel:.4g}, bf16 oracle {rel_ref:.4g}")
    assert rel <= max(1e-2, 1.5 * rel_ref)
