"""The per-layer parity bounds catch a misplaced rounding, and pass a correct stage.

``test_gpu_layer.py`` compares each stage of a GPU decoder layer with the bf16
oracle and accepts it while at most 2 % of the elements differ (0.1 % for the
normed output) and the 99.9th percentile of the error stays within 2 ulps
(bounds in ``_layer_stats.py``).  This CPU test applies the same statistics
and bounds to stages recomputed here in float64:

* a correct stage -- every product summed in float64 and then rounded at the
  points where the reference rounds (HF LlamaRMSNorm, rotate_half RoPE, SiLU
  and the residual adds in the model dtype; engines/flashinfer.py:992-1060)
  -- which differs from the oracle only by summation order, as a correct
  kernel does, must pass;
* the same stage with one rounding slip planted (a rounding dropped, or the
  wrong norm gain), which a kernel could make without any other visible
  error, must fail at least one bound.

Slips, by stage: input RMSNorm (normalised value not rounded before the gain;
the post-attention gain in place of the input gain), RoPE (``x*cos`` and
``rotate_half(x)*sin`` not rounded before their sum), the layer's tail
(o_proj output not rounded before the residual add; post-attention norm not
rounded before its gain, or given the input gain; silu(g) not rounded before
the product with up; down_proj output not rounded before the residual add),
and the normed output (not rounded before the gain; the layer's input gain in
place of the next norm's).
"""

import math

import torch
import torch.nn.functional as F

from _layer_stats import stats, within
from oracle import llama as OL
from yapd_amd.synthetic import make_t3

LPS = [150, 401]
BL, D, H, HD = 32, 1024, 16, 64


def _bf(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.bfloat16)


def _mm64(a: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """a @ w.T summed in float64 (exact up to the final rounding for these sizes), as float32."""
    return (a.double() @ w.double().T).float()


def _rms64(x, w, eps, slip=None):
    """HF LlamaRMSNorm with the variance summed in float64 and rounded to fp32.

    slip "round": the normalised value is not rounded to bf16 before the gain."""
    h = x.float()
    var = h.double().pow(2).mean(-1, keepdim=True).float()
    hn = h * torch.rsqrt(var + eps)
    if slip == "round":
        return _bf(w.float() * hn)
    return _bf(w.float() * _bf(hn).float())


def _rope(x, cos, sin, slip=None):
    """x [..., T, H, hd] (bf16 values as fp32); HF rounds each product and the sum."""
    c, s = cos.unsqueeze(-2).float(), sin.unsqueeze(-2).float()
    r = OL.rotate_half(x)
    if slip == "rope":
        return _bf(x * c + r * s)
    return _bf(_bf(x * c).float() + _bf(r * s).float())


def qkv64(bb, x, slip=None):
    lw = bb.layers[0]
    gain = bb.layers[0].ln_post if slip == "gain" else lw.ln_in
    hn = _rms64(x, gain, lw.eps_in, "round" if slip == "norm" else None)
    qkv = _bf(_mm64(hn, lw.wqkv))
    q, k, v = OL._split_qkv(bb, qkv)
    pos = torch.stack([torch.arange(cs, cs + BL) for cs in LPS])
    cos, sin = bb.cos[pos], bb.sin[pos]
    rs = "rope" if slip == "rope" else None
    return _rope(q.float(), cos, sin, rs), _rope(k.float(), cos, sin, rs), v


def tail64(bb, x, attn, slip=None):
    lw = bb.layers[0]
    o = _mm64(attn, lw.wo)
    h = _bf(x.float() + (o if slip == "o" else _bf(o).float()))
    gain = lw.ln_in if slip == "post_gain" else lw.ln_post
    hn = _rms64(h, gain, lw.eps_post, "round" if slip == "post_norm" else None)
    g, u = _bf(_mm64(hn, lw.wgu)).float().chunk(2, dim=-1)
    s = F.silu(g)
    a = _bf(s * u) if slip == "silu" else _bf(_bf(s).float() * u)
    d = _mm64(a, lw.wd)
    return _bf(h.float() + (d if slip == "down" else _bf(d).float()))


def _setup():
    model = make_t3(n_layers=1, seed=21, norm_jitter=True)
    bb = OL.backbone_from_model(model, max_pos=640, dtype=torch.bfloat16)
    g = torch.Generator().manual_seed(22)
    x = torch.randn(len(LPS), BL, D, generator=g).bfloat16()
    # attention output of the block's queries over random keys and values of
    # the magnitude the layer's projections give (std ~0.66), so the o_proj
    # input has the step's scale
    q, _, _ = OL.layer_qkv(bb, 0, x, LPS)
    att = []
    for r, lp in enumerate(LPS):
        kv = torch.randn(2, lp + BL, H, HD, generator=g) * 0.66
        att.append(OL._sdpa(q[r].float(), kv[0], kv[1], causal=False))
    return bb, x, torch.stack(att).bfloat16()


def _qkv_stats(bb, x, got):
    q_ref, k_ref, v_ref = OL.layer_qkv(bb, 0, x, LPS)
    lw = bb.layers[0]
    q_pre, k_pre, _ = OL._split_qkv(bb, F.linear(OL.rms_norm(x, lw.ln_in, lw.eps_in), lw.wqkv))
    mag_q = torch.maximum(torch.maximum(q_pre.float().abs(), OL.rotate_half(q_pre).float().abs()), q_ref.float().abs())
    mag_k = torch.maximum(torch.maximum(k_pre.float().abs(), OL.rotate_half(k_pre).float().abs()), k_ref.float().abs())
    return {"q": stats(got[0], q_ref, mag_q), "k": stats(got[1], k_ref, mag_k), "v": stats(got[2], v_ref, v_ref)}


def _tail_stats(bb, x, attn, got):
    lw = bb.layers[0]
    r_ref = OL.layer_tail(bb, 0, x, attn)
    o = F.linear(attn, lw.wo)
    h_mid = x + o
    g, u = F.linear(OL.rms_norm(h_mid, lw.ln_post, lw.eps_post), lw.wgu).chunk(2, dim=-1)
    d = F.linear(F.silu(g) * u, lw.wd)
    mag = torch.stack([x.float().abs(), o.float().abs(), h_mid.float().abs(), d.float().abs(),
                       r_ref.float().abs()]).max(0).values
    return stats(got, r_ref, mag), r_ref


def test_qkv_bounds_pass_correct_and_fail_slips():
    bb, x, _ = _setup()
    ok = _qkv_stats(bb, x, qkv64(bb, x))
    print("qkv correct (float64 sums):", {k: f"{v[0]:.3%} {v[1]:.2f}ulp" for k, v in ok.items()})
    assert all(within(k, v) for k, v in ok.items())
    for slip in ("norm", "gain", "rope"):
        st = _qkv_stats(bb, x, qkv64(bb, x, slip))
        print(f"qkv slip {slip}:", {k: f"{v[0]:.1%} {v[1]:.1f}ulp" for k, v in st.items()})
        assert not all(within(k, v) for k, v in st.items()), f"slip {slip} passes the bounds"


def test_tail_bounds_pass_correct_and_fail_slips():
    bb, x, attn = _setup()
    ok, _ = _tail_stats(bb, x, attn, tail64(bb, x, attn))
    print(f"residual correct (float64 sums): {ok[0]:.3%} differ, p99.9 {ok[1]:.2f} ulp")
    assert within("residual", ok)
    for slip in ("o", "post_norm", "post_gain", "silu", "down"):
        st, _ = _tail_stats(bb, x, attn, tail64(bb, x, attn, slip))
        print(f"residual slip {slip}: {st[0]:.1%} differ, p99.9 {st[1]:.1f} ulp")
        assert not within("residual", st), f"slip {slip} passes the bounds"


def test_normed_bounds_pass_correct_and_fail_slips():
    bb, x, attn = _setup()
    r = OL.layer_tail(bb, 0, x, attn)
    lw = bb.layers[0]
    ref = OL.rms_norm(r, bb.norm, bb.norm_eps)
    ok = stats(_rms64(r, bb.norm, bb.norm_eps), ref, ref)
    print(f"normed correct (float64 sums): {ok[0]:.4%} differ, p99.9 {ok[1]:.2f} ulp")
    assert within("normed", ok)
    for slip, out in (("round", _rms64(r, bb.norm, bb.norm_eps, "round")),
                      ("gain", _rms64(r, lw.ln_in, bb.norm_eps))):
        st = stats(out, ref, ref)
        print(f"normed slip {slip}: {st[0]:.1%} differ, p99.9 {st[1]:.1f} ulp")
        assert not within("normed", st), f"slip {slip} passes the bounds"
    assert math.isfinite(ok[1])
