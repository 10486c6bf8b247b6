"""Oracle: the T3 Llama backbone block step with torch-SDPA semantics.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Restates, on the CPU with torch ops in the model dtype:

* RMSNorm as HF ``LlamaRMSNorm`` (fp32 variance, cast to the input dtype,
  then ``weight * x``) -- used at engines/flashinfer.py:992-995, 1043-1064
  and server/engine.py:155, 172, 176;
* the fused QKV / gate-up projections of server/engine.py:119-131 and
  engines/flashinfer.py:152-168 (rows ``[q; k; v]`` and ``[gate; up]``);
* NeoX RoPE ``x*cos + rotate_half(x)*sin`` from a cos/sin table
  (engines/flashinfer.py:1009-1032, server/engine.py:145-159);
* block attention: the ``bl`` block queries see every key of ``[0, cs+bl)``
  of their own row -- the whole committed prefix plus the whole block,
  bidirectionally (engines/torch_sdpa.py:299-307 zero mask,
  engines/flashinfer.py:884-886 ``causal=False``).  Ragged cache starts are
  handled per row, which is what FlashInfer's per-row page lists compute
  (the torch-SDPA path pads ragged rows and is only exact for uniform
  starts, engines/torch_sdpa.py:309-322);
* the causal prefix prefill (engines/torch_sdpa.py:145-193);
* the token-shifted speech head ``logits[:, j] = head(hidden[:, j-1])`` with
  ``j = 0`` taken from ``shift_ctx`` (engines/flashinfer.py:1452-1461,
  chatterbox_flash/model.py:845-854).

Pinned in tests/test_oracle_llama.py against ``transformers.LlamaModel``
driven exactly as engines/torch_sdpa.py drives it.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional, Sequence

import torch
import torch.nn.functional as F


@dataclass
class LayerWeights:
    wqkv: torch.Tensor      # [(H + 2*Hkv)*hd, D]
    wo: torch.Tensor        # [D, H*hd]
    wgu: torch.Tensor       # [2F, D]
    wd: torch.Tensor        # [D, F]
    ln_in: torch.Tensor     # [D]
    ln_post: torch.Tensor   # [D]
    eps_in: float
    eps_post: float


@dataclass
class Backbone:
    layers: List[LayerWeights]
    norm: torch.Tensor
    norm_eps: float
    n_heads: int
    n_kv: int
    head_dim: int
    cos: torch.Tensor        # [max_pos, hd] in the model dtype (HF casts to x.dtype)
    sin: torch.Tensor
    dtype: torch.dtype

    @property
    def dim(self) -> int:
        return self.norm.numel()


def backbone_from_model(model, max_pos: int, dtype: Optional[torch.dtype] = None) -> Backbone:
    """Pull CPU copies of the weights off a T3-shaped model (``model.tfmr``)."""
    tf = model.tfmr
    cfg = tf.config
    H = cfg.num_attention_heads
    Hkv = cfg.num_key_value_heads
    hd = getattr(cfg, "head_dim", None) or cfg.hidden_size // H
    dt = dtype or tf.norm.weight.dtype
    layers = []
    with torch.no_grad():
        for lyr in tf.layers:
            a, m = lyr.self_attn, lyr.mlp
            layers.append(LayerWeights(
                wqkv=torch.cat([a.q_proj.weight, a.k_proj.weight, a.v_proj.weight], 0).detach().cpu().to(dt),
                wo=a.o_proj.weight.detach().cpu().to(dt),
                wgu=torch.cat([m.gate_proj.weight, m.up_proj.weight], 0).detach().cpu().to(dt),
                wd=m.down_proj.weight.detach().cpu().to(dt),
                ln_in=lyr.input_layernorm.weight.detach().cpu().to(dt),
                ln_post=lyr.post_attention_layernorm.weight.detach().cpu().to(dt),
                eps_in=float(lyr.input_layernorm.variance_epsilon),
                eps_post=float(lyr.post_attention_layernorm.variance_epsilon),
            ))
        dummy = torch.zeros(1, 1, cfg.hidden_size, dtype=dt, device=tf.norm.weight.device)
        pos = torch.arange(max_pos, device=tf.norm.weight.device).unsqueeze(0)
        cos, sin = tf.rotary_emb(dummy, pos)
    return Backbone(
        layers=layers, norm=tf.norm.weight.detach().cpu().to(dt),
        norm_eps=float(tf.norm.variance_epsilon), n_heads=H, n_kv=Hkv, head_dim=hd,
        cos=cos[0].detach().cpu().to(dt), sin=sin[0].detach().cpu().to(dt), dtype=dt,
    )


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """HF ``LlamaRMSNorm.forward``."""
    dt = x.dtype
    h = x.to(torch.float32)
    var = h.pow(2).mean(-1, keepdim=True)
    h = h * torch.rsqrt(var + eps)
    return w * h.to(dt)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    x1, x2 = x.chunk(2, dim=-1)
    return torch.cat((-x2, x1), dim=-1)


def rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """``x [..., T, H, hd]`` with ``cos/sin [..., T, hd]`` (HF ``apply_rotary_pos_emb``, unsqueeze_dim=2)."""
    c = cos.unsqueeze(-2).to(x.dtype)
    s = sin.unsqueeze(-2).to(x.dtype)
    return (x * c) + (rotate_half(x) * s)


@dataclass
class KVCache:
    """Dense per-row, per-layer K/V: ``k[layer][row]`` is ``[cap, Hkv, hd]``."""
    k: List[List[torch.Tensor]] = field(default_factory=list)
    v: List[List[torch.Tensor]] = field(default_factory=list)

    @staticmethod
    def empty(n_layers: int, n_rows: int, cap: int, Hkv: int, hd: int, dtype) -> "KVCache":
        return KVCache(
            k=[[torch.zeros(cap, Hkv, hd, dtype=dtype) for _ in range(n_rows)] for _ in range(n_layers)],
            v=[[torch.zeros(cap, Hkv, hd, dtype=dtype) for _ in range(n_rows)] for _ in range(n_layers)],
        )


def _sdpa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool) -> torch.Tensor:
    """``q [T, H, hd]``, ``k/v [S, H, hd]`` -> ``[T, H*hd]`` (scale hd^-0.5)."""
    o = F.scaled_dot_product_attention(
        q.transpose(0, 1).unsqueeze(0), k.transpose(0, 1).unsqueeze(0),
        v.transpose(0, 1).unsqueeze(0), is_causal=causal,
    )
    return o[0].transpose(0, 1).reshape(q.shape[0], -1)


def _layer_tail(bb: Backbone, lw: LayerWeights, h: torch.Tensor, attn: torch.Tensor) -> torch.Tensor:
    h = h + F.linear(attn, lw.wo)
    hn = rms_norm(h, lw.ln_post, lw.eps_post)
    gu = F.linear(hn, lw.wgu)
    g, u = gu.chunk(2, dim=-1)
    return h + F.linear(F.silu(g) * u, lw.wd)


def _split_qkv(bb: Backbone, qkv: torch.Tensor):
    H, Hkv, hd = bb.n_heads, bb.n_kv, bb.head_dim
    lead = qkv.shape[:-1]
    q = qkv[..., : H * hd].reshape(*lead, H, hd)
    k = qkv[..., H * hd: (H + Hkv) * hd].reshape(*lead, Hkv, hd)
    v = qkv[..., (H + Hkv) * hd:].reshape(*lead, Hkv, hd)
    return q, k, v


def block_forward(bb: Backbone, block_emb: torch.Tensor, cache: KVCache,
                  cache_starts: Sequence[int], n_layers: Optional[int] = None) -> torch.Tensor:
    """One block forward: ``block_emb [B, bl, D]`` -> final-normed hidden ``[B, bl, D]``.

    Writes the block's K/V tentatively at ``[cs, cs+bl)`` of every row.
    ``n_layers`` limits the stack (used only for bounded CPU timing samples).
    """
    n = len(bb.layers) if n_layers is None else n_layers
    h = block_emb.to(bb.dtype)
    for li in range(n):
        h = layer_forward(bb, li, h, cache, cache_starts)
    return rms_norm(h, bb.norm, bb.norm_eps)


def layer_forward(bb: Backbone, li: int, h: torch.Tensor, cache: KVCache,
                  cache_starts: Sequence[int]) -> torch.Tensor:
    """Decoder layer ``li`` of the block forward (torch_sdpa.py:274-341 per layer,
    server/engine.py:133-176): the residual stream ``h [B, bl, D]`` entering the layer
    -> the residual leaving it.  Writes the block's K/V of layer ``li`` at ``[cs, cs+bl)``."""
    B, bl, D = h.shape
    h = h.to(bb.dtype)
    q, k, v = layer_qkv(bb, li, h, cache_starts)
    outs = []
    for r, cs in enumerate(cache_starts):
        kc, vc = cache.k[li][r], cache.v[li][r]
        kc[cs: cs + bl] = k[r]
        vc[cs: cs + bl] = v[r]
        outs.append(_sdpa(q[r], kc[: cs + bl], vc[: cs + bl], causal=False))
    return layer_tail(bb, li, h, torch.stack(outs))


def layer_qkv(bb: Backbone, li: int, h: torch.Tensor, cache_starts: Sequence[int]):
    """First half of decoder layer ``li`` (flashinfer.py:992-1032): input RMSNorm, the fused
    QKV projection and NeoX RoPE at positions ``cs .. cs+bl-1`` -> q, k, v ``[B, bl, H, hd]``."""
    lw = bb.layers[li]
    bl = h.shape[1]
    pos = torch.stack([torch.arange(cs, cs + bl) for cs in cache_starts])  # [B, bl]
    cos, sin = bb.cos[pos], bb.sin[pos]                                      # [B, bl, hd]
    hn = rms_norm(h.to(bb.dtype), lw.ln_in, lw.eps_in)
    q, k, v = _split_qkv(bb, F.linear(hn, lw.wqkv))
    return rope(q, cos, sin), rope(k, cos, sin), v


def layer_tail(bb: Backbone, li: int, h: torch.Tensor, attn: torch.Tensor) -> torch.Tensor:
    """Second half of decoder layer ``li`` (flashinfer.py:1040-1060): o_proj and the residual
    add, post-attention RMSNorm, SwiGLU MLP and its residual add -> the residual leaving it."""
    return _layer_tail(bb, bb.layers[li], h.to(bb.dtype), attn.to(bb.dtype))


def prefix_forward(bb: Backbone, embs: Sequence[torch.Tensor], cache: KVCache) -> torch.Tensor:
    """Causal prefill of each row's prefix ``[lp_i, D]``; returns SOS hidden ``[B, 1, D]``."""
    outs = []
    for r, e in enumerate(embs):
        lp = e.shape[0]
        h = e.to(bb.dtype)
        pos = torch.arange(lp)
        cos, sin = bb.cos[pos], bb.sin[pos]
        for li, lw in enumerate(bb.layers):
            hn = rms_norm(h, lw.ln_in, lw.eps_in)
            q, k, v = _split_qkv(bb, F.linear(hn, lw.wqkv))
            q, k = rope(q, cos, sin), rope(k, cos, sin)
            cache.k[li][r][:lp] = k
            cache.v[li][r][:lp] = v
            a = _sdpa(q, k, v, causal=True)
            h = _layer_tail(bb, lw, h, a)
        h = rms_norm(h, bb.norm, bb.norm_eps)
        outs.append(h[lp - 1: lp])
    return torch.stack(outs)


def speech_head_shift(hidden: torch.Tensor, shift_ctx: torch.Tensor, w_head: torch.Tensor,
                      bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``[shift_ctx | hidden[:, :bl-1]] @ W^T`` (engines/flashinfer.py:1452-1461)."""
    bl = hidden.shape[1]
    sh = torch.cat([shift_ctx.to(hidden.dtype), hidden[:, : bl - 1]], dim=1)
    return F.linear(sh, w_head.to(hidden.dtype), None if bias is None else bias.to(hidden.dtype))
