"""Seeded synthetic workloads for the T3 block step (no checkpoints needed).

Every draw uses a CPU ``torch.Generator`` (or a seeded numpy Generator) in a
fixed order and is then moved to the target device, so inputs are identical
on every machine.  Used by the tests and ``bench.py``; the real model's
weights are not available offline.
"""

from __future__ import annotations

import math
import types
from dataclasses import dataclass
from typing import List, Optional

import numpy as np
import torch

from .scoring import omnivoice_unmask_schedule

SPEECH_VOCAB = 8194      # speech_head outputs (model.py:340-352)
MASK_ID = 8194           # = V, the extra embedding row
SOS_ID = 6561            # start_speech_token
STOP_ID = 6562           # stop_speech_token
CODEC_V = 6561           # ids < 6561 are codec tokens


@dataclass
class ScoringInputs:
    logits: torch.Tensor      # bf16 [rows, bl, V] (rows = 2*pairs with CFG)
    log_prior: torch.Tensor   # fp32 [V]
    xt: torch.Tensor          # int64 [pairs, bl]
    k_step: torch.Tensor      # int64 [pairs]
    peaks: torch.Tensor       # int64 [pairs, bl] planted argmax ids
    layout: str


def scoring_inputs(*, n_pairs: int, bl: int = 32, vocab: int = SPEECH_VOCAB, seed: int = 0,
                   layout: str = "interleaved", logit_std: float = 3.0, peak: float = 12.0,
                   dirichlet_alpha: float = 0.1, num_steps: int = 10, k_max: int = 8,
                   t_shift: float = 0.5, mask_id: int = MASK_ID, cfg: bool = True,
                   row_pitch: Optional[int] = None, device="cpu") -> ScoringInputs:
    """The CFG + PMI scoring workload: bf16 logits ~ N(0, std) with one planted
    peak per position (the same id in the cond and null rows), a
    Dirichlet(alpha) prior, per-pair step ``k ~ U{0..k_max-1}`` and a block
    whose masked count follows the OmniVoice schedule after ``k`` steps.

    ``row_pitch`` > vocab pads each logit row (a view of ``[..., :vocab]`` is returned).
    """
    g = torch.Generator().manual_seed(seed)
    rows = 2 * n_pairs if cfg else n_pairs
    pitch = row_pitch or vocab
    base = torch.randn(rows, bl, vocab, generator=g) * logit_std
    peaks = torch.randint(0, vocab, (n_pairs, bl), generator=g)
    if cfg:
        if layout == "interleaved":
            cond_rows = torch.arange(n_pairs) * 2
            null_rows = cond_rows + 1
        elif layout == "stacked":
            cond_rows = torch.arange(n_pairs)
            null_rows = cond_rows + n_pairs
        else:
            raise ValueError(layout)
        for rows_idx in (cond_rows, null_rows):
            base[rows_idx[:, None], torch.arange(bl)[None, :], peaks] += peak
    else:
        base[torch.arange(n_pairs)[:, None], torch.arange(bl)[None, :], peaks] += peak
    buf = torch.zeros(rows, bl, pitch, dtype=torch.bfloat16)
    buf[..., :vocab] = base.to(torch.bfloat16)
    rng = np.random.default_rng(seed)
    prior = torch.from_numpy(rng.dirichlet(np.full(vocab, dirichlet_alpha))).float()
    log_prior = prior.clamp_min(1e-8).log()
    k_step = torch.randint(0, k_max, (n_pairs,), generator=g)
    sched = omnivoice_unmask_schedule(bl, num_steps, t_shift)
    xt = torch.randint(0, CODEC_V, (n_pairs, bl), generator=g)
    for p in range(n_pairs):
        n_masked = bl - sum(sched[: int(k_step[p])])
        perm = torch.randperm(bl, generator=g)[:n_masked]
        xt[p, perm] = mask_id
    logits = buf.to(device)[..., :vocab]
    return ScoringInputs(logits, log_prior.to(device), xt.to(device), k_step.to(device),
                         peaks.to(device), layout)


def split_cond_null(logits: torch.Tensor, n_pairs: int, layout: str):
    """Cond/null logit views ``[pairs, bl, V]`` for either CFG row layout."""
    if layout == "interleaved":
        return logits[0::2], logits[1::2]
    return logits[:n_pairs], logits[n_pairs: 2 * n_pairs]


def uniform_lengths(n: int, lo: int, hi: int, seed: int) -> List[int]:
    g = torch.Generator().manual_seed(seed)
    return torch.randint(lo, hi + 1, (n,), generator=g).tolist()


def log_uniform_lengths(n: int, lo: int, hi: int, seed: int) -> List[int]:
    g = torch.Generator().manual_seed(seed)
    u = torch.rand(n, generator=g, dtype=torch.float64)
    return [int(round(math.exp(math.log(lo) + float(x) * (math.log(hi) - math.log(lo))))) for x in u]


# --------------------------------------------------------------------------- #
# Synthetic T3 backbone
# --------------------------------------------------------------------------- #

class SyntheticT3(torch.nn.Module):
    """T3-shaped model: ``tfmr`` (a transformers ``LlamaModel``), ``speech_head``
    (bias-free Linear D -> V) and ``speech_emb`` (V + 1 rows: the extra row is
    MASK, chatterbox_flash/model.py:340-352)."""

    def __init__(self, tfmr, speech_head, speech_emb, speech_pos_emb=None):
        super().__init__()
        self.tfmr = tfmr
        self.speech_head = speech_head
        self.speech_emb = speech_emb
        self.hp = types.SimpleNamespace(input_pos_emb="learned" if speech_pos_emb is not None else None)
        if speech_pos_emb is not None:
            self.speech_pos_emb = speech_pos_emb

    @property
    def device(self) -> torch.device:
        return self.tfmr.norm.weight.device

    def _embed_speech_tokens(self, tokens: torch.Tensor) -> torch.Tensor:
        """chatterbox_flash/model.py:397-402: the token rows, plus the learned
        position embedding when ``hp.input_pos_emb == "learned"``."""
        emb = self.speech_emb(tokens)
        if self.hp.input_pos_emb == "learned":
            emb = emb + self.speech_pos_emb(tokens)
        return emb

    embed_speech_tokens = _embed_speech_tokens


class LearnedPositions(torch.nn.Module):
    """Learned position table with chatterbox-tts's call convention (the
    ``speech_pos_emb`` that model.py:401 adds): ``forward(tokens [B, n])`` returns
    the rows of positions ``0 .. n-1`` -- positions inside the tensor passed,
    whatever the tokens are.  chatterbox-tts 0.1.7 is not installed here, so
    this convention is restated from its published module, not checked
    against it."""

    def __init__(self, n_positions: int, dim: int, device=None, dtype=None):
        super().__init__()
        self.emb = torch.nn.Embedding(n_positions, dim, device=device, dtype=dtype)

    def forward(self, tokens: torch.Tensor) -> torch.Tensor:
        return self.emb(torch.arange(tokens.shape[1], device=tokens.device))


def make_t3(*, n_layers: int = 30, hidden: int = 1024, heads: int = 16, ffn: int = 4096,
            vocab: int = SPEECH_VOCAB, rope_theta: float = 10000.0, rope_parameters: Optional[dict] = None,
            eps: float = 1e-5, max_positions: int = 8192, seed: int = 0, dtype=torch.bfloat16, device="cpu",
            norm_jitter: bool = False, weight_std: float = 0.02, learned_pos_emb: bool = False) -> SyntheticT3:
    """Random-init T3 backbone with a fixed draw order.

    Per layer, in order: q, k, v, o, gate, up, down ~ N(0, weight_std); then
    (if ``norm_jitter``) input/post-attention RMSNorm gains ~ U(0.5, 1.5),
    else 1 (HF init).  Then the final-norm gain (same rule), speech head
    ~ N(0, weight_std) and speech embeddings ~ N(0, 1); with ``learned_pos_emb``
    last a learned speech position table (``max_positions`` rows) ~ N(0, 0.02).
    """
    from transformers import LlamaConfig, LlamaModel
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding

    kw = dict(hidden_size=hidden, intermediate_size=ffn, num_hidden_layers=n_layers, num_attention_heads=heads,
              num_key_value_heads=heads, head_dim=hidden // heads, rms_norm_eps=eps, vocab_size=8,
              max_position_embeddings=max_positions, attn_implementation="sdpa")
    if rope_parameters is None:
        kw["rope_theta"] = rope_theta
    else:
        kw["rope_parameters"] = dict(rope_parameters)
    cfg = LlamaConfig(**kw)
    with torch.device("meta"):
        tf = LlamaModel(cfg)
    tf = tf.to_empty(device=device).to(dtype)
    g = torch.Generator().manual_seed(seed)

    def normal(shape, std):
        return (torch.randn(*shape, generator=g) * std).to(dtype)

    def gain(n):
        return (torch.rand(n, generator=g) + 0.5).to(dtype) if norm_jitter else torch.ones(n, dtype=dtype)

    hd = hidden // heads
    with torch.no_grad():
        for lyr in tf.layers:
            a, m = lyr.self_attn, lyr.mlp
            a.q_proj.weight.copy_(normal((heads * hd, hidden), weight_std))
            a.k_proj.weight.copy_(normal((heads * hd, hidden), weight_std))
            a.v_proj.weight.copy_(normal((heads * hd, hidden), weight_std))
            a.o_proj.weight.copy_(normal((hidden, heads * hd), weight_std))
            m.gate_proj.weight.copy_(normal((ffn, hidden), weight_std))
            m.up_proj.weight.copy_(normal((ffn, hidden), weight_std))
            m.down_proj.weight.copy_(normal((hidden, ffn), weight_std))
            lyr.input_layernorm.weight.copy_(gain(hidden))
            lyr.post_attention_layernorm.weight.copy_(gain(hidden))
        tf.norm.weight.copy_(gain(hidden))
        tf.embed_tokens.weight.zero_()
        tf.rotary_emb = LlamaRotaryEmbedding(config=cfg).to(device)  # fp32 inv_freq
        head = torch.nn.Linear(hidden, vocab, bias=False, device=device, dtype=dtype)
        head.weight.copy_(normal((vocab, hidden), weight_std))
        emb = torch.nn.Embedding(vocab + 1, hidden, device=device, dtype=dtype)
        emb.weight.copy_(normal((vocab + 1, hidden), 1.0))
        pos = None
        if learned_pos_emb:
            pos = LearnedPositions(max_positions, hidden, device=device, dtype=dtype)
            pos.emb.weight.copy_(normal((max_positions, hidden), 0.02))
    return SyntheticT3(tf, head, emb, pos).eval()


class _TableFlow:
    """Token -> "mel" stand-in: frames 2t and 2t + 1 carry token t's id in channel 0."""

    def __init__(self, n_mels: int = 80):
        self.n_mels = n_mels

    def inference(self, *, token, token_len, prompt_token, prompt_token_len, prompt_feat, prompt_feat_len,
                  embedding, finalize, n_timesteps, meanflow):
        B, T = token.shape
        mels = torch.zeros(B, self.n_mels, 2 * T, dtype=torch.float32, device=token.device)
        mels[:, 0, :] = token.float().repeat_interleave(2, dim=1)
        return mels, None


class _TableHift:
    """Mel -> waveform stand-in: each token's 960 samples are row `token` of a fixed table."""

    def __init__(self, table: torch.Tensor):
        self.table = table  # [V, 960] fp32

    def inference(self, *, speech_feat, cache_source):
        tok = speech_feat[:, 0, 0::2].long()  # [B, T]
        B, T = tok.shape
        return self.table.to(speech_feat.device)[tok].reshape(B, T * self.table.shape[1]), None


class TableS3Gen:
    """An S3Gen stand-in whose audio is position-local and exact: token t always yields the same
    960 samples (a seeded table, amplitude up to ~1.2 so clipping is exercised), whatever its
    neighbours.  Vocoding any window of a token sequence therefore gives exactly the slice of one
    vocode of the whole sequence, which makes chunked streaming checkable against a one-shot
    render.  ``trim_fade`` has the shape of S3Gen's (20 ms of zeros, then a 20 ms raised-cosine
    ramp at 24 kHz)."""

    def __init__(self, vocab: int = 6561, seed: int = 0, device: str = "cpu"):
        g = torch.Generator().manual_seed(seed)
        self.table = (torch.rand(vocab, 960, generator=g) * 2.4 - 1.2).to(device)
        self.dtype = torch.float32
        self.flow = _TableFlow()
        self.mel2wav = _TableHift(self.table)
        n = 480
        ramp = (torch.cos(torch.linspace(math.pi, 0.0, n)) + 1) / 2
        self.trim_fade = torch.cat([torch.zeros(n), ramp])

    @staticmethod
    def ref_dict() -> dict:
        return dict(prompt_token=torch.zeros(1, 4, dtype=torch.long), prompt_token_len=torch.tensor([4]),
                    prompt_feat=torch.zeros(1, 8, 80), embedding=torch.zeros(1, 192))

    def render(self, tokens) -> np.ndarray:
        """One vocode of the whole token sequence, fp32 numpy (what the table gives)."""
        return self.table.cpu()[torch.as_tensor(list(tokens), dtype=torch.long)].reshape(-1).numpy()
