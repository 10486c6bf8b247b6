"""``HipEngine``: the MI355X (gfx950) block-diffusion engine.

Implements the engine protocol of chatterbox_flash/engines/base.py:42-141 as
a drop-in next to FlashInferEngine (engines/flashinfer.py:56-1563):

* paged KV per layer (any page table; static per-row slices by default, as
  engines/flashinfer.py:104-116), bf16, written by the fused QKV epilogue;
* ``block_forward`` = one native call (``yapd_t3_block_forward``) running the
  30 decoder layers and the final norm on the caller's stream;
* ``capture_cuda_graph`` captures that call plus the token-shifted speech
  head in a HIP graph (engines/flashinfer.py:1147-1310); ``block_forward_graph``
  replays it and returns views of persistent buffers
  (engines/flashinfer.py:1477-1563);
* ``prefix_forward`` prefills the conditioning prefix with the same kernels,
  causally, in packed steps of 64-token segments (engines/flashinfer.py:678-854
  does it with a ragged FlashInfer prefill).

Only bf16 is supported (the deployed dtype); other dtypes raise ValueError.
"""

from __future__ import annotations

import ctypes
import logging
import math
import os
from typing import Dict, List, Optional, Tuple, Union

import numpy as np
import torch
from torch import Tensor

from .. import kernels
from ..paged import PAGE_SIZE, AttnPlan, PagedKV, copy_from_host_async, to_device_async

logger = logging.getLogger(__name__)

CacheStarts = Union[int, List[int]]
PREFILL_CHUNK = 64      # tokens per prefill segment (the attention kernel's query limit)
# Tokens per prefill step: 16384 rows fill the o/down GEMM grids in one round of 256 x 256 tiles
# (the step's own shape); measured on the 512-row prefill: 8192 285.8 ms, 12288 267.6, 16384 241.2,
# 20480 266.6, 24576 257.8, 32768 241.9, 65536 249.7, 262144 255.3 (64-token chunk steps: 276-280).
PREFILL_TOKENS = 16384


class _Buffers:
    """Per-(rows, bl) activations; persistent so a captured graph can replay."""

    def __init__(self, rows: int, bl: int, D: int, H: int, F: int, dev: torch.device):
        N = rows * bl
        bf = torch.bfloat16
        self.rows, self.bl = rows, bl
        self.emb = torch.zeros(N, D, dtype=bf, device=dev)
        self.residual = torch.empty(N, D, dtype=bf, device=dev)
        self.q = torch.empty(N, H * 64, dtype=bf, device=dev)
        self.attn = torch.empty(N, H * 64, dtype=bf, device=dev)
        self.normed = torch.empty(N, D, dtype=bf, device=dev)
        self.delta = torch.empty(N, D, dtype=bf, device=dev)
        self.act = torch.empty(N, F, dtype=bf, device=dev)
        self.hidden = torch.empty(N, D, dtype=bf, device=dev)
        self.pos0 = torch.zeros(rows, dtype=torch.int32, device=dev)


def _quant_bits_from(quant_bits: Optional[int]) -> int:
    """0 (bf16 weights), 4 or 8.  Unset: ``CHATTERBOX_FLASH_MLX_QUANT_BITS`` as the Metal engine reads it
    (engines/mlx.py:224-235: an unparsable value, or a width it does not quantise to, is ignored with a
    warning); the widths it accepts but this engine does not build (2, 3, 6) raise, as does a group size
    other than 64."""
    if quant_bits is None:
        raw = os.environ.get("CHATTERBOX_FLASH_MLX_QUANT_BITS", "").strip()
        if not raw:
            return 0
        try:
            quant_bits = int(raw)
        except ValueError:
            logger.warning("Ignoring invalid CHATTERBOX_FLASH_MLX_QUANT_BITS=%r", raw)
            return 0
        if quant_bits not in (2, 3, 4, 6, 8):
            logger.warning("Unsupported MLX quant bits=%d; skipping.", quant_bits)
            return 0
        group = int(os.environ.get("CHATTERBOX_FLASH_MLX_QUANT_GROUP", "64"))
        if group != 64:
            raise ValueError(f"HipEngine quantises with group size 64; got CHATTERBOX_FLASH_MLX_QUANT_GROUP={group}")
    if quant_bits not in (0, 4, 8):
        raise ValueError(f"HipEngine quantises to 4 or 8 bits; got {quant_bits}")
    return int(quant_bits)


class HipEngine:
    """Paged-KV engine on hand-written gfx950 kernels (``backend="hip"``)."""

    def __init__(self, model, max_seq_len: int, dtype: torch.dtype, *, batch_size: int = 1,
                 page_size: int = 16, page_table_seed: Optional[int] = None, attn_target_items: int = 192,
                 quant_bits: Optional[int] = None):
        """``quant_bits`` 4 or 8 runs every layer projection on affine group-quantised weights (MLX
        layout, group 64; engines/mlx.py:221-255); ``None`` takes ``CHATTERBOX_FLASH_MLX_QUANT_BITS``
        from the environment as the reference's Metal engine does (unset: bf16 weights)."""
        if dtype != torch.bfloat16:
            raise ValueError(f"HipEngine runs bf16 only; got {dtype}")
        if page_size != PAGE_SIZE:
            raise ValueError(f"HipEngine uses {PAGE_SIZE}-token pages; got page_size={page_size}")
        kernels.load_library()
        tf = model.tfmr
        cfg = tf.config
        dev = torch.device(getattr(model, "device", tf.norm.weight.device))
        if dev.type != "cuda":
            raise ValueError("HipEngine needs the model on a GPU")
        H = cfg.num_attention_heads
        Hkv = cfg.num_key_value_heads
        hd = getattr(cfg, "head_dim", None) or cfg.hidden_size // H
        D = cfg.hidden_size
        if Hkv != H or hd != 64 or H % 4 != 0 or D % 512 != 0:
            raise ValueError(f"HipEngine needs n_kv == n_heads, head_dim 64, heads % 4 == 0, hidden % 512 == 0 "
                             f"(got H={H}, Hkv={Hkv}, hd={hd}, D={D})")
        self._model = model
        self._device = dev
        self._dtype = dtype
        self._max_seq_len = int(max_seq_len)
        self._batch_size = B = max(1, int(batch_size))
        self._page_size = PAGE_SIZE
        self._num_layers = L = cfg.num_hidden_layers
        self._num_heads = H
        self._hidden = D
        self._attn_target = int(attn_target_items)
        self._quant_bits = _quant_bits_from(quant_bits)

        # ---- weights: fused / re-laid-out copies (engines/flashinfer.py:152-187) ----
        self._w: List[Dict[str, Tensor]] = []
        with torch.no_grad():
            for lyr in tf.layers:
                a, mlp = lyr.self_attn, lyr.mlp
                wqkv = torch.cat([a.q_proj.weight, a.k_proj.weight, a.v_proj.weight], 0).to(dtype).contiguous()
                wgu = kernels.interleave_gate_up(mlp.gate_proj.weight.to(dtype), mlp.up_proj.weight.to(dtype))
                self._w.append(dict(
                    wqkv=wqkv, wo=a.o_proj.weight.to(dtype).contiguous(), wgu=wgu,
                    wd=mlp.down_proj.weight.to(dtype).contiguous(),
                    ln_in=lyr.input_layernorm.weight.to(dtype).contiguous(),
                    ln_post=lyr.post_attention_layernorm.weight.to(dtype).contiguous(),
                    eps_in=float(lyr.input_layernorm.variance_epsilon),
                    eps_post=float(lyr.post_attention_layernorm.variance_epsilon)))
            self._final_norm = tf.norm.weight.to(dtype).contiguous()
            self._final_eps = float(tf.norm.variance_epsilon)
            self._ffn = self._w[0]["wd"].shape[1]
            self._wdq: Optional[Tensor] = None
            if self._quant_bits:
                # Quantise the fused copies row by row (groups of 64 along the input dim,
                # so fusing and interleaving rows commutes with quantising); the bf16
                # copies are dropped.  One layer's dequantised weights (bf16) are the
                # scratch of the dequantise-once route the native step takes at many rows.
                from ..quant import quantize_affine
                for w in self._w:
                    for key in ("wqkv", "wo", "wgu", "wd"):
                        w["q_" + key] = quantize_affine(w[key], self._quant_bits)
                        w[key] = None
                F = self._ffn
                self._wdq = torch.empty(3 * H * 64 * D + D * H * 64 + 2 * F * D + D * F, dtype=dtype, device=dev)
            # RoPE table from the model's own rotary embedding (handles llama3
            # scaling; engines/flashinfer.py:195-255), values of the model dtype.
            dummy = torch.zeros(1, 1, D, device=dev, dtype=dtype)
            cos, sin = tf.rotary_emb(dummy, torch.arange(self._max_seq_len, device=dev).unsqueeze(0))
            self._cos = cos[0].float().contiguous()
            self._sin = sin[0].float().contiguous()
            # The fused qkv kernel reads columns 0..31 only: HF builds the tables
            # as cat(freqs, freqs), so columns d and d + 32 are equal.
            if not (torch.equal(self._cos[:, :32], self._cos[:, 32:])
                    and torch.equal(self._sin[:, :32], self._sin[:, 32:])):
                raise ValueError("rotary table is not in cat(freqs, freqs) layout; the hip qkv kernel needs it")

        # ---- paged KV ----
        self._pages_per_row = math.ceil(self._max_seq_len / PAGE_SIZE)
        self._kv = PagedKV(n_layers=L, n_rows=B, pages_per_row=self._pages_per_row, n_heads=H, device=dev,
                           shuffle_seed=page_table_seed)
        self._cache_lens: List[int] = [0] * B
        self._prefix_lens: List[int] = [0] * B

        # ---- native model descriptor ----
        self._c_layers = (kernels.T3Layer * L)()
        for li, w in enumerate(self._w):
            lay = kernels.T3Layer(
                kernels.ptr(w["wqkv"]), kernels.ptr(w["wo"]), kernels.ptr(w["wgu"]), kernels.ptr(w["wd"]),
                w["ln_in"].data_ptr(), w["ln_post"].data_ptr(), w["eps_in"], w["eps_post"],
                self._kv.pools[li].data_ptr())
            if self._quant_bits:
                lay.qbits = self._quant_bits
                for key, field in (("wqkv", "q_qkv"), ("wo", "q_o"), ("wgu", "q_gate_up"), ("wd", "q_down")):
                    pk, sc, bi = w["q_" + key]
                    setattr(lay, field, kernels.T3QWeight(pk.data_ptr(), sc.data_ptr(), bi.data_ptr()))
            self._c_layers[li] = lay
        self._c_model = kernels.T3Model(
            L, D, H, self._ffn, ctypes.cast(self._c_layers, ctypes.POINTER(kernels.T3Layer)),
            self._final_norm.data_ptr(), self._final_eps, self._cos.data_ptr(), self._sin.data_ptr(),
            self._cos.shape[0], self._kv.n_pages, self._kv.table.data_ptr(), self._kv.table.stride(0),
            self._kv.table.shape[1])

        self._bufs: Dict[Tuple[int, int], _Buffers] = {}
        self._plans: Dict[Tuple, AttnPlan] = {}

        # ---- graph state ----
        self._use_cuda_graph = False
        self._graphs: Dict[bool, torch.cuda.CUDAGraph] = {}  # keyed by "plan splits a row"
        self._g_bl = 0
        self._g_plan: Optional[_GraphPlan] = None
        self._g_cs_key = None
        self._head_w: Optional[Tensor] = None
        self._g_shift_ctx: Optional[Tensor] = None
        self._g_logits_buf: Optional[Tensor] = None
        self._g_logits: Optional[Tensor] = None
        logger.info("HipEngine: layers=%d heads=%d dim=%d batch=%d max_seq=%d pages/row=%d KV=%.2f GiB",
                    L, H, D, B, self._max_seq_len, self._pages_per_row,
                    L * self._kv.bytes_per_layer / 2 ** 30)

    # ------------------------------------------------------------------ #
    #  Introspection / lifecycle (engines/base.py:46-67)
    # ------------------------------------------------------------------ #

    @property
    def batch_size(self) -> int:
        return self._batch_size

    @property
    def quant_bits(self) -> int:
        """4 or 8 when the layer projections run on quantised weights, else 0."""
        return self._quant_bits

    @property
    def cache_len(self) -> int:
        return self._cache_lens[0]

    @cache_len.setter
    def cache_len(self, value: int) -> None:
        self._cache_lens = [int(value)] * self._batch_size

    @property
    def cache_lens(self) -> List[int]:
        return self._cache_lens

    @property
    def prefix_lens(self) -> List[int]:
        return self._prefix_lens

    @property
    def has_cuda_graph(self) -> bool:
        return self._use_cuda_graph

    @property
    def kv(self) -> PagedKV:
        return self._kv

    def reset(self) -> None:
        self._cache_lens = [0] * self._batch_size
        self._prefix_lens = [0] * self._batch_size
        self._g_cs_key = None

    def can_reuse(self, max_seq_len: int, dtype: torch.dtype, *, batch_size: int = 1, page_size: int = 16) -> bool:
        return (self._max_seq_len >= max_seq_len and self._dtype == dtype
                and self._batch_size == max(1, batch_size) and self._page_size == page_size)

    def advance_cache(self, block_len: int) -> None:
        for bi in range(self._batch_size):
            self._cache_lens[bi] += int(block_len)

    # ------------------------------------------------------------------ #
    #  Native forward
    # ------------------------------------------------------------------ #

    def _buffers(self, rows: int, bl: int) -> _Buffers:
        key = (rows, bl)
        if key not in self._bufs:
            self._bufs[key] = _Buffers(rows, bl, self._hidden, self._num_heads, self._ffn, self._device)
        return self._bufs[key]

    def _plan(self, kv_len: List[int], bl: int) -> AttnPlan:
        key = (tuple(kv_len), bl)
        plan = self._plans.get(key)
        if plan is None:
            if len(self._plans) > 64:
                self._plans.clear()
            plan = AttnPlan(kv_len, bl, self._num_heads, self._device, target_items=self._attn_target)
            self._plans[key] = plan
        return plan

    def _starts(self, cache_starts: CacheStarts, rows: int) -> List[int]:
        starts = [int(cache_starts)] * rows if isinstance(cache_starts, int) else [int(c) for c in cache_starts]
        if len(starts) != rows:
            raise ValueError(f"cache_starts has {len(starts)} entries for {rows} rows")
        return starts

    def _check_capacity(self, starts: List[int], bl: int) -> None:
        if max(starts) + bl > min(self._max_seq_len, self._pages_per_row * PAGE_SIZE):
            raise ValueError(f"block [{max(starts)}, {max(starts) + bl}) exceeds max_seq_len {self._max_seq_len}")
        if min(starts) < 0:
            raise ValueError("negative cache start")

    def _workspace(self, buf: _Buffers, plan: "AttnPlan | _GraphPlan", merge: bool = True) -> kernels.T3Workspace:
        n_merge = 0 if plan.merge is None or not merge else int(plan.merge.shape[0])
        return kernels.T3Workspace(
            buf.residual.data_ptr(), buf.q.data_ptr(), buf.attn.data_ptr(), buf.normed.data_ptr(),
            buf.delta.data_ptr(), buf.act.data_ptr(), plan.work.data_ptr(), int(plan.work.shape[0]),
            kernels.ptr(plan.merge), n_merge,
            kernels.ptr(getattr(plan, "counts", None)), kernels.ptr(plan.part_o), kernels.ptr(plan.part_ml),
            int(plan.n_slots), kernels.ptr(self._wdq), 0 if self._wdq is None else self._wdq.numel())

    def _descriptor(self, row0: int, table: Optional[Tensor] = None) -> "kernels.T3Model":
        """The native model descriptor whose batch row 0 is page-table row ``row0``, or whose
        rows are those of ``table`` (page-table rows gathered for a subset of the batch)."""
        if table is None and row0 == 0:
            return self._c_model
        m = kernels.T3Model.from_buffer_copy(self._c_model)
        if table is not None:
            m.page_table = table.data_ptr()
            m.table_stride = table.stride(0)
        else:
            m.page_table = self._kv.table.data_ptr() + row0 * self._kv.table.stride(0) * self._kv.table.element_size()
        return m

    def _run(self, buf: _Buffers, plan, kv_len_dev: Tensor, *, causal: bool = False,
             head_w: Optional[Tensor] = None, shift_ctx: Optional[Tensor] = None,
             logits: Optional[Tensor] = None, row0: int = 0, table: Optional[Tensor] = None,
             merge: bool = True) -> None:
        """``merge=False`` leaves out the split-KV merge launch (only for a plan that splits no row)."""
        ws = self._workspace(buf, plan, merge)
        V = 0 if head_w is None else int(head_w.shape[0])
        c_model = self._descriptor(row0, table)
        kernels.check(kernels.load_library().yapd_t3_block_forward(
            ctypes.byref(c_model), ctypes.byref(ws), buf.emb.data_ptr(), buf.rows, buf.bl,
            buf.pos0.data_ptr(), kv_len_dev.data_ptr(), int(causal), buf.hidden.data_ptr(),
            kernels.ptr(head_w), V, kernels.ptr(shift_ctx), kernels.ptr(logits),
            0 if logits is None else logits.stride(1), kernels.stream_ptr(self._device)))

    # ------------------------------------------------------------------ #
    #  Prefix forward (engines/base.py:71-83)
    # ------------------------------------------------------------------ #

    def prefix_forward(self, prefix_emb_or_list: Union[Tensor, List[Tensor]]) -> Tensor:
        """Prefill each row's prefix causally; returns the SOS hidden ``(B, 1, D)``."""
        B = self._batch_size
        D = self._hidden
        if isinstance(prefix_emb_or_list, list):
            embs = [e.reshape(-1, D) for e in prefix_emb_or_list]
            if len(embs) == 1 and B > 1:
                embs = embs * B
            if len(embs) != B:
                raise ValueError(f"prefix list length {len(embs)} != engine batch {B}")
        else:
            t = prefix_emb_or_list
            if t.size(0) not in (1, B):
                raise ValueError(f"prefix batch {t.size(0)} must be 1 or engine batch {B}")
            embs = [t[min(i, t.size(0) - 1)] for i in range(B)]
        sos = self._prefill(0, embs)
        lps = [int(e.shape[0]) for e in embs]
        self._cache_lens = list(lps)
        self._prefix_lens = list(lps)
        return sos

    def prefix_forward_rows(self, row0: int, embs: List[Tensor]) -> Tensor:
        """Prefill only rows ``[row0, row0 + len(embs))`` (their KV pages); the other rows and
        their caches are untouched.  Returns those rows' SOS hidden ``(n, 1, D)``."""
        n = len(embs)
        if not 1 <= n or row0 < 0 or row0 + n > self._batch_size:
            raise ValueError(f"rows [{row0}, {row0 + n}) outside the engine batch {self._batch_size}")
        embs = [e.reshape(-1, self._hidden) for e in embs]
        sos = self._prefill(row0, embs)
        for i, e in enumerate(embs):
            self._cache_lens[row0 + i] = self._prefix_lens[row0 + i] = int(e.shape[0])
        return sos

    def _prefill(self, row0: int, embs: List[Tensor]) -> Tensor:
        """Causal forward of ragged prefixes on batch rows row0.. in steps of up to
        ``PREFILL_TOKENS`` tokens (``yapd_t3_prefill_packed``).  A step's rows are segments of
        at most 64 consecutive tokens of one prefix (the attention kernel's query limit),
        packed back to back: the prefixes are cut into segments in order and the segments
        into steps, so a step may hold several consecutive segments of one prefix -- the QKV
        launch writes all of the step's keys before the attention launch reads them, and causal
        masking orders them -- and no token of padding is computed."""
        n, D = len(embs), self._hidden
        lps = np.array([int(e.shape[0]) for e in embs], dtype=np.int64)
        if lps.min() < 1 or lps.max() > self._max_seq_len:
            raise ValueError("prefix length must be in [1, max_seq_len]")
        dev, dt = self._device, self._dtype
        flat = torch.cat([e.to(device=dev, dtype=dt) for e in embs])  # the prefixes back to back
        offs = np.concatenate([[0], np.cumsum(lps)[:-1]])
        # segments in prefix order: (prefix, first position, token count)
        n_seg = (lps + PREFILL_CHUNK - 1) // PREFILL_CHUNK
        seg_row = np.repeat(np.arange(n), n_seg)
        seg_pos = (np.arange(int(n_seg.sum())) - np.repeat(np.cumsum(n_seg) - n_seg, n_seg)) * PREFILL_CHUNK
        seg_cnt = np.minimum(PREFILL_CHUNK, lps[seg_row] - seg_pos)
        seg_end = np.cumsum(seg_cnt)
        # activations for the largest step, in power-of-two row counts so few sizes are cached
        need = min(PREFILL_TOKENS, int(seg_end[-1]))
        buf = self._buffers(1 << max(0, math.ceil(math.log2(-(-need // PREFILL_CHUNK)))), PREFILL_CHUNK)
        sos = torch.empty(n, 1, D, dtype=dt, device=dev)
        s0 = 0
        while s0 < len(seg_row):
            # the next segments up to the token budget (at least one)
            base = seg_end[s0 - 1] if s0 else 0
            s1 = max(s0 + 1, int(np.searchsorted(seg_end, base + PREFILL_TOKENS, side="right")))
            rows, pos, cnt = seg_row[s0:s1], seg_pos[s0:s1], seg_cnt[s0:s1]
            row_start = np.concatenate([[0], np.cumsum(cnt)])
            T = int(row_start[-1])
            tok_row = np.repeat(np.arange(s1 - s0), cnt)
            tok_src = offs[rows][tok_row] + pos[tok_row] + (np.arange(T) - row_start[tok_row])
            torch.index_select(flat, 0, to_device_async(tok_src, torch.long, dev), out=buf.emb[:T])
            table = self._kv.table[to_device_async(rows + row0, torch.long, dev)]
            pos0 = to_device_async(pos, torch.int32, dev)
            plan = self._plan([int(p + c) for p, c in zip(pos, cnt)], PREFILL_CHUNK)
            ws = self._workspace(buf, plan)
            row_start_dev = to_device_async(row_start, torch.int32, dev)
            tok_row_dev = to_device_async(tok_row, torch.int32, dev)
            kernels.check(kernels.load_library().yapd_t3_prefill_packed(
                ctypes.byref(self._descriptor(row0, table)), ctypes.byref(ws), buf.emb.data_ptr(), T, s1 - s0,
                PREFILL_CHUNK, row_start_dev.data_ptr(), tok_row_dev.data_ptr(), pos0.data_ptr(),
                plan.kv_len.data_ptr(), buf.hidden.data_ptr(), kernels.stream_ptr(dev)))
            last = np.nonzero(pos + cnt == lps[rows])[0]  # segments holding a prefix's last token
            if len(last):
                src = row_start[last] + cnt[last] - 1
                sos[to_device_async(rows[last], torch.long, dev), 0] = buf.hidden[to_device_async(src, torch.long, dev)]
            s0 = s1
        return sos

    def causal_forward(self, emb: Tensor) -> Tensor:
        """Final-normed hidden of every position of one causal chunk of batch row 0 at positions
        0..n-1 (n <= 64), e.g. the unconditional prior pass of model.py:438-460.  Writes that row's
        KV for those positions."""
        n, D = emb.shape
        if D != self._hidden or not 1 <= n <= PREFILL_CHUNK or n > self._max_seq_len:
            raise ValueError(f"causal_forward needs [n, {self._hidden}] with 1 <= n <= {PREFILL_CHUNK}, "
                             f"n <= max_seq_len; got {tuple(emb.shape)}")
        buf = self._buffers(1, n)
        buf.emb.copy_(emb.to(device=self._device, dtype=self._dtype))
        buf.pos0.fill_(0)
        plan = self._plan([n], n)
        self._run(buf, plan, plan.kv_len, causal=True)
        return buf.hidden.view(n, D).clone()

    # ------------------------------------------------------------------ #
    #  Block forward (engines/base.py:85-98)
    # ------------------------------------------------------------------ #

    def block_forward(self, block_emb: Tensor, cache_starts: CacheStarts) -> Tensor:
        """Eager block forward; writes the block KV tentatively at ``[cs, cs+bl)``."""
        B, bl, D = block_emb.shape
        if B != self._batch_size or D != self._hidden:
            raise ValueError(f"block_emb must be ({self._batch_size}, bl, {self._hidden}); got {tuple(block_emb.shape)}")
        if not 1 <= bl <= 64:
            raise ValueError("block length must be in [1, 64]")
        starts = self._starts(cache_starts, B)
        self._check_capacity(starts, bl)
        buf = self._buffers(B, bl)
        buf.emb.copy_(block_emb.reshape(B * bl, D))
        copy_from_host_async(buf.pos0, starts)
        plan = self._plan([s + bl for s in starts], bl)
        self._run(buf, plan, plan.kv_len)
        return buf.hidden.view(B, bl, D).clone()

    def layer_forward(self, li: int, x: Tensor, cache_starts: CacheStarts) -> Dict[str, Tensor]:
        """Run decoder layer ``li`` alone on the residual stream ``x [B, bl, D]`` entering it
        (teacher forcing: any input, e.g. what this engine's layer ``li-1`` produced): the same
        native block forward with a one-layer model descriptor.  Returns the layer's rotated
        queries ``q [B, bl, H, 64]``, its attention output ``attn [B, bl, H*64]``, the
        ``residual`` leaving it and that residual normed by the next layer's input norm
        (``hidden``; the final norm after the last layer).  Writes layer ``li``'s block KV at
        ``[cs, cs+bl)``."""
        B, bl, D = x.shape
        if not 0 <= li < self._num_layers:
            raise ValueError(f"layer {li} outside [0, {self._num_layers})")
        if B != self._batch_size or D != self._hidden or not 1 <= bl <= 64:
            raise ValueError(f"x must be ({self._batch_size}, 1..64, {self._hidden}); got {tuple(x.shape)}")
        starts = self._starts(cache_starts, B)
        self._check_capacity(starts, bl)
        m = kernels.T3Model.from_buffer_copy(self._c_model)
        m.n_layers = 1
        m.layers = ctypes.pointer(self._c_layers[li])
        if li + 1 < self._num_layers:
            m.final_norm = self._w[li + 1]["ln_in"].data_ptr()
            m.final_eps = self._w[li + 1]["eps_in"]
        buf = self._buffers(B, bl)
        buf.emb.copy_(x.reshape(B * bl, D))
        copy_from_host_async(buf.pos0, starts)
        plan = self._plan([s + bl for s in starts], bl)
        ws = self._workspace(buf, plan)
        kernels.check(kernels.load_library().yapd_t3_block_forward(
            ctypes.byref(m), ctypes.byref(ws), buf.emb.data_ptr(), B, bl, buf.pos0.data_ptr(),
            plan.kv_len.data_ptr(), 0, buf.hidden.data_ptr(), None, 0, None, None, 0,
            kernels.stream_ptr(self._device)))
        return dict(q=buf.q.view(B, bl, self._num_heads, 64).clone(), attn=buf.attn.view(B, bl, -1).clone(),
                    residual=buf.residual.view(B, bl, D).clone(), hidden=buf.hidden.view(B, bl, D).clone())

    # ------------------------------------------------------------------ #
    #  Graph path (engines/base.py:100-113, 119-141)
    # ------------------------------------------------------------------ #

    def set_shift_ctx(self, ctx: Tensor) -> None:
        if self._g_shift_ctx is not None:
            if ctx.size(0) < self._batch_size:
                self._g_shift_ctx.copy_(ctx.expand(self._batch_size, -1, -1))
            else:
                self._g_shift_ctx.copy_(ctx)

    def capture_cuda_graph(self, block_size: int, *, speech_head: Optional[torch.nn.Linear] = None) -> None:
        if self._use_cuda_graph and self._g_bl == block_size:
            return
        B, bl, D = self._batch_size, int(block_size), self._hidden
        buf = self._buffers(B, bl)
        self._g_bl = bl
        self._g_plan = _GraphPlan(B, bl, self._num_heads, self._device, self._attn_target)
        starts = [min(c, self._max_seq_len - bl) for c in self._cache_lens]
        # the new plan and buffers hold nothing yet: refresh them even if the
        # starts equal those of an earlier capture at another block size
        self._g_cs_key = None
        self._update_graph_inputs(starts)
        if speech_head is not None:
            self._head_w = speech_head.weight.detach().to(self._dtype).contiguous()
            if speech_head.bias is not None:
                raise ValueError("HipEngine folds a bias-free speech head (T3 speech_head has no bias)")
            V = self._head_w.shape[0]
            pitch = (V + 7) // 8 * 8  # 16-byte aligned rows
            self._g_shift_ctx = torch.zeros(B, 1, D, dtype=self._dtype, device=self._device)
            self._g_logits_buf = torch.zeros(B, bl, pitch, dtype=self._dtype, device=self._device)
            self._g_logits = self._g_logits_buf[..., :V]
        body = lambda merge: self._run(buf, self._g_plan, self._g_plan.kv_len, head_w=self._head_w,
                                       shift_ctx=self._g_shift_ctx, logits=self._g_logits, merge=merge)
        body(True)  # warm-up outside the graph
        torch.cuda.synchronize(self._device)
        # Two graphs: one with the split-KV merge launch, and one without for
        # plans that split no row (the host knows which when it plans).
        self._graphs = {}
        for merge in (True, False):
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                body(merge)
            self._graphs[merge] = graph
        self._use_cuda_graph = True
        logger.info("HipEngine: graph captured (block=%d, batch=%d, head=%s)", bl, B, self._head_w is not None)

    def _update_graph_inputs(self, starts: List[int]) -> None:
        key = tuple(starts)
        if key == self._g_cs_key:
            return
        bl = self._g_bl
        self._check_capacity(starts, bl)
        buf = self._buffers(self._batch_size, bl)
        copy_from_host_async(buf.pos0, starts)
        self._g_plan.update([s + bl for s in starts])
        self._g_cs_key = key

    def block_forward_graph(self, block_emb: Tensor, cache_starts: CacheStarts) -> Tuple[Tensor, Optional[Tensor]]:
        bl = block_emb.size(1)
        if not self._use_cuda_graph or bl != self._g_bl:
            return self.block_forward(block_emb, cache_starts), None
        B, D = self._batch_size, self._hidden
        buf = self._buffers(B, bl)
        buf.emb.copy_(block_emb.reshape(B * bl, D))
        self._update_graph_inputs(self._starts(cache_starts, B))
        self._graphs[self._g_plan.n_merge_live > 0].replay()
        return buf.hidden.view(B, bl, D), self._g_logits


class _GraphPlan:
    """Attention plan with fixed-capacity device buffers, refreshed in place.

    The captured grid is sized by the capacity; the kernels read the live
    item counts from ``counts``.
    """

    def __init__(self, rows: int, bl: int, n_heads: int, device: torch.device, target_items: int):
        self.rows, self.bl, self.target = rows, bl, target_items
        cap_items = rows + target_items
        self.work = torch.zeros(cap_items, 4, dtype=torch.int32, device=device)
        self.merge = torch.zeros(rows, 3, dtype=torch.int32, device=device)
        self.counts = torch.zeros(2, dtype=torch.int32, device=device)
        self.kv_len = torch.ones(rows, dtype=torch.int32, device=device)
        self.n_slots = cap_items
        self.part_o = torch.empty(cap_items, bl, n_heads, 64, dtype=torch.float32, device=device)
        self.part_ml = torch.empty(cap_items, bl, n_heads, 2, dtype=torch.float32, device=device)
        self.update([bl] * rows)

    def update(self, kv_len: List[int]) -> None:
        work, merge, n_slots = kernels.attn_plan(kv_len, target_items=self.target)
        if work.shape[0] > self.work.shape[0] or n_slots > self.n_slots:
            raise RuntimeError("attention plan exceeds the captured capacity")
        # stream-ordered uploads from pinned staging: no host sync between blocks
        copy_from_host_async(self.work[: work.shape[0]], work)
        if merge.shape[0]:
            copy_from_host_async(self.merge[: merge.shape[0]], merge)
        copy_from_host_async(self.counts, [work.shape[0], merge.shape[0]])
        self.n_merge_live = int(merge.shape[0])  # rows split by the current plan (host copy)
        copy_from_host_async(self.kv_len, kv_len)
