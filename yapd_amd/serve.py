"""Continuous-batching block-diffusion engine on the native step.

The slot scheduler of server/engine.py (``FlashEngine``, :275-663): every tick
runs one batched block-diffusion step over all active requests, each at its
own block, denoise step and sequence position; requests join at tick
boundaries (ragged prefill into free slots) and leave on EOS or when their
speech budget is committed.  The token math is the reference's (OmniVoice
schedule, PMI quantile early decoding, uncond block prior, zero-text CFG with
``(cond_i, null_i)`` rows, Gumbel-max sampling, Gumbel position noise).

Built for the native path rather than translated:

* one tick = block gather + embed (torch glue), the native 30-layer forward
  with the token-shifted head, the CFG/PMI/quantile scorer and the native
  state update (``yapd_tick_update``) -- all stream-ordered, no host sync;
* the per-tick ``flags.cpu()`` of server/engine.py:635 becomes an async copy
  into pinned memory that the host reads ``lag`` ticks later, so the GPU
  never waits for the host; the attention work list is planned from per-row
  upper bounds of the cache length (a row grows by at most one block per
  tick) and the kernel masks by the true device length;
* the KV cache is paged, so retiring a request swaps page-table rows instead
  of copying KV rows (server/engine.py:467-487 copies them).

Admission (prefill) does synchronise once per admitted batch.
"""

from __future__ import annotations

import collections
import time
from dataclasses import dataclass, field
from typing import Deque, List, Optional

import torch

from . import kernels
from .embed import SpeechEmbedder
from .engines.hip import HipEngine
from .paged import PAGE_SIZE, to_device_async
from .scoring import BlockScorer
from .voc_stream import maybe_vocode


@dataclass
class Request:
    """A synthesis request (the T3 part of server/engine.py:49-83).

    ``prefix`` is the row's prefix embedding ``[lp, D]`` (conditioning, text
    and the SOS embedding last) on the engine's device; building it from text
    is host glue of the caller (server/engine.py:378-402).
    """
    rid: int
    prefix: torch.Tensor
    n_speech: int
    priority: int = 0
    # engine state
    slot: int = -1
    lp: int = 0
    cpu_len: int = 0
    known_tick: int = 0
    committed: list = field(default_factory=list)
    t3_done: bool = False
    # streaming audio (server/engine.py:56-57, 67-72, 77-80): sink(bytes | None), None = end of stream
    sink: object = None
    emitted_tok: int = 0      # committed tokens handed to the vocoder
    voc_tail: object = None   # crossfade tail of the last chunk (device tensor)
    voc_tail_ready: object = None  # event recorded after the launch that wrote voc_tail
    first_chunk_sent: bool = False
    finished: bool = False    # audio stream closed
    t_first_pcm: float = 0.0
    audio_samples: int = 0
    # metrics (perf_counter)
    t_recv: float = 0.0
    t_admit: float = 0.0
    t_first_commit: float = 0.0
    t_done: float = 0.0
    n_tokens: int = 0


class _AsyncPlan:
    """Attention plan with fixed-capacity device buffers, refreshed every tick
    from pinned staging buffers (a ring, so a refresh never waits for the GPU).
    The launch grid is the capacity; the kernels read the live counts, and the
    merge launch is left out of a tick whose plan splits no row."""

    def __init__(self, rows: int, bl: int, n_heads: int, device: torch.device, target_items: int, depth: int = 4):
        self.rows, self.bl, self.target = rows, bl, target_items
        cap = rows + target_items
        self.cap = cap
        # work items, merge records and the two counts in one device block, filled by one copy
        self._n = cap * 4 + rows * 3 + 2
        self._blob = torch.zeros(self._n, dtype=torch.int32, device=device)
        self.work, self.merge, self.counts = self._views(self._blob)
        self.n_slots = cap
        self.part_o = torch.empty(cap, bl, n_heads, 64, dtype=torch.float32, device=device)
        self.part_ml = torch.empty(cap, bl, n_heads, 2, dtype=torch.float32, device=device)
        self._stage = [torch.zeros(self._n, dtype=torch.int32).pin_memory() for _ in range(depth)]
        self._events: List[Optional[torch.cuda.Event]] = [None] * depth
        self._next = 0
        self.n_merge_live = 0  # split rows of the current plan (0: the merge launch is left out)

    def _views(self, blob: torch.Tensor):
        """(work [cap, 4], merge [rows, 3], counts [2]) inside one int32 block."""
        w_end = self.cap * 4
        m_end = w_end + self.rows * 3
        return blob[:w_end].view(self.cap, 4), blob[w_end:m_end].view(self.rows, 3), blob[m_end:m_end + 2]

    def update(self, kv_upper: List[int]) -> None:
        work, merge, n_slots = kernels.attn_plan(kv_upper, target_items=self.target)
        if work.shape[0] > self.cap or merge.shape[0] > self.rows or n_slots > self.n_slots:
            raise RuntimeError("attention plan exceeds the engine's capacity")
        self.n_merge_live = int(merge.shape[0])
        i = self._next
        self._next = (i + 1) % len(self._stage)
        if self._events[i] is not None:
            self._events[i].synchronize()  # issued `depth` ticks ago
        blob = self._stage[i]
        w, m, c = self._views(blob)
        w.numpy()[: work.shape[0]] = work
        if merge.shape[0]:
            m.numpy()[: merge.shape[0]] = merge
        c.numpy()[:] = (work.shape[0], merge.shape[0])
        self._blob.copy_(blob, non_blocking=True)  # one copy of the whole block (a few KB)
        ev = torch.cuda.Event()
        ev.record()
        self._events[i] = ev


class HipFlashEngine:
    """Continuous-batching scheduler over :class:`HipEngine` (server/engine.py FlashEngine)."""

    def __init__(self, model, *, log_prior: torch.Tensor, mask_id: int, stop_id: int, codec_vocab: int,
                 max_active: int = 128, max_prefix_tokens: int = 512, max_speech_tokens: int = 624,
                 num_steps: int = 10, temperature: float = 0.6, time_shift_tau: float = 0.1,
                 omnivoice_t_shift: float = 0.5, cfg_scale: float = 1.0, position_temperature: float = 5.0,
                 prefill_max: int = 16, block_size: int = 16, lag: int = 2, seed: int = 1234,
                 page_table_seed: Optional[int] = None, vocoder=None):
        """``vocoder``: a :class:`yapd_amd.voc_stream.Vocoder` (or None); committed tokens are
        handed to it in chunks as they are read back (server/engine.py:211-258)."""
        if block_size % PAGE_SIZE and PAGE_SIZE % block_size:
            raise ValueError("block size must divide or be a multiple of the 16-token page")
        if lag < 1:
            raise ValueError("lag must be >= 1 (results are read back asynchronously)")
        self.dev = torch.device(getattr(model, "device", model.tfmr.norm.weight.device))
        self.BS = int(block_size)
        self.K = int(num_steps)
        self.temp = float(temperature)
        self.posT = float(position_temperature)
        self.cfg = float(cfg_scale)
        self.MASK, self.STOP, self.CODEC_V = int(mask_id), int(stop_id), int(codec_vocab)
        self.nb = 2 if cfg_scale > 0 else 1
        self.S = int(max_active)
        self.N_max = int(max_speech_tokens)
        self.L = int(max_prefix_tokens) + self.N_max + self.BS  # server/engine.py:325
        self.prefill_max = int(prefill_max)
        self.lag = int(lag)
        self.seed = int(seed)
        self.vocoder = vocoder
        S, nb, BS = self.S, self.nb, self.BS

        self.eng = HipEngine(model, self.L, torch.bfloat16, batch_size=S * nb, page_table_seed=page_table_seed)
        D = self.eng._hidden
        self.D = D
        head = model.speech_head
        if head.bias is not None:
            raise ValueError("the speech head must be bias-free (T3's is)")
        self.head_w = head.weight.detach().to(torch.bfloat16).contiguous()
        self.V = int(self.head_w.shape[0])
        self.embed = SpeechEmbedder(model, self.BS, self.dev)
        dev = self.dev

        # ---- per-slot state (server/engine.py:338-345) ----
        self.xt = torch.full((S, self.N_max), self.MASK, dtype=torch.int64, device=dev)
        self.blk_start = torch.zeros(S, dtype=torch.int64, device=dev)
        self.k_step = torch.zeros(S, dtype=torch.int64, device=dev)
        self.cache_len = torch.zeros(S, dtype=torch.int64, device=dev)
        self.n_speech = torch.zeros(S, dtype=torch.int64, device=dev)
        self.is_commit = torch.zeros(S, dtype=torch.uint8, device=dev)
        self.shift_ctx = torch.zeros(S * nb, 1, D, dtype=torch.bfloat16, device=dev)

        # ---- step buffers ----
        pitch = (self.V + 7) // 8 * 8
        self.logits_buf = torch.zeros(S * nb, BS, pitch, dtype=torch.bfloat16, device=dev)
        self.logits = self.logits_buf[..., : self.V]
        self.xt_blk = torch.empty(S, BS, dtype=torch.int64, device=dev)
        self.toks = torch.empty(S * nb * BS, dtype=torch.int64, device=dev)
        self.kv_dev = torch.empty(S * nb, dtype=torch.int32, device=dev)
        self.flags = torch.zeros(S, 6, dtype=torch.int64, device=dev)
        self.xt_final = torch.zeros(S, BS, dtype=torch.int64, device=dev)
        self.ar = torch.arange(BS, device=dev)
        self.scorer = BlockScorer(n_pairs=S, block_size=BS, log_prior=log_prior.to(dev), mask_id=self.MASK,
                                  stop_id=self.STOP, num_steps=self.K, time_shift_tau=time_shift_tau,
                                  omnivoice_t_shift=omnivoice_t_shift, cfg_scale=self.cfg, device=dev)
        self.plan = _AsyncPlan(S * nb, BS, self.eng._num_heads, dev, self.eng._attn_target)

        # ---- asynchronous result read-back: a ring of pinned buffers ----
        depth = self.lag + 1
        self._res = [(torch.zeros(S, 6, dtype=torch.int64).pin_memory(),
                      torch.zeros(S, BS, dtype=torch.int64).pin_memory()) for _ in range(depth)]
        self._pending: Deque = collections.deque()  # (ring index, tick id, snapshot of active, event)
        self._ring_next = 0

        self.active: List[Request] = []
        self.waiting: Deque[Request] = collections.deque()
        self.finished: List[Request] = []
        self.tick_id = 0
        self.commit_blocks = 0
        self.tick_time = 0.0

    # ------------------------------------------------------------------ #
    #  Public API
    # ------------------------------------------------------------------ #

    def submit(self, req: Request) -> None:
        if req.n_speech < self.BS or req.n_speech % self.BS or req.n_speech > self.N_max - self.BS:
            raise ValueError(f"n_speech must be a multiple of {self.BS} in [{self.BS}, {self.N_max - self.BS}]")
        lp = int(req.prefix.shape[0])
        if lp < 1 or lp + self.N_max + self.BS > self.L or req.prefix.shape[-1] != self.D:
            raise ValueError(f"prefix must be [1..{self.L - self.N_max - self.BS}, {self.D}]")
        if req.prefix.device != self.dev:
            raise ValueError("prefix must already be on the engine's device")
        req.t_recv = time.perf_counter()
        self.waiting.append(req)

    @property
    def idle(self) -> bool:
        return not self.active and not self.waiting and not self._pending

    def run_until_idle(self, max_ticks: int = 1_000_000) -> None:
        for _ in range(max_ticks):
            if self.idle:
                return
            self.tick()
        raise RuntimeError("engine did not drain within max_ticks")

    def stats(self) -> dict:
        return dict(active=len(self.active), waiting=len(self.waiting), ticks=self.tick_id,
                    avg_tick_ms=round(self.tick_time / max(1, self.tick_id) * 1e3, 3),
                    commit_blocks=self.commit_blocks, finished=len(self.finished))

    # ------------------------------------------------------------------ #
    #  One tick (server/engine.py:624-651)
    # ------------------------------------------------------------------ #

    @torch.inference_mode()
    def tick(self) -> None:
        t0 = time.perf_counter()
        # results of the tick `lag` back are complete by now (the GPU is on the next one)
        while self._pending and (len(self._pending) >= self.lag or not self.active):
            self._consume(self._pending.popleft())
        self._admit()
        A = len(self.active)
        if A == 0:
            return
        # cache lengths can have grown by one block per tick not yet read back
        nb, BS = self.nb, self.BS
        ub = [min(r.cpu_len + BS * (self.tick_id - r.known_tick), self.L - BS) for r in self.active]
        self.plan.update([u + BS for u in ub for _ in range(nb)])
        self._step_gpu(A)
        i = self._ring_next
        self._ring_next = (i + 1) % len(self._res)
        hf, hx = self._res[i]
        hf[:A].copy_(self.flags[:A], non_blocking=True)
        hx[:A].copy_(self.xt_final[:A], non_blocking=True)
        ev = torch.cuda.Event()
        ev.record()
        self._pending.append((i, self.tick_id, list(self.active), ev))
        self.tick_id += 1
        self.tick_time += time.perf_counter() - t0

    def _step_gpu(self, A: int) -> None:
        """One batched step over slots [0, A) (server/engine.py:491-622), stream-ordered."""
        nb, BS = self.nb, self.BS
        R = A * nb
        xt_blk = self.xt_blk[:A]
        torch.gather(self.xt[:A], 1, self.blk_start[:A, None] + self.ar, out=xt_blk)
        self.toks[: R * BS].view(A, nb, BS).copy_(xt_blk[:, None, :])
        buf = self.eng._buffers(R, BS)
        self.embed(self.toks[: R * BS], buf.emb)
        buf.pos0.view(A, nb).copy_(self.cache_len[:A, None])
        torch.add(buf.pos0, BS, out=self.kv_dev[:R])
        self.eng._run(buf, self.plan, self.kv_dev[:R], head_w=self.head_w, shift_ctx=self.shift_ctx[:R],
                      logits=self.logits[:R], merge=self.plan.n_merge_live > 0)
        res = self.scorer(self.logits[:R], xt_blk, self.k_step[:A], layout="interleaved" if nb == 2 else "stacked",
                          temperature=self.temp, position_noise=self.posT > 0, seed=self.seed,
                          rng_offset=self.tick_id << 24, n_pairs=A)
        kernels.tick_update(xt=self.xt, xt_blk=xt_blk, xt_new=res.xt, k_step=self.k_step[:A],
                            cache_len=self.cache_len[:A], blk_start=self.blk_start[:A], is_commit=self.is_commit[:A],
                            n_speech=self.n_speech[:A], hidden=buf.hidden, shift_ctx=self.shift_ctx,
                            flags=self.flags[:A], xt_final=self.xt_final[:A], n_branch=nb, K=self.K,
                            mask_id=self.MASK, stop_id=self.STOP, max_len=self.L)

    # ------------------------------------------------------------------ #
    #  Host bookkeeping (server/engine.py:636-656, :208-256)
    # ------------------------------------------------------------------ #

    def _consume(self, item) -> None:
        i, tick, snapshot, ev = item
        ev.synchronize()
        hf, hx = self._res[i]
        flags = hf[: len(snapshot)].numpy()
        xtf = hx[: len(snapshot)].numpy()
        now = time.perf_counter()
        for s, r in enumerate(snapshot):
            if r.t3_done:
                continue  # already retired; this was one of its trailing ticks
            was_commit, _nmask, eos, _k, bstart, nsp = (int(v) for v in flags[s])
            r.known_tick = tick + 1  # the cache length after this tick is known now
            if was_commit:
                r.cpu_len = r.lp + bstart
                self._push(r, xtf[s].tolist(), now)
                self.commit_blocks += 1
                if bstart >= nsp:
                    self._finish(r, now)
            elif eos:
                toks = xtf[s].tolist()
                self._push(r, toks[: toks.index(self.STOP)], now)
                self._finish(r, now)

    def _push(self, r: Request, toks: List[int], now: float) -> None:
        add = [t for t in toks if t < self.CODEC_V]
        if add and not r.committed:
            r.t_first_commit = now
        r.committed.extend(add)
        if self.vocoder is not None:
            maybe_vocode(self.vocoder, r, final=False)

    def _finish(self, r: Request, now: float) -> None:
        r.t3_done = True
        r.t_done = now
        r.n_tokens = len(r.committed)
        self._free_slot(r)
        self.finished.append(r)
        if self.vocoder is not None:
            maybe_vocode(self.vocoder, r, final=True)

    def _free_slot(self, r: Request) -> None:
        """Swap-with-last compaction (server/engine.py:467-487); the KV follows its page-table rows."""
        i, last, nb = r.slot, len(self.active) - 1, self.nb
        if i != last:
            mv = self.active[last]
            for t in (self.blk_start, self.k_step, self.cache_len, self.n_speech, self.is_commit):
                t[i] = t[last]
            self.xt[i] = self.xt[last]
            self.shift_ctx[i * nb:(i + 1) * nb] = self.shift_ctx[last * nb:(last + 1) * nb]
            for b in range(nb):
                self.eng._kv.swap_rows(i * nb + b, last * nb + b)
            mv.slot = i
            self.active[i] = mv
        self.active.pop()
        r.slot = -1

    # ------------------------------------------------------------------ #
    #  Admission / ragged prefill (server/engine.py:404-465)
    # ------------------------------------------------------------------ #

    def _admit(self) -> None:
        free = self.S - len(self.active)
        if free <= 0 or not self.waiting:
            return
        take = sorted(self.waiting, key=lambda q: (q.priority, q.t_recv, q.rid))[: min(free, self.prefill_max)]
        for q in take:
            self.waiting.remove(q)
        nb, base = self.nb, len(self.active)
        embs = []
        for q in take:
            embs.append(q.prefix)
            if nb == 2:  # zero-text null prefix: zeros except the SOS embedding last (server/engine.py:399-401)
                null = torch.zeros_like(q.prefix)
                null[-1] = q.prefix[-1]
                embs.append(null)
        sos = self.eng.prefix_forward_rows(base * nb, embs)
        G = len(take)
        self.shift_ctx[base * nb:(base + G) * nb] = sos
        # the new slots are base..base+G-1: one fill or one upload per state tensor
        sl = slice(base, base + G)
        self.blk_start[sl] = 0
        self.k_step[sl] = 0
        self.is_commit[sl] = 0
        self.xt[sl] = self.MASK
        lps = [int(q.prefix.shape[0]) for q in take]
        self.cache_len[sl] = to_device_async(lps, self.cache_len.dtype, self.dev)
        self.n_speech[sl] = to_device_async([q.n_speech for q in take], self.n_speech.dtype, self.dev)
        now = time.perf_counter()
        for g, q in enumerate(take):
            q.slot, q.lp, q.cpu_len, q.known_tick, q.t_admit = base + g, lps[g], lps[g], self.tick_id, now
            self.active.append(q)
