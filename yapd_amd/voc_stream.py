"""Chunked streaming vocoder: committed speech tokens -> 24 kHz 16-bit PCM.

The micro-batched worker of server/vocoder.py:52-357 behind the same
interface (``Vocoder(s3gen, ref_dict, device, chunk_first=..., chunk=...)``,
``enqueue``, ``finalize_empty``, ``run``, ``stats``), and the engine-side
hand-off of server/engine.py:223-258 (``maybe_vocode``).  A request's
committed tokens are vocoded in windows that reach ``lookback`` tokens back
before the emitted part; windows of all requests are padded into
micro-batches of bucketed width and height and run through S3Gen's flow and
HiFT models together; each chunk's join with the previous one is a 20 ms
linear crossfade over the samples the previous chunk withheld.

Built for the GPU rather than translated:

* the per-chunk post-processing (first-chunk trim fade, crossfade with the
  withheld tail, tail withholding, clip, int16) of a whole micro-batch is one
  launch of ``yapd_voc_stitch`` (voc_stitch.hip); only the int16 PCM crosses
  to the host (half the bytes of the reference's fp32 ``.cpu()``), into
  pinned memory, and the worker thread does no per-sample numpy work while
  the engine thread runs;
* the crossfade tails stay on the device between a request's chunks (a
  numpy tail handed in from another process, as ``send_tail`` does, is
  accepted too);
* the two lanes (first chunks and top-ups, bulk) run on their own streams at
  the default priority: work on streams of different priorities has hung on
  this platform, so the first-chunk lane is favoured by scheduling alone
  (its own thread, its own batches), not by stream priority.

S3Gen itself (``flow.inference``, ``mel2wav.inference``, ``trim_fade``,
``dtype``) is the caller's model; ``yapd_amd.vocoder.install_fused_snake``
puts the fused Snake kernels into its HiFT generator.
"""

from __future__ import annotations

import logging
import sys
import threading
import time
from collections import defaultdict, deque
from dataclasses import dataclass
from typing import Deque, Dict, List, Optional

import numpy as np
import torch

from . import kernels

logger = logging.getLogger(__name__)

SR = 24000
SAMPLES_PER_TOKEN = 960  # 25 tokens/s: 2 mel frames of 480 samples per token
MEL_PER_TOKEN = 2


@dataclass
class VocJob:
    """One chunk of one request (server/vocoder.py:41-49)."""
    req: object
    window: list              # token ids: lookback context + the emitted tokens
    emit_off: int             # tokens of the window before the emit point
    first: bool               # first chunk of the request
    final: bool               # last chunk: close the stream after it
    end_marker: bool = False  # no audio, only close the stream
    deadline: float = float("inf")


def _silence_cfm_progress() -> None:
    """S3Gen's CFM loop prints and wraps every call in tqdm (server/vocoder.py:28-33); when
    chatterbox's flow-matching module is loaded, shadow both at module level."""
    fm = sys.modules.get("chatterbox.models.s3gen.flow_matching")
    if fm is not None:
        fm.tqdm = lambda it, **kw: it
        fm.print = lambda *a, **k: None


def _first_at_least(buckets, n: int) -> int:
    return next((b for b in buckets if b >= n), n)


class Vocoder:
    """Micro-batched chunked-streaming S3Gen vocoder (server/vocoder.py:52-357).

    Knobs and their meaning are the reference's: ``chunk_first`` tokens for a
    request's first chunk, then ``chunk_second`` or the ``topup_sizes`` until
    ``topup_until`` tokens, then ``chunk``; ``lookback`` tokens of left context
    per window; ``fade`` crossfade samples; ``max_batch`` / ``first_max_batch``
    jobs per bulk / first-lane micro-batch; ``pre_roll`` zero samples before a
    stream's audio; ``n_cfm_timesteps`` flow-matching steps.
    """

    B_BUCKETS = (4, 8, 16, 24, 32, 48, 64, 96)
    W_BUCKETS = (4, 8, 12, 13, 15, 16, 20, 21, 24, 28, 32, 36, 40, 44, 52, 60, 64, 68, 76, 80, 84, 96)

    def __init__(self, s3gen, ref_dict: dict, device, *, chunk_first: int = 12, chunk: int = 80,
                 chunk_second: int = 0, topup_sizes: tuple = (), lookback: int = 16, topup_until: int = 0,
                 fade: int = 480, max_batch: int = 48, pre_roll: int = 0, first_max_batch: int = 24,
                 n_cfm_timesteps: int = 1):
        if fade < 1:
            raise ValueError("fade must be >= 1 sample")
        _silence_cfm_progress()
        self.s3gen = s3gen
        self.device = torch.device(device)
        self.dtype = s3gen.dtype
        self.chunk_first, self.chunk, self.chunk_second = chunk_first, chunk, chunk_second
        self.topup_sizes = tuple(topup_sizes)
        self.topup_until = topup_until or (
            chunk_first + (sum(self.topup_sizes) if self.topup_sizes else chunk_second))
        self.lookback, self.fade, self.pre_roll = lookback, fade, pre_roll
        self.max_batch, self.first_max_batch = max_batch, first_max_batch
        self.n_cfm = n_cfm_timesteps

        # the shared voice's conditioning, cast once (floating tensors to the model dtype)
        self.ref = {}
        for k, v in ref_dict.items():
            if torch.is_tensor(v):
                v = v.to(device=self.device)
                if v.dtype.is_floating_point:
                    v = v.to(self.dtype)
            self.ref[k] = v
        self.prompt_token = self.ref["prompt_token"]
        self.prompt_token_len = self.ref["prompt_token_len"]
        self.prompt_feat = self.ref["prompt_feat"]
        self.embedding = self.ref["embedding"]

        # stitch tables on the device: S3Gen's trim fade and the linear crossfade ramps
        # (np.linspace in float32 and one minus it, server/vocoder.py:107-109)
        fin = np.linspace(0.0, 1.0, fade, dtype=np.float32)
        fout = (np.float32(1.0) - fin).astype(np.float32)
        self.trim = s3gen.trim_fade.detach().float().reshape(-1).to(self.device).contiguous()
        self.fade_in = torch.from_numpy(fin).to(self.device)
        self.fade_out = torch.from_numpy(fout).to(self.device)

        self.q: Deque[VocJob] = deque()                       # bulk lane
        self.q_topup: Dict[int, Deque[VocJob]] = defaultdict(deque)  # top-ups, by window width
        self.q_first: Deque[VocJob] = deque()                 # first chunks
        self.topup_last_width = -1
        self.first_streak = 0
        self.lock = threading.Lock()
        self.wake = threading.Event()
        self.wake_first = threading.Event()
        self.stop_flag = False

        self.batches = 0
        self.jobs = 0
        self.gpu_time = 0.0

    # ------------------------------------------------------------------ #
    #  Producer side (engine thread), server/vocoder.py:123-161
    # ------------------------------------------------------------------ #

    def enqueue(self, req, final: bool, n_emit: Optional[int] = None) -> None:
        """Queue the chunk emitting ``req.committed[req.emitted_tok : +n_emit]`` (all of it when
        ``n_emit`` is None)."""
        e_start = req.emitted_tok
        e_end = len(req.committed) if n_emit is None else e_start + n_emit
        first = e_start == 0
        if self.topup_sizes:
            priority = first or e_start == self.chunk_first
        else:
            priority = first or (self.chunk_second > 0 and e_start < self.topup_until)
        width = n_emit if (priority and not first and n_emit) else self.chunk
        w_start = min(0 if first else max(0, e_end - (self.lookback + width)), e_start)
        t0 = getattr(req, "t_recv", 0.0) or time.perf_counter()
        job = VocJob(req=req, window=list(req.committed[w_start:e_end]), emit_off=e_start - w_start, first=first,
                     final=final, deadline=t0 + 0.4 + e_start / 25.0)
        with self.lock:
            if first:
                self.q_first.append(job)
            elif priority:
                self.q_topup[len(job.window)].append(job)
            else:
                self.q.append(job)
        (self.wake_first if priority else self.wake).set()

    def finalize_empty(self, req) -> None:
        """Close a stream that has no audio left (server/vocoder.py:157-160)."""
        with self.lock:
            self.q.append(VocJob(req, [], 0, False, True, end_marker=True))
        self.wake.set()

    # ------------------------------------------------------------------ #
    #  Consumer side (worker threads), server/vocoder.py:165-280
    # ------------------------------------------------------------------ #

    def run(self) -> None:
        """Serve both lanes until ``close()``: the first-chunk lane on a thread of its own, the
        bulk lane on the calling thread, each with its own stream."""
        t = threading.Thread(target=self._run_lane, args=(True,), daemon=True)
        t.start()
        try:
            self._run_lane(False)
        finally:
            t.join()

    def close(self) -> None:
        self.stop_flag = True
        self.wake.set()
        self.wake_first.set()

    def _run_lane(self, priority: bool) -> None:
        stream = torch.cuda.Stream(self.device)  # default priority (see the module docstring)
        wake = self.wake_first if priority else self.wake
        take = self._take_first if priority else self._take_bulk
        with torch.cuda.stream(stream):
            while not self.stop_flag:
                jobs = take()
                if not jobs:
                    wake.wait(timeout=0.005)
                    wake.clear()
                    continue
                try:
                    self._process(jobs)
                except Exception:
                    logger.exception("vocoder batch failed; closing %d streams", len(jobs))
                    for j in jobs:
                        self._emit(j.req, None)

    def _pick_first_source(self):
        """(queue, width, from_first) the first-chunk lane serves next: first chunks, except that
        after three first-chunk batches in a row a pending top-up width gets a turn; top-up
        widths rotate upwards (server/vocoder.py:187-196)."""
        widths = sorted(w for w, dq in self.q_topup.items() if dq)
        width = next((w for w in widths if w > self.topup_last_width), widths[0] if widths else None)
        use_first = bool(self.q_first) and (not widths or self.first_streak < 3)
        src = self.q_first if use_first else (self.q_topup[width] if width is not None else self.q_first)
        return src, width, use_first

    def _take_first(self) -> List[VocJob]:
        with self.lock:
            src, _, _ = self._pick_first_source()
            n = len(src)
        if 0 < n < 4:
            time.sleep(0.006)  # a short coalescing window for small first batches
        with self.lock:
            src, width, use_first = self._pick_first_source()
            jobs = [src.popleft() for _ in range(min(len(src), self.first_max_batch))]
            if jobs:
                if use_first:
                    self.first_streak += 1
                else:
                    self.first_streak = 0
                    if width is not None:
                        self.topup_last_width = width
            return jobs

    def _take_bulk(self) -> List[VocJob]:
        with self.lock:
            n_avail = len(self.q)
        if 0 < n_avail < self.max_batch // 2:
            time.sleep(0.004)  # let the batch fill to a useful size
        with self.lock:
            out: List[VocJob] = []
            held: List[VocJob] = []
            while self.q and len(out) < self.max_batch:
                j = self.q.popleft()
                # a later chunk of a request whose first chunk has not been emitted yet waits:
                # it needs that chunk's crossfade tail (server/vocoder.py:224-228)
                if not j.end_marker and j.window and j.req.audio_samples == 0:
                    held.append(j)
                else:
                    out.append(j)
            self.q.extendleft(reversed(held))
            return out

    def batch_geometry(self, lens: List[int]):
        """(T, Bp): bucketed window width and batch height (server/vocoder.py:240-249)."""
        mx = max(lens)
        T = _first_at_least(self.W_BUCKETS, mx)
        Bp = _first_at_least(self.B_BUCKETS, len(lens) + int(T > mx))
        return T, Bp

    @torch.inference_mode()
    def _process(self, jobs: List[VocJob]) -> None:
        t0 = time.perf_counter()
        real = [j for j in jobs if not j.end_marker and j.window]
        for j in jobs:
            if j.end_marker or not j.window:
                self._finish(j.req)
        if not real:
            return
        lens = [len(j.window) for j in real]
        T, Bp = self.batch_geometry(lens)
        tok_host = torch.zeros(Bp, T, dtype=torch.long)
        for i, j in enumerate(real):
            tok_host[i, : lens[i]] = torch.tensor(j.window, dtype=torch.long)
        tok = tok_host.to(self.device, non_blocking=False)
        tok_len = torch.tensor(lens + [T] * (Bp - len(real)), dtype=torch.long, device=self.device)
        mels, _ = self.s3gen.flow.inference(
            token=tok, token_len=tok_len, prompt_token=self.prompt_token, prompt_token_len=self.prompt_token_len,
            prompt_feat=self.prompt_feat, prompt_feat_len=None, embedding=self.embedding, finalize=True,
            n_timesteps=self.n_cfm, meanflow=True)                     # (Bp, 80, 2T)
        wavs, _ = self.s3gen.mel2wav.inference(
            speech_feat=mels.float(), cache_source=torch.zeros(Bp, 1, 0, device=self.device))  # (Bp, samples)
        wavs = wavs.float()
        if wavs.stride(-1) != 1:
            wavs = wavs.contiguous()
        pcm_host, spans, tails = self._stitch(real, lens, wavs)
        self.gpu_time += time.perf_counter() - t0
        self.batches += 1
        self.jobs += len(jobs)
        for j, (off, n), tail in zip(real, spans, tails):
            self._deliver(j, pcm_host[off: off + n].numpy().tobytes(), n, tail)

    def _stitch(self, real: List[VocJob], lens: List[int], wavs: torch.Tensor):
        """Stitch the batch on the device; returns the pinned int16 PCM, each job's span of it and
        the tail each job left.  The geometry is server/vocoder.py:284-310 per job.  Jobs of one
        request run in order: a request's k-th job of the batch goes into launch k, after the
        launch that made the tail it blends with (the reference post-processes jobs one by one)."""
        kernels.require(wavs.is_cuda, "the vocoder batch must be on a GPU (the stitch has no CPU path)")
        fade, S = self.fade, wavs.shape[1]
        dev = self.device
        stream = torch.cuda.current_stream(dev)
        seen: Dict[int, int] = {}
        rounds: List[List[int]] = []
        for i, j in enumerate(real):
            k = seen.get(id(j.req), 0)
            seen[id(j.req)] = k + 1
            if k == len(rounds):
                rounds.append([])
            rounds[k].append(i)
        spans: List[tuple] = [None] * len(real)
        tails_after: List[Optional[torch.Tensor]] = [None] * len(real)
        geo = []
        pcm_at = 0
        for idx in rounds:  # sizes first: one PCM buffer for all launches
            for i in idx:
                j, n_samp = real[i], min(lens[i] * SAMPLES_PER_TOKEN, S)
                off = j.emit_off * SAMPLES_PER_TOKEN
                lo = min(off if j.first else max(0, off - fade), n_samp)
                n_all = (self.pre_roll if j.first else 0) + n_samp - lo
                n_out = n_all - fade if (not j.final and n_all > fade) else n_all
                geo.append((i, lo, n_samp - lo, n_all, n_out, off))
                spans[i] = (pcm_at, n_out)
                pcm_at += n_out
        pcm = torch.empty(max(pcm_at, 1), dtype=torch.int16, device=dev)
        g = iter(geo)
        for idx in rounds:
            rows, tails_in, n_tail_out = [], [], 0
            for _ in idx:
                i, lo, n_seg, n_all, n_out, off = next(g)
                j = real[i]
                n_blend, tail_in = 0, -1
                tail = None if j.first else j.req.voc_tail
                if tail is not None and off - lo > 0:
                    ready = getattr(j.req, "voc_tail_ready", None)
                    if ready is not None and torch.is_tensor(tail) and tail.is_cuda:
                        # the tail may come from another lane's stream: order this
                        # stream after the launch that wrote it
                        stream.wait_event(ready)
                    if not torch.is_tensor(tail):  # handed over from another process as numpy
                        tail = torch.from_numpy(np.ascontiguousarray(tail, dtype=np.float32).reshape(-1))
                    n_blend = min(tail.numel(), off - lo, n_seg)
                    if n_blend > 0:
                        tail = tail.reshape(-1)[:fade].to(dev, torch.float32)
                        if tail.numel() < fade:
                            tail = torch.cat([tail, tail.new_zeros(fade - tail.numel())])
                        if tail.is_cuda:
                            tail.record_stream(stream)  # may come from another lane's stream
                        tail_in = len(tails_in)
                        tails_in.append(tail)
                trim = int(j.first and n_seg >= self.trim.numel())
                tail_out = -1
                if n_out < n_all:
                    tail_out, n_tail_out = n_tail_out, n_tail_out + 1
                rows.append([i, lo, n_seg, n_blend, trim, n_all - n_seg, n_out, tail_in, tail_out, spans[i][0], 0, 0])
            t_in = torch.stack(tails_in) if tails_in else None
            t_out = torch.empty(n_tail_out, fade, dtype=torch.float32, device=dev) if n_tail_out else None
            kernels.voc_stitch(wavs, torch.tensor(rows, dtype=torch.int32).to(dev), self.fade_in, self.fade_out,
                               self.trim, t_in, t_out, pcm)
            written = torch.cuda.Event()
            written.record(stream)
            for r in rows:  # the next launch (or the next batch, on any lane) blends with these tails
                tails_after[r[0]] = t_out[r[8]] if r[8] >= 0 else None
                real[r[0]].req.voc_tail = tails_after[r[0]]
                real[r[0]].req.voc_tail_ready = written
        pcm_host = torch.empty(pcm.numel(), dtype=torch.int16, pin_memory=True)
        pcm_host.copy_(pcm, non_blocking=True)
        done = torch.cuda.Event()
        done.record(stream)
        done.synchronize()
        return pcm_host, spans, tails_after

    def _deliver(self, j: VocJob, pcm: bytes, n: int, tail: Optional[torch.Tensor]) -> None:
        r = j.req
        if j.first and tail is not None:
            # a first-chunk worker in another process hands the tail back (server/vocoder.py:305-311)
            st = getattr(r, "send_tail", None)
            if st is not None:
                st(tail.cpu().numpy())
        r.audio_samples += n
        if r.t_first_pcm == 0.0:
            r.t_first_pcm = time.perf_counter()
        self._emit(r, pcm)
        if j.final:
            self._finish(r)

    def _finish(self, r) -> None:
        if r.finished:
            return
        r.finished = True
        r.t_done = time.perf_counter()
        self._emit(r, None)

    def _emit(self, r, data) -> None:
        if r.sink is not None:
            r.sink(data)

    def stats(self) -> dict:
        return dict(voc_batches=self.batches, voc_jobs=self.jobs, voc_queue=len(self.q),
                    voc_gpu_s=round(self.gpu_time, 2))


def chunk_target(voc: Vocoder, r) -> int:
    """Tokens the request's next chunk emits (server/engine.py:227-240)."""
    if not r.first_chunk_sent:
        return voc.chunk_first
    if voc.topup_sizes:
        cursor = voc.chunk_first
        for size in voc.topup_sizes:
            if r.emitted_tok < cursor + size:
                return size
            cursor += size
        return voc.chunk
    if voc.chunk_second and r.emitted_tok < voc.topup_until:
        return voc.chunk_second
    return voc.chunk


def maybe_vocode(voc: Vocoder, r, final: bool) -> None:
    """Hand the request's newly committed tokens to the vocoder in chunk-sized jobs
    (``EngineBase._maybe_vocode``, server/engine.py:223-258).  Once T3 is done (``r.t3_done``),
    whatever is left goes as the final job, or an end marker closes the stream."""
    avail = len(r.committed) - r.emitted_tok
    while True:
        target = chunk_target(voc, r)
        if r.t3_done and 0 < avail <= target:
            voc.enqueue(r, final=True)
            r.emitted_tok = len(r.committed)
            r.first_chunk_sent = True
            return
        if avail < target:
            break
        last = r.t3_done and avail == target
        voc.enqueue(r, final=last, n_emit=target)
        r.emitted_tok += target
        r.first_chunk_sent = True
        avail -= target
        if last:
            return
    if r.t3_done and avail == 0:
        voc.finalize_empty(r)
