"""Oracle: the chunked streaming vocoder's host arithmetic -- test infrastructure.

Only tests/ may import this module (nothing in yapd_amd/ does).  It restates,
in numpy and plain Python, what server/vocoder.py does around the S3Gen
models:

* ``fade_tables``   -- the 20 ms linear crossfade ramps, vocoder.py:108-109;
* ``job_window``    -- the token window a job vocodes and where its emitted
                       part starts, ``Vocoder.enqueue`` vocoder.py:123-147;
* ``batch_shape``   -- padded micro-batch width and height from the W / B
                       buckets, ``Vocoder._process`` vocoder.py:240-251;
* ``postprocess``   -- first-chunk trim fade, crossfade with the previous
                       chunk's withheld tail, tail withholding, clip and int16
                       conversion, ``Vocoder._postprocess`` vocoder.py:284-320;
* ``chunk_targets`` -- how many tokens each enqueue emits as committed tokens
                       arrive, ``EngineBase._maybe_vocode``
                       server/engine.py:223-258.

Pinned in tests/test_oracle_voc_stream.py by: hand-computed windows and
buckets of the reference's defaults; the identity that, for a vocoder whose
samples depend only on their own token, the stitched chunk stream equals one
vocode of the whole token sequence (to one int16 step); a crossfade of a
constant tail into silence that must be the descending ramp; exact sample
counts; and brute force over the chunk-target schedule (every committed token
emitted exactly once, in order).
"""

from __future__ import annotations

from typing import List, Optional, Sequence, Tuple

import numpy as np

SR = 24000
SAMPLES_PER_TOKEN = 960
B_BUCKETS = (4, 8, 16, 24, 32, 48, 64, 96)
W_BUCKETS = (4, 8, 12, 13, 15, 16, 20, 21, 24, 28, 32, 36, 40, 44, 52, 60, 64, 68, 76, 80, 84, 96)


def fade_tables(fade: int) -> Tuple[np.ndarray, np.ndarray]:
    """(fade_in, fade_out) of vocoder.py:108-109: a float32 linspace 0..1 and one minus it."""
    fin = np.linspace(0.0, 1.0, fade, dtype=np.float32)
    return fin, (1.0 - fin).astype(np.float32)


def job_window(e_start: int, e_end: int, *, chunk: int, lookback: int, chunk_first: int, chunk_second: int = 0,
               topup_sizes: Sequence[int] = (), topup_until: int = 0, n_emit: Optional[int] = None):
    """(w_start, emit_off, first, priority) of a job emitting tokens [e_start, e_end), vocoder.py:123-147.

    The window starts ``lookback + emit_width`` tokens before e_end (never
    after e_start, never before 0); the first job starts at 0.  Priority jobs
    (first chunks, and the top-up chunks right after them) go to the
    first-chunk lane.
    """
    first = e_start == 0
    until = topup_until or (chunk_first + (sum(topup_sizes) if topup_sizes else chunk_second))
    if topup_sizes:
        priority = first or e_start == chunk_first
    else:
        priority = first or (chunk_second > 0 and e_start < until)
    emit_width = n_emit if (priority and not first and n_emit) else chunk
    w_start = 0 if first else max(0, e_end - (lookback + emit_width))
    w_start = min(w_start, e_start)
    return w_start, e_start - w_start, first, priority


def batch_shape(lens: Sequence[int]) -> Tuple[int, int]:
    """(T, Bp) of vocoder.py:240-251: the smallest W bucket >= the longest window (else that
    length); one extra full-width row when T exceeds every real row; the smallest B bucket that
    holds the rows (else the row count)."""
    mx = max(lens)
    T = next((t for t in W_BUCKETS if t >= mx), mx)
    need = len(lens) + int(T > mx)
    Bp = next((b for b in B_BUCKETS if b >= need), need)
    return T, Bp


def postprocess(wav: np.ndarray, emit_off: int, first: bool, final: bool, tail: Optional[np.ndarray],
                fade_in: np.ndarray, fade_out: np.ndarray, trim: np.ndarray, pre_roll: int = 0):
    """(pcm int16, new tail or None) of one job, vocoder.py:284-320.

    ``wav`` is the job's row of the batch cut to its window's samples
    (``n_tok * 960``).  Emitted audio starts ``fade`` samples before the emit
    point (the overlap the previous chunk withheld), blended as
    ``tail * fade_out + seg * fade_in``; a first chunk starts at the emit point
    and has the trim fade applied when it is at least that long.  Unless the
    job is final, the last ``fade`` samples are withheld as the next tail.
    """
    fade = len(fade_in)
    off = emit_off * SAMPLES_PER_TOKEN
    wav = np.array(wav, dtype=np.float32, copy=True)
    if first:
        seg = wav[off:]
        if len(seg) >= len(trim):
            seg[: len(trim)] *= trim
    else:
        lo = max(0, off - fade)
        seg = wav[lo:]
        n_ov = off - lo
        if tail is not None and n_ov > 0:
            n = min(len(tail), n_ov, len(seg))
            seg[:n] = tail[:n] * fade_out[:n] + seg[:n] * fade_in[:n]
    out = seg
    if first and pre_roll:
        out = np.concatenate((np.zeros(pre_roll, dtype=np.float32), out))
    if not final and len(out) > fade:
        new_tail = out[-fade:].copy()
        out = out[:-fade]
    else:
        new_tail = None
    pcm = (np.clip(out, -1.0, 1.0) * np.float32(32767.0)).astype("<i2")
    return pcm, new_tail


def chunk_targets(n_tokens: int, arrivals: Sequence[int], *, chunk_first: int, chunk: int, chunk_second: int = 0,
                  topup_sizes: Sequence[int] = (), topup_until: int = 0) -> List[Tuple[int, int, bool]]:
    """The enqueue calls ``_maybe_vocode`` (server/engine.py:223-258) makes for one request.

    ``arrivals`` are the sizes of the committed-token batches as they arrive
    (summing to n_tokens); after the last one T3 is done.  Returns
    ``(e_start, e_end, final)`` per call; an ``(n, n, True)`` entry is the
    empty end marker of ``finalize_empty``.
    """
    until = topup_until or (chunk_first + (sum(topup_sizes) if topup_sizes else chunk_second))
    calls = []
    committed = emitted = 0
    first_sent = False

    def target():
        if not first_sent:
            return chunk_first
        if topup_sizes:
            cursor = chunk_first
            for size in topup_sizes:
                if emitted < cursor + size:
                    return size
                cursor += size
            return chunk
        if chunk_second and emitted < until:
            return chunk_second
        return chunk

    def vocode(done):
        nonlocal emitted, first_sent
        avail = committed - emitted
        while True:
            t = target()
            if done and 0 < avail <= t:
                calls.append((emitted, committed, True))
                emitted = committed
                first_sent = True
                return
            if avail >= t:
                last = done and avail == t
                calls.append((emitted, emitted + t, last))
                emitted += t
                first_sent = True
                avail -= t
                if last:
                    return
            else:
                break
        if done and avail == 0:
            calls.append((committed, committed, True))

    for a in arrivals:
        committed += a
        vocode(False)
    assert committed == n_tokens
    vocode(True)
    return calls


def stream_pcm(tokens: Sequence[int], arrivals: Sequence[int], cfg: dict, render, trim: np.ndarray,
               fade: int = 480, pre_roll: int = 0):
    """One request's audio as the reference streams it: (int16 PCM of all its chunks in order,
    samples of a withheld tail never emitted).

    ``cfg`` holds the schedule knobs (chunk_first, chunk, lookback and optionally chunk_second,
    topup_sizes, topup_until); ``render(tokens)`` is the vocoder's fp32 waveform of a window.
    An end marker closes the stream without emitting the tail the last chunk withheld
    (finalize_empty, server/vocoder.py:157-160, 232-235), so when every token went out in
    non-final chunks before T3 ended, the last ``fade`` samples are dropped.
    """
    fin, fout = fade_tables(fade)
    tcfg = {k: v for k, v in cfg.items() if k != "lookback"}
    tail, out = None, []
    for e_start, e_end, final in chunk_targets(len(tokens), arrivals, **tcfg):
        if e_start == e_end:  # end marker
            return (np.concatenate(out) if out else np.zeros(0, np.int16)), (0 if tail is None else len(tail))
        w0, off, first, _ = job_window(e_start, e_end, **cfg)
        pcm, tail = postprocess(render(tokens[w0:e_end]), off, first, final, tail, fin, fout, trim, pre_roll=pre_roll)
        out.append(pcm)
    return (np.concatenate(out) if out else np.zeros(0, np.int16)), 0
