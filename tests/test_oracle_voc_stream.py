"""Pins of oracle/voc_stream.py (the streaming vocoder's host arithmetic, server/vocoder.py:52-357,
server/engine.py:223-258) on the CPU.

* Windows and buckets: hand-computed cases of the reference's default schedule (chunk_first 12,
  chunk 80, lookback 16), of a chunk_second schedule and of a top-up schedule.
* The crossfade's direction: a constant tail faded into silence is the descending ramp.
* The stitch identity: with a vocoder whose samples depend only on their own token
  (``TableS3Gen``), the chunk stream -- windows with lookback, first-chunk trim, crossfades,
  withheld tails -- reproduces one vocode of the whole sequence to one int16 step, with exactly
  n * 960 (+ pre-roll) samples, for every schedule, length and arrival pattern tried (less the
  withheld 480 when an end marker closes the stream, which the reference drops).
* The chunk-target schedule by brute force: every committed token is emitted exactly once, in
  order, the last call is the only final one, and chunk sizes follow the schedule.
"""

import numpy as np
import pytest

from oracle import voc_stream as OV
from yapd_amd.synthetic import TableS3Gen

DEFAULT = dict(chunk_first=12, chunk=80, lookback=16)


def test_windows_of_the_default_schedule():
    jw = lambda a, b, n=None: OV.job_window(a, b, n_emit=n, **DEFAULT)
    assert jw(0, 12, 12) == (0, 0, True, True)
    assert jw(12, 92, 80) == (0, 12, False, False)       # 92 - (16 + 80) < 0
    assert jw(92, 172, 80) == (76, 16, False, False)     # 16 tokens of lookback
    assert jw(172, 200) == (104, 68, False, False)       # final remainder: window still 96 wide
    assert jw(172, 180) == (84, 88, False, False)        # short final: window reaches 96 back


def test_windows_of_topup_and_chunk_second_schedules():
    top = dict(chunk_first=12, chunk=80, lookback=16, topup_sizes=(8, 16))
    assert OV.job_window(12, 20, n_emit=8, **top) == (0, 12, False, True)   # priority, width 8
    assert OV.job_window(20, 36, n_emit=16, **top) == (0, 20, False, False)  # only e_start == 12 is priority
    sec = dict(chunk_first=12, chunk=80, lookback=16, chunk_second=20)
    assert OV.job_window(12, 32, n_emit=20, **sec) == (0, 12, False, True)
    assert OV.job_window(32, 112, n_emit=80, **sec) == (16, 16, False, False)


def test_batch_buckets():
    assert OV.batch_shape([64] * 4) == (64, 4)          # exact width: no padding row
    assert OV.batch_shape([50, 12]) == (52, 4)          # 52 > 50: one full-width row, 3 -> 4
    assert OV.batch_shape([96] * 5) == (96, 8)
    assert OV.batch_shape([97]) == (97, 4)              # wider than every bucket: the length itself
    assert OV.batch_shape([10] * 100) == (12, 101)      # taller than every bucket
    assert OV.batch_shape([13, 13, 13]) == (13, 4)


def test_fade_tables():
    fin, fout = OV.fade_tables(480)
    assert fin.dtype == fout.dtype == np.float32 and fin.shape == fout.shape == (480,)
    assert fin[0] == 0 and fin[-1] == 1 and np.all(np.diff(fin) > 0)
    assert np.all(np.abs(fin.astype(np.float64) + fout - 1) <= np.finfo(np.float32).eps)


def test_crossfade_direction_constant_tail_into_silence():
    fade = 480
    fin, fout = OV.fade_tables(fade)
    wav = np.zeros(3 * 960, np.float32)
    pcm, tail = OV.postprocess(wav, emit_off=1, first=False, final=False, tail=np.ones(fade, np.float32),
                               fade_in=fin, fade_out=fout, trim=np.ones(960, np.float32))
    # emitted audio starts fade samples before the emit point: the ramp, then silence; the last
    # fade samples are withheld
    assert len(pcm) == 3 * 960 - (960 - fade) - fade
    assert np.array_equal(pcm[:fade], (fout * np.float32(32767)).astype(np.int16))
    assert pcm[0] == 32767 and pcm[fade - 1] == 0 and not pcm[fade:].any()
    assert tail is not None and not tail.any()


def test_first_chunk_trim_and_short_chunks():
    fin, fout = OV.fade_tables(480)
    trim = TableS3Gen().trim_fade.numpy()
    wav = np.full(960, 0.5, np.float32)
    pcm, tail = OV.postprocess(wav, 0, True, True, None, fin, fout, trim)
    assert np.array_equal(pcm, ((wav * trim).clip(-1, 1) * np.float32(32767)).astype(np.int16))
    assert not pcm[:480].any() and tail is None
    # a first chunk shorter than the trim fade is not trimmed; <= fade samples withhold no tail
    pcm, tail = OV.postprocess(np.full(400, 0.5, np.float32), 0, True, False, None, fin, fout, trim)
    assert np.all(pcm == 16383) and tail is None
    pcm, tail = OV.postprocess(np.full(400, 0.5, np.float32), 0, True, False, None, fin, fout, trim, pre_roll=200)
    assert len(pcm) == 600 - 480 and not pcm.any() and len(tail) == 480


SCHEDULES = [
    DEFAULT,
    dict(chunk_first=12, chunk=80, lookback=16, chunk_second=20),
    dict(chunk_first=12, chunk=40, lookback=8, topup_sizes=(8, 16, 24)),
    dict(chunk_first=4, chunk=13, lookback=3),
]


@pytest.mark.parametrize("cfg", SCHEDULES)
@pytest.mark.parametrize("pre_roll", [0, 240])
def test_stream_equals_one_shot_render(cfg, pre_roll):
    s3 = TableS3Gen(vocab=512, seed=3)
    rng = np.random.default_rng(5)
    fin, fout = OV.fade_tables(480)
    for n in (1, 4, 11, 12, 13, 50, 93, 200, 333):
        tokens = rng.integers(0, 512, n).tolist()
        cuts = np.sort(rng.choice(np.arange(1, n), size=min(n - 1, rng.integers(0, 6)), replace=False)) if n > 1 else []
        arrivals = np.diff(np.concatenate([[0], cuts, [n]])).astype(int).tolist()
        got, dropped = OV.stream_pcm(tokens, arrivals, cfg, s3.render, s3.trim_fade.numpy(), pre_roll=pre_roll)
        ref, _ = OV.postprocess(s3.render(tokens), 0, True, True, None, fin, fout, s3.trim_fade.numpy(),
                                pre_roll=pre_roll)
        assert dropped in (0, 480)
        assert len(got) == n * 960 + pre_roll - dropped, (n, arrivals)
        assert np.abs(got.astype(np.int32) - ref[: len(got)]).max() <= 1, (n, arrivals)


@pytest.mark.parametrize("cfg", SCHEDULES)
def test_chunk_targets_emit_every_token_once(cfg):
    rng = np.random.default_rng(7)
    tcfg = {k: v for k, v in cfg.items() if k != "lookback"}
    for _ in range(300):
        n = int(rng.integers(0, 400))
        arrivals = []
        left = n
        while left > 0:
            a = int(rng.integers(1, 40))
            arrivals.append(min(a, left))
            left -= arrivals[-1]
        calls = OV.chunk_targets(n, arrivals, **tcfg)
        pos = 0
        for i, (a, b, final) in enumerate(calls):
            assert a == pos and b >= a
            assert final == (i == len(calls) - 1)
            pos = b
        assert pos == n and calls[-1][2]
        sizes = [b - a for a, b, _ in calls if b > a]
        if sizes:
            assert sizes[0] == min(cfg["chunk_first"], n)
        assert all(s <= max(cfg["chunk"], cfg["chunk_first"], cfg.get("chunk_second", 0),
                            *cfg.get("topup_sizes", (0,))) for s in sizes)


def test_chunk_targets_hand_case():
    # 100 tokens arriving 16 at a time then 4: the first 12 at once, 80 when 92 have arrived,
    # the remaining 8 as the final chunk when T3 ends
    assert OV.chunk_targets(100, [16] * 6 + [4], chunk_first=12, chunk=80) == [
        (0, 12, False), (12, 92, False), (92, 100, True)]
    # everything emitted before T3 ends: an end marker closes the stream
    assert OV.chunk_targets(92, [12, 80], chunk_first=12, chunk=80) == [
        (0, 12, False), (12, 92, False), (92, 92, True)]
