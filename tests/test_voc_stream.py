"""Host logic of the streaming vocoder (yapd_amd/voc_stream.py) on the CPU: the engine-side
hand-off and the worker's queues against the oracle (server/engine.py:223-258,
server/vocoder.py:123-235).  No kernel runs here; the batch path must refuse a CPU device."""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import voc_stream as OV
from yapd_amd.synthetic import TableS3Gen
from yapd_amd.voc_stream import Vocoder, VocJob, maybe_vocode

SCHEDULES = [
    dict(chunk_first=12, chunk=80, lookback=16),
    dict(chunk_first=12, chunk=80, lookback=16, chunk_second=20),
    dict(chunk_first=12, chunk=40, lookback=8, topup_sizes=(8, 16, 24)),
    dict(chunk_first=4, chunk=13, lookback=3),
]


def req(rid=0):
    return SimpleNamespace(rid=rid, committed=[], emitted_tok=0, first_chunk_sent=False, t3_done=False,
                           audio_samples=0, voc_tail=None, sink=None, finished=False, t_first_pcm=0.0,
                           t_done=0.0, t_recv=0.0)


def vocoder(**cfg):
    s3 = TableS3Gen(vocab=64)
    return Vocoder(s3, TableS3Gen.ref_dict(), "cpu", **cfg)


def record(voc):
    calls = []
    enq, fin = voc.enqueue, voc.finalize_empty

    def enqueue(r, final, n_emit=None):
        e_end = len(r.committed) if n_emit is None else r.emitted_tok + n_emit
        calls.append((r.emitted_tok, e_end, final, n_emit))
        enq(r, final, n_emit)

    def finalize_empty(r):
        calls.append((len(r.committed), len(r.committed), True, None))
        fin(r)

    voc.enqueue, voc.finalize_empty = enqueue, finalize_empty
    return calls


def random_arrivals(rng, n):
    out, left = [], n
    while left > 0:
        out.append(min(int(rng.integers(1, 40)), left))
        left -= out[-1]
    return out


@pytest.mark.parametrize("cfg", SCHEDULES)
def test_hand_off_follows_the_oracle_schedule(cfg):
    rng = np.random.default_rng(11)
    tcfg = {k: v for k, v in cfg.items() if k != "lookback"}
    for _ in range(60):
        voc = vocoder(**cfg)
        calls = record(voc)
        n = int(rng.integers(0, 300))
        arrivals = random_arrivals(rng, n)
        r = req()
        for a in arrivals:
            r.committed.extend(range(len(r.committed), len(r.committed) + a))
            maybe_vocode(voc, r, final=False)
        r.t3_done = True
        maybe_vocode(voc, r, final=True)
        assert [c[:3] for c in calls] == OV.chunk_targets(n, arrivals, **tcfg)
        # every job's window, emit offset and lane are the oracle's
        jobs = list(voc.q_first) + [j for dq in voc.q_topup.values() for j in dq] + list(voc.q)
        by_start = {j.window[j.emit_off] if j.window else None: j for j in jobs if not j.end_marker}
        for e_start, e_end, final, n_emit in calls:
            if e_start == e_end:
                continue
            j = by_start[e_start]  # tokens are their own positions
            w0, off, first, prio = OV.job_window(e_start, e_end, n_emit=n_emit, **cfg)
            assert (j.window, j.emit_off, j.first, j.final) == (list(range(w0, e_end)), off, first, final)
            lane = voc.q_first if first else (voc.q_topup[len(j.window)] if prio else voc.q)
            assert any(x is j for x in lane)


def test_bulk_lane_holds_later_chunks_until_the_first_is_out():
    voc = vocoder(chunk_first=4, chunk=8, lookback=2)
    a, b = req(0), req(1)
    b.audio_samples = 960
    ja = VocJob(a, [1, 2, 3], 1, False, False)
    jb = VocJob(b, [1, 2, 3], 1, False, False)
    end = VocJob(a, [], 0, False, True, end_marker=True)
    voc.q.extend([ja, jb, end])
    got = voc._take_bulk()
    assert got == [jb, end] and list(voc.q) == [ja]
    a.audio_samples = 960
    assert voc._take_bulk() == [ja]


def test_first_lane_gives_top_ups_a_turn_after_three_first_batches():
    voc = vocoder(chunk_first=4, chunk=8, lookback=2, topup_sizes=(4,))
    voc.first_max_batch = 1
    for i in range(6):
        voc.q_first.append(VocJob(req(i), [1] * 4, 0, True, False))
    voc.q_topup[6].append(VocJob(req(9), [1] * 6, 2, False, False))
    voc.q_topup[8].append(VocJob(req(10), [1] * 8, 2, False, False))
    order = []
    for _ in range(7):
        jobs = voc._take_first()
        order.append("first" if jobs[0].first else len(jobs[0].window))
    # three first batches, then the narrowest pending top-up width, then first chunks again,
    # and widths rotate upwards
    assert order == ["first", "first", "first", 6, "first", "first", "first"]
    assert voc._take_first()[0].window == [1] * 8


def test_batch_geometry_is_the_oracle_s():
    voc = vocoder()
    rng = np.random.default_rng(2)
    for _ in range(200):
        lens = rng.integers(1, 120, int(rng.integers(1, 110))).tolist()
        assert voc.batch_geometry(lens) == OV.batch_shape(lens)


def test_the_batch_path_refuses_a_cpu_device():
    voc = vocoder(chunk_first=4, chunk=8, lookback=2)
    r = req()
    r.committed = [1, 2, 3, 4]
    maybe_vocode(voc, r, final=False)
    with pytest.raises(ValueError, match="GPU"):
        voc._process(voc._take_first())
