"""The streaming vocoder on the GPU against the oracle (server/vocoder.py:52-357,
server/engine.py:223-258).

* The stitch kernel, through ``Vocoder._stitch``, equals ``oracle.voc_stream.postprocess`` run job
  after job on the same waveform rows, bit for bit in the int16 PCM and in the fp32 tails: first
  chunks with and without the trim fade, crossfades from device and numpy tails (full and short),
  no tail, no overlap, outputs too short to withhold a tail, pre-roll, two chunks of one request
  in one batch (the second blends with the tail the first just made).
* The whole worker with a position-local S3Gen stand-in (``TableS3Gen``): every request's PCM
  equals the oracle's stream (``stream_pcm``) bit for bit -- driven synchronously over four
  chunk schedules, and with the two lanes on their own threads and streams while requests arrive.
* The serving engine hands committed tokens to the vocoder: every finished request's stream is
  closed exactly once and its audio is the one-shot render of its committed tokens to one int16
  step, n * 960 samples long (480 fewer when an end marker closed the stream).
"""

import threading
import time

import numpy as np
import pytest
import torch

from oracle import voc_stream as OV
from yapd_amd.serve import HipFlashEngine, Request
from yapd_amd.synthetic import MASK_ID, SOS_ID, STOP_ID, TableS3Gen, make_t3
from yapd_amd.voc_stream import Vocoder, VocJob, maybe_vocode

pytestmark = pytest.mark.gpu

SCHEDULES = [
    dict(chunk_first=12, chunk=80, lookback=16),
    dict(chunk_first=12, chunk=80, lookback=16, chunk_second=20),
    dict(chunk_first=12, chunk=40, lookback=8, topup_sizes=(8, 16, 24)),
    dict(chunk_first=4, chunk=13, lookback=3),
]


class Req:
    def __init__(self, rid):
        self.rid, self.committed, self.emitted_tok, self.first_chunk_sent = rid, [], 0, False
        self.t3_done, self.audio_samples, self.voc_tail, self.finished = False, 0, None, False
        self.t_first_pcm = self.t_done = self.t_recv = 0.0
        self.chunks, self.closed = [], 0

    def sink(self, data):
        if data is None:
            self.closed += 1
        else:
            self.chunks.append(data)

    def pcm(self):
        return np.frombuffer(b"".join(self.chunks), dtype="<i2")


def test_stitch_matches_oracle_job_by_job(dev):
    g = torch.Generator(device=dev).manual_seed(4)
    for pre_roll in (0, 240):
        s3 = TableS3Gen(vocab=64, device=dev)
        voc = Vocoder(s3, TableS3Gen.ref_dict(), dev, pre_roll=pre_roll)
        fin, fout = OV.fade_tables(480)
        trim = s3.trim_fade.numpy()
        wavs = (torch.rand(10, 12 * 960, generator=g, device=dev) * 3 - 1.5).contiguous()
        a, b, c, d, e, f, h, k = (Req(i) for i in range(8))
        rnd = np.random.default_rng(pre_roll)
        c.voc_tail = torch.from_numpy(rnd.uniform(-1, 1, 480).astype(np.float32)).to(dev)
        d.voc_tail = rnd.uniform(-1, 1, 480).astype(np.float32)
        e.voc_tail = torch.from_numpy(rnd.uniform(-1, 1, 480).astype(np.float32)).to(dev)
        h.voc_tail = rnd.uniform(-1, 1, 200).astype(np.float32)
        k.voc_tail = torch.from_numpy(rnd.uniform(-1, 1, 480).astype(np.float32)).to(dev)
        jobs = [
            (VocJob(a, [0] * 12, 0, True, False), 12),   # first, trimmed, tail withheld
            (VocJob(b, [0] * 1, 0, True, True), 1),      # first, final, one token
            (VocJob(c, [0] * 9, 4, False, False), 9),    # crossfade from a device tail
            (VocJob(d, [0] * 7, 4, False, True), 7),     # crossfade from a numpy tail, final
            (VocJob(e, [0] * 6, 0, False, False), 6),    # no overlap: the tail is not used
            (VocJob(f, [0] * 5, 3, False, False), 5),    # no tail: the overlap goes out unblended
            (VocJob(h, [0] * 3, 2, False, False), 3),    # short numpy tail: 200 blended samples
            (VocJob(k, [0] * 1, 1, False, False), 1),    # 480 samples out: no tail withheld
            (VocJob(k, [0] * 4, 1, False, False), 4),    # second job of k in the batch
            (VocJob(k, [0] * 2, 1, False, True), 2),     # third job of k
        ]
        before = {}
        for j, _ in jobs:
            t = j.req.voc_tail
            before.setdefault(id(j.req), None if t is None else (t.cpu().numpy() if torch.is_tensor(t) else t.copy()))
        pcm_host, spans, tails = voc._stitch([j for j, _ in jobs], [n for _, n in jobs], wavs)
        chain = dict(before)
        for i, ((j, n), (off, cnt), tail) in enumerate(zip(jobs, spans, tails)):
            ref, ref_tail = OV.postprocess(wavs[i, : n * 960].cpu().numpy(), j.emit_off, j.first, j.final,
                                           chain[id(j.req)], fin, fout, trim, pre_roll=pre_roll)
            chain[id(j.req)] = ref_tail
            got = pcm_host[off: off + cnt].numpy()
            assert np.array_equal(got, ref), (pre_roll, i)
            assert (tail is None) == (ref_tail is None), (pre_roll, i)
            if tail is not None:
                assert np.array_equal(tail.cpu().numpy(), ref_tail), (pre_roll, i)
        for j, _ in jobs:  # the request keeps the tail of its last job
            t = j.req.voc_tail
            assert (t is None) == (chain[id(j.req)] is None)
    # a waveform row shorter than a first chunk's trim fade: no trim, as the reference
    voc = Vocoder(TableS3Gen(vocab=64, device=dev), TableS3Gen.ref_dict(), dev)
    wavs = (torch.rand(1, 700, generator=g, device=dev) * 2 - 1).contiguous()
    r = Req(0)
    pcm_host, spans, _ = voc._stitch([VocJob(r, [0], 0, True, True)], [1], wavs)
    ref, _ = OV.postprocess(wavs[0].cpu().numpy(), 0, True, True, None, fin, fout, trim)
    assert np.array_equal(pcm_host[: spans[0][1]].numpy(), ref)


def drain(voc):
    while True:
        jobs = voc._take_first()
        if not jobs:
            jobs = voc._take_bulk()
        if not jobs:
            return
        voc._process(jobs)


@pytest.mark.parametrize("cfg", SCHEDULES)
def test_worker_streams_equal_the_oracle(dev, cfg):
    s3 = TableS3Gen(vocab=512, seed=2, device=dev)
    voc = Vocoder(s3, TableS3Gen.ref_dict(), dev, max_batch=8, first_max_batch=4, **cfg)
    rng = np.random.default_rng(3)
    reqs, plans = [], []
    for rid in range(10):
        n = int(rng.integers(1, 260))
        toks = rng.integers(0, 512, n).tolist()
        arrivals, left = [], n
        while left:
            arrivals.append(min(int(rng.integers(1, 48)), left))
            left -= arrivals[-1]
        r = Req(rid)
        reqs.append(r)
        plans.append((toks, arrivals))
    # interleave the requests' arrivals; vocode what is queued after every round
    step = 0
    while any(not r.t3_done for r in reqs):
        for r, (toks, arr) in zip(reqs, plans):
            if r.t3_done:
                continue
            if step < len(arr):
                n0 = sum(arr[:step])
                r.committed.extend(toks[n0: n0 + arr[step]])
                maybe_vocode(voc, r, final=False)
            else:
                r.t3_done = True
                maybe_vocode(voc, r, final=True)
        drain(voc)
        step += 1
    drain(voc)
    for r, (toks, arr) in zip(reqs, plans):
        ref, dropped = OV.stream_pcm(toks, arr, cfg, s3.render, s3.trim_fade.numpy())
        assert r.closed == 1 and r.finished
        assert np.array_equal(r.pcm(), ref), (r.rid, len(r.pcm()), len(ref))
        assert len(ref) == len(toks) * 960 - dropped


# with a second-chunk size or top-up widths, a request's top-up chunk runs on the first-chunk lane
# while its next chunk can go to the bulk lane, which then blends with a tail the other lane's
# stream wrote (ordered by the event stored with the tail)
@pytest.mark.parametrize("cfg", [dict(chunk_first=12, chunk=40, lookback=16),
                                 dict(chunk_first=12, chunk=80, lookback=16, chunk_second=20),
                                 dict(chunk_first=12, chunk=40, lookback=8, topup_sizes=(8, 16, 24))],
                         ids=["default", "chunk_second", "topup"])
def test_worker_lanes_on_threads(dev, cfg):
    s3 = TableS3Gen(vocab=512, seed=7, device=dev)
    voc = Vocoder(s3, TableS3Gen.ref_dict(), dev, max_batch=16, first_max_batch=8, **cfg)
    worker = threading.Thread(target=voc.run, daemon=True)
    worker.start()
    rng = np.random.default_rng(8)
    reqs, plans = [], []
    for rid in range(12):
        n = int(rng.integers(20, 200))
        toks = rng.integers(0, 512, n).tolist()
        arrivals, left = [], n
        while left:
            arrivals.append(min(16, left))
            left -= arrivals[-1]
        reqs.append(Req(rid))
        plans.append((toks, arrivals))
    try:
        for step in range(max(len(a) for _, a in plans) + 1):
            for r, (toks, arr) in zip(reqs, plans):
                if r.t3_done:
                    continue
                if step < len(arr):
                    r.committed.extend(toks[16 * step: 16 * step + arr[step]])
                    maybe_vocode(voc, r, final=False)
                else:
                    r.t3_done = True
                    maybe_vocode(voc, r, final=True)
            time.sleep(0.003)
        t_end = time.time() + 60
        while any(r.closed == 0 for r in reqs) and time.time() < t_end:
            time.sleep(0.01)
    finally:
        voc.close()
        worker.join(timeout=30)
    assert not worker.is_alive()
    for r, (toks, arr) in zip(reqs, plans):
        ref, _ = OV.stream_pcm(toks, arr, cfg, s3.render, s3.trim_fade.numpy())
        assert r.closed == 1
        assert np.array_equal(r.pcm(), ref), r.rid
    assert voc.stats()["voc_jobs"] >= len(reqs)


def test_engine_hands_committed_tokens_to_the_vocoder(dev):
    model = make_t3(n_layers=2, seed=5, device=dev)
    V = model.speech_head.weight.shape[0]
    log_prior = torch.log_softmax(torch.randn(V, generator=torch.Generator().manual_seed(1)), 0)
    s3 = TableS3Gen(vocab=SOS_ID, seed=1, device=dev)
    voc = Vocoder(s3, TableS3Gen.ref_dict(), dev, chunk_first=12, chunk=40, lookback=16)
    eng = HipFlashEngine(model, log_prior=log_prior, mask_id=MASK_ID, stop_id=STOP_ID, codec_vocab=SOS_ID,
                         max_active=4, max_prefix_tokens=96, max_speech_tokens=96, num_steps=4, temperature=0.0,
                         position_temperature=0.0, cfg_scale=0.5, block_size=16, page_table_seed=2, vocoder=voc)
    worker = threading.Thread(target=voc.run, daemon=True)
    worker.start()
    g = torch.Generator().manual_seed(3)
    sos = model._embed_speech_tokens(torch.tensor([[SOS_ID]], device=dev))[0, 0].detach()
    reqs, sinks = [], []
    for i, (lp, ns) in enumerate([(23, 32), (61, 48), (40, 64), (17, 80), (70, 48), (33, 64)]):
        pre = (torch.randn(lp, 1024, generator=g) * 0.5).to(dev, torch.bfloat16)
        pre[-1] = sos.to(torch.bfloat16)
        r = Request(rid=i, prefix=pre, n_speech=ns)
        k = Req(i)
        r.sink = k.sink
        reqs.append(r)
        sinks.append(k)
        eng.submit(r)
    try:
        eng.run_until_idle(max_ticks=2000)
        t_end = time.time() + 60
        while any(k.closed == 0 for k in sinks) and time.time() < t_end:
            time.sleep(0.01)
    finally:
        voc.close()
        worker.join(timeout=30)
    trim = s3.trim_fade.numpy()
    fin, fout = OV.fade_tables(480)
    for r, k in zip(reqs, sinks):
        assert k.closed == 1 and r.finished and r.t3_done
        n = len(r.committed)
        got = k.pcm()
        assert len(got) in (n * 960, n * 960 - 480), (r.rid, n, len(got))
        if n:
            ref, _ = OV.postprocess(s3.render(r.committed), 0, True, True, None, fin, fout, trim)
            assert np.abs(got.astype(np.int32) - ref[: len(got)]).max() <= 1, r.rid
        assert r.audio_samples == len(got)


class _HiftStandIn:
    """A HiFT-shaped generator (fused Snake installed) as S3Gen's mel2wav: its waveform depends on
    the neighbouring frames, so stitched chunks differ from a one-shot render; each of its samples
    is repeated 15 times to give S3Gen's 480 samples per mel frame."""

    def __init__(self, dev):
        from test_gpu_vocoder import HiFTGenerator
        from yapd_amd.vocoder import install_fused_snake
        g = torch.Generator().manual_seed(12)
        gen = HiFTGenerator(g)
        for p in gen.parameters():
            p.data.mul_(0.5)
        self.gen = gen.to(dev).eval()
        assert install_fused_snake(self.gen) == 48

    def inference(self, *, speech_feat, cache_source):
        B, _, T = speech_feat.shape
        s = torch.zeros(B, 1, 32 * T, device=speech_feat.device)
        return self.gen.decode(speech_feat, s).repeat_interleave(15, dim=-1), None


class _MelTableFlow:
    """Tokens -> mels from a fixed table (both frames of a token get its row)."""

    def __init__(self, dev, vocab=512):
        g = torch.Generator().manual_seed(13)
        self.table = (torch.randn(vocab, 80, generator=g) * 0.5).to(dev)

    def inference(self, *, token, **kw):
        return self.table[token].repeat_interleave(2, dim=1).transpose(1, 2).contiguous(), None


def test_worker_on_a_hift_shaped_generator(dev):
    cfg = dict(chunk_first=12, chunk=40, lookback=16)
    s3 = TableS3Gen(vocab=512, device=dev)
    s3.flow, s3.mel2wav = _MelTableFlow(dev), _HiftStandIn(dev)
    voc = Vocoder(s3, TableS3Gen.ref_dict(), dev, max_batch=6, first_max_batch=3, pre_roll=120, **cfg)
    fin, fout = OV.fade_tables(480)
    trim = s3.trim_fade.numpy()
    checked = [0]
    orig = voc._stitch

    def stitch_checked(real, lens, wavs):
        chain = {}
        for j in real:
            t = j.req.voc_tail
            chain.setdefault(id(j.req), None if t is None else t.cpu().numpy())
        pcm_host, spans, tails = orig(real, lens, wavs)
        for i, (j, n, (off, cnt)) in enumerate(zip(real, lens, spans)):
            ref, ref_tail = OV.postprocess(wavs[i, : n * 960].cpu().numpy(), j.emit_off, j.first, j.final,
                                           chain[id(j.req)], fin, fout, trim, pre_roll=120)
            chain[id(j.req)] = ref_tail
            assert np.array_equal(pcm_host[off: off + cnt].numpy(), ref), (j.req.rid, i)
            checked[0] += 1
        return pcm_host, spans, tails

    voc._stitch = stitch_checked
    rng = np.random.default_rng(21)
    reqs, plans = [], []
    for rid in range(7):
        n = int(rng.integers(5, 150))
        toks = rng.integers(0, 512, n).tolist()
        arrivals, left = [], n
        while left:
            arrivals.append(min(int(rng.integers(4, 30)), left))
            left -= arrivals[-1]
        reqs.append(Req(rid))
        plans.append((toks, arrivals))
    step = 0
    while any(not r.t3_done for r in reqs):
        for r, (toks, arr) in zip(reqs, plans):
            if r.t3_done:
                continue
            if step < len(arr):
                n0 = sum(arr[:step])
                r.committed.extend(toks[n0: n0 + arr[step]])
                maybe_vocode(voc, r, final=False)
            else:
                r.t3_done = True
                maybe_vocode(voc, r, final=True)
        drain(voc)
        step += 1
    drain(voc)
    zeros = lambda window: np.zeros(len(window) * 960, np.float32)
    for r, (toks, arr) in zip(reqs, plans):
        want, _ = OV.stream_pcm(toks, arr, cfg, zeros, trim, pre_roll=120)
        assert r.closed == 1 and len(r.pcm()) == len(want), r.rid
        assert np.abs(r.pcm().astype(np.int32)).max() > 0
    assert checked[0] >= len(reqs) * 2


def test_stitch_skips_jobs_that_do_not_fit_their_buffers(dev):
    from yapd_amd import kernels as K
    wav = torch.rand(2, 4 * 960, device=dev) * 2 - 1
    fin = torch.linspace(0, 1, 480, device=dev)
    fout = 1 - fin
    trim = torch.ones(960, device=dev)
    t_in = torch.rand(1, 480, device=dev)
    t_out = torch.full((1, 480), 7.0, device=dev)
    pcm = torch.full((8000,), 12345, dtype=torch.int16, device=dev)
    n = 4 * 960
    jobs = torch.tensor([
        [0, 0, n, 0, 0, 0, n, -1, -1, 0, 0, 0],            # valid: row 0 whole, no tail
        [2, 0, n, 0, 0, 0, n, -1, -1, 0, 0, 0],            # row out of range
        [1, 960, n, 0, 0, 0, n, -1, -1, 0, 0, 0],          # samples past the row
        [1, 0, n, 0, 0, 0, n, -1, -1, 6000, 0, 0],         # PCM past the buffer
        [1, 0, n, 480, 0, 0, n, 3, -1, 4000, 0, 0],        # blend from a missing tail
        [1, 0, n, 0, 0, 0, n - 100, -1, 0, 4000, 0, 0],    # withheld samples != fade
        [1, 0, n, 0, 0, 0, n - 480, -1, 5, 4000, 0, 0],    # tail row out of range
    ], dtype=torch.int32, device=dev)
    K.voc_stitch(wav, jobs, fin, fout, trim, t_in, t_out, pcm)
    got = pcm.cpu().numpy()
    ref = (np.clip(wav[0].cpu().numpy(), -1, 1) * np.float32(32767)).astype(np.int16)
    assert np.array_equal(got[:n], ref)
    assert np.all(got[n:] == 12345) and bool((t_out == 7.0).all())
    with pytest.raises(ValueError, match="n_jobs"):
        K.voc_stitch(wav, torch.zeros(70000, 12, dtype=torch.int32, device=dev), fin, fout, trim, None, None, pcm)
