#!/usr/bin/env python3
"""Benchmark: the full 30-layer T3 block-diffusion decode step on one MI355X.

Workload (synthetic, seeded): 256 CFG pairs = 512 rows in generate()'s
stacked order, block 32, prefix lengths U[150, 600] per pair (both rows of a
pair share it), prefixes prefilled through the engine, shuffled page table,
30-layer Llama (hidden 1024, 16 x 64 heads, FFN 4096, RMSNorm eps 1e-5, RoPE
theta 10000, linear weights N(0, 0.02)), speech head V = 8194, then CFG
(w = 0.5) + PMI (Dirichlet(0.1) prior) + time-shifted-quantile unmask
(tau = 3.0, K = 10, t_shift 0.5).  One step = embedding -> backbone -> head ->
scoring, replayed as one HIP graph.

Prints one JSON line.  ``value`` = speech tokens/s = pairs * block / step time.
``roofline`` describes the dominant kernel (the gate/up + SiLU GEMM) against
the published bf16 peak and, as ``peak_measured``, against the sustained MFMA
rate of a register-only calibration kernel on random operands spread like the
step's (``peak_measured_constant_operands``: the same kernel on few-bit
constants, which draw less power and run faster) and, as ``vendor_gemm``, against
hipBLASLt's plain GEMM of the same shape (torch ``F.linear``, no SiLU) timed in
the same run (both that and the fused kernel as 20 calls over four layers'
weights in one graph replay, ``ours_same_timing_us``); ``kernels`` adds attention and scoring against the HBM roofline.  Per-kernel durations come from HIP events
on the stream the kernel runs on, right after the timed region: around single
launches for the GEMMs, and around one graph replay of 20 back-to-back calls
for attention and scoring (calls shorter than their host launch work),
rotating inputs so that none is served from the 256 MB MALL.  ``cpu_baseline``
times the oracle (torch on the host cores) on a bounded sample of the same
step.

``secondary`` (skipped with ``--no-secondary``) carries, from the same run,
the headline figures of the prefill, serve, attention-stress and vocoder
workloads below (about 15 s more).

``--workload serve`` runs the continuous-batching engine (server defaults:
128 slots, block 16, K = 10, temperature 0.6, position temperature 5, CFG 1)
over a queue of requests and reports committed speech tokens per second.

``--workload vocoder`` times the HiFT vocoder's elementwise family on the
last-stage tensors of a 48-chunk micro-batch of 80-token chunks
([48, 64, 19201] fp32) against the HBM roofline, and the streaming
vocoder's chunk stitch on a 48-job batch.

``--workload prefill`` times the prefix prefill of the step's rows (causal,
packed steps of 64-token segments through the paged KV) in prefix tokens per
second.

``--workload attn_stress`` instead measures 30 layers of block attention
back to back over 256 sequences with log-uniform [64, 2048] prefixes, block
16, each layer's pages drawn at random from its own 65,536-page pool; and
``--workload quant`` the four 4-bit and 8-bit affine-quantised projections of
30 layers at M = 8192.  Each prints its own JSON line.
"""

from __future__ import annotations

import argparse
import copy
import json
import math
import os
import subprocess
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--pairs", type=int, default=256)
    ap.add_argument("--block", type=int, default=32)
    ap.add_argument("--layers", type=int, default=30)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-layers", type=int, default=2, help="layers in the CPU baseline sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-secondary", action="store_true",
                    help="step workload: skip the prefill / serve / attention-stress figures")
    ap.add_argument("--workload", choices=["step", "attn_stress", "quant", "serve", "vocoder", "prefill"],
                    default="step")
    ap.add_argument("--requests", type=int, default=384, help="serve workload: number of requests")
    ap.add_argument("--kernel-sample", action="store_true",
                    help="only run each kernel of the step at the bench shape x3 and a 1 GiB copy, for rocprofv3 --pmc")
    return ap.parse_args()


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def time_launches(fn, reps, dev):
    """Average device time of ``fn`` (one or more launches) over ``reps`` with stream events."""
    s = torch.cuda.current_stream(dev)
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(reps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(reps)]
    fn()
    for i in range(reps):
        starts[i].record(s)
        fn()
        ends[i].record(s)
    torch.cuda.synchronize(dev)
    return sum(a.elapsed_time(b) for a, b in zip(starts, ends)) / reps  # ms


def time_graphs(fns, reps, dev):
    """Average device time of one call when ``reps`` calls, cycling through ``fns``, are captured
    back to back in one HIP graph: one replay between the events, so neither host launch work nor
    the graph's own launch latency is counted per call."""
    s = torch.cuda.current_stream(dev)
    for fn in fns:
        fn()
    torch.cuda.synchronize(dev)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(reps):
            fns[i % len(fns)]()
    g.replay()
    torch.cuda.synchronize(dev)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(s)
    g.replay()
    end.record(s)
    torch.cuda.synchronize(dev)
    return start.elapsed_time(end) / reps  # ms


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "yapd_amd runs the step on one GPU; multi-GPU (data-parallel over pairs) is not "
                                   "part of it", "n_gpus": args.gpus}))
        sys.exit(2)
    from yapd_amd import kernels
    from yapd_amd.engines.hip import HipEngine
    from yapd_amd.paged import AttnPlan
    from yapd_amd.step import DecodeStep
    from yapd_amd.synthetic import MASK_ID, STOP_ID, make_t3, scoring_inputs, uniform_lengths

    kernels.load_library()
    dev = torch.device("cuda:0")
    Bp, bl, L = args.pairs, args.block, args.layers
    if args.kernel_sample and args.workload == "step":
        kernel_sample(dev, Bp, bl)
        return
    if args.workload == "attn_stress":
        print(json.dumps(attn_stress(args, dev)), flush=True)
        return
    if args.workload == "quant":
        quant_projections(args, dev)
        return
    if args.workload == "serve":
        print(json.dumps(serve(args, dev)), flush=True)
        return
    if args.workload == "vocoder":
        out = vocoder_workload(args, dev)
        if out is not None:
            print(json.dumps(out), flush=True)
        return
    if args.workload == "prefill":
        prefill_workload(args, dev)
        return
    B = 2 * Bp
    D, H, F, V = 1024, 16, 4096, 8194
    t0 = time.time()
    # the deployed T3's speech embedding adds a learned position table (model.py:397-402)
    model = make_t3(n_layers=L, seed=args.seed, device=dev, learned_pos_emb=True)
    lens = uniform_lengths(Bp, 150, 600, seed=args.seed + 1)
    lps = lens + lens  # stacked rows: cond 0..Bp-1, null Bp..2Bp-1
    max_seq = max(lps) + 2 * bl
    eng = HipEngine(model, max_seq, torch.bfloat16, batch_size=B, page_table_seed=args.seed + 2)
    g = torch.Generator().manual_seed(args.seed + 3)
    prefixes = [torch.randn(lp, D, generator=g).to(torch.bfloat16) for lp in lens]
    sos = eng.prefix_forward([p.to(dev) for p in prefixes + prefixes])
    torch.cuda.synchronize(dev)
    log(f"model + prefill ready in {time.time() - t0:.1f}s (KV {L * eng.kv.bytes_per_layer / 2**30:.1f} GiB)")

    sc_in = scoring_inputs(n_pairs=Bp, bl=bl, vocab=V, seed=args.seed + 4, layout="stacked")
    step = DecodeStep(eng, model, n_pairs=Bp, block_size=bl, log_prior=sc_in.log_prior.to(dev), mask_id=MASK_ID,
                      stop_id=STOP_ID, num_steps=10, time_shift_tau=3.0, omnivoice_t_shift=0.5, cfg_scale=0.5)
    step.xt.copy_(sc_in.xt.to(dev))
    step.k_step.copy_(sc_in.k_step.to(dev))
    step.capture(lps, sos)
    for _ in range(args.warmup):
        step.replay()
    torch.cuda.synchronize(dev)
    st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize(dev)
    st.record()
    for _ in range(args.steps):
        step.replay()
    en.record()
    torch.cuda.synchronize(dev)
    ms = st.elapsed_time(en) / args.steps
    log(f"step {ms:.3f} ms")

    # ---- per-kernel durations (HIP events around single launches, same stream) ----
    # Each launch takes the next layer's weights / KV pool, as the step does, so
    # no launch finds its operands in the 256 MB MALL from the previous one.
    buf = eng._buffers(B, bl)
    plan = eng._g_plan
    N = B * bl
    layer = [0]

    def nxt():
        layer[0] = (layer[0] + 1) % L
        return layer[0]
    ms_swiglu = time_launches(lambda: kernels.gemm_swiglu(buf.normed, eng._w[nxt()]["wgu"], buf.act), 20, dev)
    ms_qkv = time_launches(lambda: kernels.gemm_qkv_rope_kv(buf.normed, eng._w[nxt()]["wqkv"], eng._cos, eng._sin,
                                                            buf.pos0, bl, buf.q, eng.kv.pools[layer[0]],
                                                            eng.kv.table), 20, dev)
    # o_proj / down_proj as the step runs them: with the residual add in the epilogue
    ms_o = time_launches(lambda: kernels.gemm_bf16_residual(buf.attn, eng._w[nxt()]["wo"], buf.delta), 20, dev)
    ms_down = time_launches(lambda: kernels.gemm_bf16_residual(buf.act, eng._w[nxt()]["wd"], buf.delta), 20, dev)
    # the vendor library on the gate/up shape (hipBLASLt through F.linear, plain bf16 store, no SiLU):
    # what the part gives a plain GEMM of this size, for context next to the fused kernel.  Both are
    # timed the same way here, 20 calls over four layers' weights replayed as one graph, which counts
    # every kernel the library launches but no host work (single event-timed launches add ~10 us to
    # the library's call)
    ms_vendor = time_graphs([lambda li=li: torch.nn.functional.linear(buf.normed, eng._w[li]["wgu"])
                             for li in range(4)], 20, dev)
    ms_swiglu_graph = time_graphs([lambda li=li: kernels.gemm_swiglu(buf.normed, eng._w[li]["wgu"], buf.act)
                                   for li in range(4)], 20, dev)
    eager_plan = AttnPlan(plan.kv_len.tolist(), bl, H, dev)
    # four layers' pools in turn (each ~0.9 GB of K/V, so no replay finds its pool in the 256 MB MALL),
    # replayed as graphs like the step
    ms_attn = time_graphs([lambda li=li: eager_plan.run(buf.q.view(B, bl, H, 64), eng.kv.pools[li], eng.kv.table,
                                                        buf.attn.view(B, bl, H, 64), 0.125) for li in range(4)],
                          20, dev)
    # scoring on two rotated logits sets (the 268 MB input must not sit in the 256 MB MALL)
    sets = [eng._g_logits]
    spare = torch.empty_like(eng._g_logits_buf)
    spare.copy_(eng._g_logits_buf)
    sets.append(spare[..., :V])
    # replayed as graphs (one per input set), like the step, so no host launch time is counted
    ms_score = time_graphs([lambda lg=lg: step.scorer(lg, step.xt, step.k_step, layout="stacked") for lg in sets],
                           20, dev)

    peak_meas = measured_mfma_peak(dev)
    peak_meas_const = measured_mfma_peak(dev, random_operands=False)
    csrc = torch.empty(COPY_BYTES, dtype=torch.uint8, device=dev).fill_(1)
    cdst = torch.empty_like(csrc)
    ms_copy = time_launches(lambda: cdst.copy_(csrc), 10, dev)
    copy_gbs = 2 * COPY_BYTES / (ms_copy * 1e-3) / 1e9
    read_gbs = measured_read_rate(csrc, dev)
    del csrc, cdst
    flops_swiglu = 2.0 * N * (2 * F) * D
    tf_swiglu = flops_swiglu / (ms_swiglu * 1e-3) / 1e12
    kv_len = plan.kv_len.tolist()
    attn_bytes = sum(kv_len) * H * 64 * 2 * 2 + 2 * N * H * 64 * 2 + sum((k + 15) // 16 for k in kv_len) * 4
    score_bytes = B * bl * V * 2 + V * 4 + Bp * bl * (8 + 8 + 4 + 1 + 8) + Bp * 13
    gbs_attn = attn_bytes / (ms_attn * 1e-3) / 1e9
    gbs_score = score_bytes / (ms_score * 1e-3) / 1e9
    proj_flops = 2.0 * N * D * (3 * H * 64 + H * 64 + 2 * F + F) * L + 2.0 * N * D * V
    log(f"vendor plain GEMM on the gate/up shape (hipBLASLt), graph-timed: {ms_vendor*1e3:.1f} us "
        f"({flops_swiglu / (ms_vendor * 1e-3) / 1e12:.0f} TF/s); gate/up + SiLU timed the same way: "
        f"{ms_swiglu_graph*1e3:.1f} us")
    log(f"gate/up {ms_swiglu*1e3:.1f} us ({tf_swiglu:.0f} TF/s), qkv {ms_qkv*1e3:.1f}, o {ms_o*1e3:.1f}, "
        f"down {ms_down*1e3:.1f}, attn {ms_attn*1e3:.1f} us ({gbs_attn:.0f} GB/s), score {ms_score*1e3:.1f} us "
        f"({gbs_score:.0f} GB/s)")

    traffic = None
    tpath = os.path.join(ROOT, "profiles", "gemm_swiglu_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("bytes_per_launch")

    secondary = None
    if not args.no_secondary:
        secondary = secondary_workloads(args, dev, model, eng, prefixes, lps, sc_in)

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(model, eng, lps, bl, sc_in, args.cpu_layers, L)

    tok_s = Bp * bl / (ms * 1e-3)
    out = {
        "metric": "speech tokens/sec, 30-layer T3 step at B=256; attn/score HBM GB/s % peak",
        "value": round(tok_s, 1),
        "unit": "speech tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded random-init weights of the T3 architecture, random prefixes)",
        "config": {"workload": "T3 block-diffusion decode step: embed + 30-layer backbone + speech head + "
                               "CFG/PMI/quantile unmask", "pairs": Bp, "rows": B, "block": bl, "layers": L,
                   "hidden": D, "heads": H, "ffn": F, "vocab": V, "prefix_len": "U[150,600] per pair",
                   "page_table": "shuffled", "cfg_w": 0.5, "quantile_tau": 3.0, "K": 10},
        "rows_positions_per_s": round(B * bl / (ms * 1e-3), 1),
        # one block costs K = 10 denoise steps + 1 commit forward (same shape)
        "committed_speech_tokens_per_s_est": round(tok_s / 11.0, 1),
        "projection_tflops": round(proj_flops / (ms * 1e-3) / 1e12, 1),
        "roofline": {"kernel": "gemm_pt_kernel<swiglu> (persistent; gate/up + SiLU*up, M=%d N=%d K=%d)" % (N, 2 * F, D),
                     "bound": "mfma", "achieved": round(tf_swiglu, 1), "peak": BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tf_swiglu / BF16_PEAK_TFLOPS, 4), "traffic": traffic,
                     "peak_measured": round(peak_meas, 1), "frac_of_measured": round(tf_swiglu / peak_meas, 4),
                     "peak_measured_constant_operands": round(peak_meas_const, 1),
                     "vendor_gemm": {"library": "hipBLASLt (torch F.linear), same shape, plain store without SiLU",
                                     "timing": "20 calls over four layers' weights in one graph replay",
                                     "us": round(ms_vendor * 1e3, 1),
                                     "ours_same_timing_us": round(ms_swiglu_graph * 1e3, 1),
                                     "achieved": round(flops_swiglu / (ms_vendor * 1e-3) / 1e12, 1),
                                     "frac": round(flops_swiglu / (ms_vendor * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4)}},
        "kernels": {
            "attention": {"us": round(ms_attn * 1e3, 1), "achieved": round(gbs_attn, 1), "peak": HBM_PEAK_GBS,
                          "unit": "GB/s", "frac": round(gbs_attn / HBM_PEAK_GBS, 4),
                          "frac_of_measured_read": round(gbs_attn / read_gbs, 4)},
            "scoring": {"us": round(ms_score * 1e3, 1), "achieved": round(gbs_score, 1), "peak": HBM_PEAK_GBS,
                        "unit": "GB/s", "frac": round(gbs_score / HBM_PEAK_GBS, 4),
                        "frac_of_measured_read": round(gbs_score / read_gbs, 4)},
            "gemm_us": {"qkv_rope_kv": round(ms_qkv * 1e3, 1), "o_proj": round(ms_o * 1e3, 1),
                        "gate_up_swiglu": round(ms_swiglu * 1e3, 1), "down": round(ms_down * 1e3, 1)},
            "measured_copy_GBps": round(copy_gbs, 1),
            "measured_read_GBps": round(read_gbs, 1),
        },
        "cpu_baseline": cpu,
        "secondary": secondary,
    }
    print(json.dumps(out), flush=True)


def secondary_workloads(args, dev, model, eng, prefixes, lps, sc_in):
    """The other workloads' headline figures, measured in the same run after the step: the prefix
    prefill of the step's 512 rows (through the step's engine, rewriting the same KV), continuous
    batching on the same model, 30 layers of attention over the stress shape, and the vocoder's
    elementwise family and chunk stitch.  The full objects come from ``--workload prefill | serve |
    attn_stress | vocoder``."""
    L, D = args.layers, 1024
    embs = [p.to(dev) for p in prefixes + prefixes]
    ms_pf, wall_pf = time_prefill(eng, embs, 2, dev)
    tokens = sum(lps)
    tf_pf = prefill_flops(lps, L, D) / (ms_pf * 1e-3) / 1e12
    log(f"prefill: {tokens} prefix tokens, {ms_pf:.1f} ms, {tokens / (ms_pf * 1e-3):.0f} tokens/s, {tf_pf:.0f} TF/s")
    del embs
    sv = serve(args, dev, model)
    torch.cuda.empty_cache()
    st = attn_stress(args, dev)
    torch.cuda.empty_cache()
    voc_args = copy.copy(args)
    voc_args.no_cpu_baseline = True
    vc = vocoder_workload(voc_args, dev)
    torch.cuda.empty_cache()
    qf = quant_figures(args, dev)
    torch.cuda.empty_cache()
    ms_q4 = quant_step(args, dev, model, prefixes, lps, sc_in, bits=4)
    return {
        "prefill": {"value": round(tokens / (ms_pf * 1e-3), 1), "unit": "prefix tokens/s", "ms": round(ms_pf, 3),
                    "wall_ms": round(wall_pf, 2), "prefix_tokens": tokens, "rows": len(lps), "layers": L,
                    "achieved_tflops": round(tf_pf, 1), "frac": round(tf_pf / BF16_PEAK_TFLOPS, 4)},
        "serve": {"value": sv["value"], "unit": sv["unit"], "requests": sv["config"]["requests"],
                  "slots": sv["config"]["slots"], "block": sv["config"]["block"], "ticks": sv["ticks"],
                  "ms_per_tick": sv["ms_per_tick"], "ttfc_s_median": sv["ttfc_s_median"], "wall_s": sv["wall_s"]},
        "attn_stress": {"value": st["value"], "unit": st["unit"], "ms_30_layers": st["ms_per_step"],
                        "frac": st["roofline"]["frac"], "sequences": st["config"]["sequences"],
                        "block": st["config"]["block"], "layers": st["config"]["layers"]},
        "vocoder": {"value": vc["value"], "unit": vc["unit"], "kernel": "residual_bias_snake",
                    "frac": vc["roofline"]["frac"], "shape": [vc["config"]["batch"], vc["config"]["channels"],
                                                              vc["config"]["samples"]],
                    "stitch_us": vc["kernels"]["stitch"]["us"], "stitch_jobs": vc["kernels"]["stitch"]["jobs"]},
        "quant": {"projections": {f"bits{b}": {"ms_30_layers": round(ms, 4), "tflops": round(tf, 1),
                                               "frac": round(tf / BF16_PEAK_TFLOPS, 4),
                                               "fused_kernel": {"ms_30_layers": round(ms_f, 4),
                                                                "tflops": round(tf_f, 1)}}
                                  for b, (ms, tf, ms_f, tf_f) in qf.items()},
                  "route": "each weight dequantised once into bf16 scratch (timed), then the bf16 GEMM",
                  "shapes": "qkv 3072x1024, o 1024x1024, gate/up 8192x1024, down 1024x4096 at M = 8192",
                  "step_4bit": {"ms_per_step": round(ms_q4, 4),
                                "value": round(args.pairs * args.block / (ms_q4 * 1e-3), 1),
                                "unit": "speech tokens/s"}},
    }


COPY_BYTES = 1 << 30


def measured_mfma_peak(dev, random_operands=True):
    """Sustained bf16 MFMA TFLOP/s of the register-only calibration kernel
    (8 waves per SIMD, 2000 rounds of 8 independent 32x32x16 MFMAs) on random
    operands spread like the step's (the default) or on few-bit constants."""
    from yapd_amd import kernels
    blocks, iters = 2048, 2000
    out = torch.empty(blocks * 256, dtype=torch.float32, device=dev)
    flops = kernels.mfma_peak_probe(blocks, iters, out, random_operands)
    ms = time_launches(lambda: kernels.mfma_peak_probe(blocks, iters, out, random_operands), 5, dev)
    return flops / (ms * 1e-3) / 1e12


def measured_read_rate(src, dev):
    """Streaming HBM read rate (GB/s) of the read calibration kernel over `src`
    (1 GiB, four times the 256 MB MALL, so each pass comes from HBM): 4
    workgroups of 256 threads per CU, each streaming a contiguous share with
    eight non-temporal 16-byte loads in flight per thread."""
    from yapd_amd import kernels
    blocks = 4 * torch.cuda.get_device_properties(dev).multi_processor_count
    out = torch.empty(blocks * 256, dtype=torch.int32, device=dev)
    nbytes = kernels.hbm_read_probe(src, blocks, out)
    ms = time_launches(lambda: kernels.hbm_read_probe(src, blocks, out), 10, dev)
    return nbytes / (ms * 1e-3) / 1e9


def attn_stress(args, dev):
    """30 layers of block attention back to back: 256 sequences, prefixes
    round(exp(U[ln 64, ln 2048])), block 16, 16 x 64 heads; each layer's pages
    are distinct random pages of its own 65,536-page pool (4 GiB per layer).
    Only the referenced pages are filled (N(0, 1) bf16)."""
    import numpy as np
    from yapd_amd.paged import AttnPlan
    from yapd_amd.synthetic import log_uniform_lengths
    rows, bl, H, n_pages, L = 256, 16, 16, 65536, args.layers
    lengths = log_uniform_lengths(rows, 64, 2048, seed=args.seed)
    kv_len = [x + bl for x in lengths]
    ppr = (max(kv_len) + 15) // 16
    g = torch.Generator(device=dev).manual_seed(args.seed)
    used = [(k + 15) // 16 for k in kv_len]
    n_used = sum(used)
    fill = torch.randn(n_used, 2, H, 1024, generator=g, device=dev).to(torch.bfloat16)
    pools, tables = [], []
    for layer in range(L):
        perm = np.random.default_rng(args.seed * 1000 + layer).permutation(n_pages)[: rows * ppr]
        table = torch.from_numpy(perm.reshape(rows, ppr).astype(np.int32)).to(dev)
        pool = torch.empty(n_pages, 2, H, 1024, dtype=torch.bfloat16, device=dev)
        idx = torch.cat([table[r, :u] for r, u in enumerate(used)]).long()
        pool.index_copy_(0, idx, fill)
        pools.append(pool)
        tables.append(table)
    del fill
    q = torch.randn(rows, bl, H, 64, generator=g, device=dev).to(torch.bfloat16)
    out = torch.empty_like(q)
    plan = AttnPlan(kv_len, bl, H, dev)
    torch.cuda.synchronize(dev)

    def all_layers():
        for layer in range(L):
            plan.run(q, pools[layer], tables[layer], out, 0.125)
    ms = time_launches(all_layers, max(args.steps // 4, 3), dev)
    byts = L * (sum(kv_len) * H * 64 * 2 * 2 + 2 * rows * bl * H * 64 * 2 + n_used * 4)
    gbs = byts / (ms * 1e-3) / 1e9
    log(f"attention stress: {L} layers {ms:.3f} ms, {gbs:.0f} GB/s")
    del pools, tables
    return {
        "metric": "block attention HBM GB/s, 30 layers back to back (attention stress)", "value": round(gbs, 1),
        "unit": "GB/s", "n_gpus": 1, "ms_per_step": round(ms, 4), "higher_is_better": True, "dtype": "bf16",
        "data": "synthetic (N(0,1) K/V/q, random distinct pages)",
        "config": {"workload": "paged block attention", "sequences": rows, "block": bl, "heads": H,
                   "prefix_len": "round(exp(U[ln64, ln2048]))", "pool_pages_per_layer": n_pages, "layers": L,
                   "kv_positions_per_layer": sum(kv_len)},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes_per_layer": byts // L}}


def time_prefill(eng, embs, reps, dev):
    """(device ms, wall ms) per ``eng.prefix_forward(embs)``, averaged over ``reps`` calls."""
    torch.cuda.synchronize(dev)
    st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.time()
    st.record()
    for _ in range(reps):
        eng.prefix_forward(embs)
    en.record()
    torch.cuda.synchronize(dev)
    return st.elapsed_time(en) / reps, (time.time() - t0) * 1e3 / reps


def prefill_flops(lps, L, D):
    """Algorithmic flops of a prefill: the projections of every real prefix token plus causal attention."""
    return 2.0 * sum(lps) * D * 16384 * L + sum(4.0 * 16 * 64 * lp * (lp + 1) / 2 for lp in lps) * L


def prefill_workload(args, dev):
    """Prefix prefill (HipEngine.prefix_forward, engines/flashinfer.py:678-854 semantics) of the
    step's 512 rows: prefixes U[150, 600] per pair (cond and null rows share the length), 30
    layers, causal, in packed steps of 64-token segments writing the paged KV.  Algorithmic work:
    the projections of the real prefix tokens (2 * D * 16,384 flops per token and layer) plus
    causal attention; any padding the engine computed would count against the rate."""
    from yapd_amd.engines.hip import HipEngine
    from yapd_amd.synthetic import make_t3, uniform_lengths
    Bp, L, D = args.pairs, args.layers, 1024
    # the deployed T3's speech embedding adds a learned position table (model.py:397-402)
    model = make_t3(n_layers=L, seed=args.seed, device=dev, learned_pos_emb=True)
    lens = uniform_lengths(Bp, 150, 600, seed=args.seed + 1)
    lps = lens + lens
    eng = HipEngine(model, max(lps) + 64, torch.bfloat16, batch_size=len(lps), page_table_seed=args.seed + 2)
    g = torch.Generator().manual_seed(args.seed + 3)
    embs = [torch.randn(lp, D, generator=g).to(torch.bfloat16).to(dev) for lp in lps]
    eng.prefix_forward(embs)  # warm-up (plans, buffers)
    ms, wall = time_prefill(eng, embs, max(2, args.steps // 5), dev)
    tokens = sum(lps)
    flops = prefill_flops(lps, L, D)
    tflops = flops / (ms * 1e-3) / 1e12
    log(f"prefill: {len(lps)} rows, {tokens} prefix tokens, {ms:.1f} ms ({wall:.1f} ms wall), "
        f"{tokens / (ms * 1e-3):.0f} tokens/s, {tflops:.0f} TF/s")
    cpu = None
    if not args.no_cpu_baseline:
        from dataclasses import replace
        from oracle import llama as OL
        threads = os.cpu_count() or 1
        torch.set_num_threads(threads)
        n_rows, n_layers = 8, 2
        bb = OL.backbone_from_model(model, max_pos=max(lps) + 64, dtype=torch.bfloat16)
        bb = replace(bb, layers=bb.layers[:n_layers])
        cache = OL.KVCache.empty(n_layers, n_rows, max(lps), 16, 64, torch.bfloat16)
        sample = [e.cpu() for e in embs[:n_rows]]
        t = time.time()
        OL.prefix_forward(bb, sample, cache)
        dt = (time.time() - t) * L / n_layers
        cpu = {"value": round(sum(lps[:n_rows]) / dt, 1), "unit": "prefix tokens/s", "cores": threads, "kind": "port",
               "sample": f"oracle torch-CPU bf16 causal prefill of {n_rows} rows ({sum(lps[:n_rows])} tokens), "
                         f"{n_layers} of {L} layers, time x {L}/{n_layers}"}
    print(json.dumps({
        "metric": "prefix prefill tokens/sec, 30-layer T3, 512 rows", "value": round(tokens / (ms * 1e-3), 1),
        "unit": "prefix tokens/s", "n_gpus": 1, "ms_per_step": round(ms, 3), "higher_is_better": True,
        "dtype": "bf16", "data": "synthetic (seeded random-init T3 weights, N(0,1) prefix embeddings)",
        "config": {"workload": "prefix prefill (causal, packed steps of 64-token segments, paged KV)", "rows": len(lps),
                   "prefix_len": "U[150,600] per pair", "layers": L, "prefix_tokens": tokens,
                   "wall_ms": round(wall, 2)},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / BF16_PEAK_TFLOPS, 4), "flops_per_prefill": flops, "traffic": None},
        "cpu_baseline": cpu}), flush=True)


def vocoder_workload(args, dev):
    """The HiFT generator's elementwise ops between its convolutions (server/kernels.py:35-67)
    on the last upsampling stage of a 48-job micro-batch of 80-token chunks: 160 mel frames
    x 120 = 19,200 samples + 1 from the reflection pad, 64 channels, fp32.  Two input sets
    alternate so no launch finds its inputs in the 256 MB MALL.  Roofline kernel:
    residual_bias_snake (the resblock's fused residual add + next Snake, 16 B per element)."""
    from yapd_amd.vocoder import load_snake_extension
    ops = load_snake_extension()
    B, C, T = 48, 64, 19201
    n = B * C * T
    g = torch.Generator(device=dev).manual_seed(args.seed)
    sets = [[torch.randn(B, C, T, generator=g, device=dev) for _ in range(3)] for _ in range(2)]
    alpha = [torch.rand(C, generator=g, device=dev) * 2 + 0.2 for _ in range(3)]
    bias = torch.randn(C, generator=g, device=dev) * 0.1
    if args.kernel_sample:  # for rocprofv3 --pmc: the roofline kernel and the copy calibration, x3 each
        src = torch.empty(COPY_BYTES, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize(dev)
        for i in range(3):
            ops.residual_bias_snake(*sets[i % 2][:2], bias, alpha[0])
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize(dev)
        print(json.dumps({"kernel_sample": "residual_bias_snake [%d, %d, %d] x3; copy %d bytes x3"
                                           % (B, C, T, COPY_BYTES)}))
        return None
    it = [0]

    def pick():
        it[0] ^= 1
        return sets[it[0]]
    cases = {  # name -> (launch, fp32 tensors read + written per element)
        "snake": (lambda: ops.snake(pick()[0], alpha[0]), 2),
        "snake_bias": (lambda: ops.snake_bias(pick()[0], alpha[0], bias), 2),
        "residual_bias": (lambda: ops.residual_bias(*pick()[:2], bias), 3),
        "residual_bias_snake": (lambda: ops.residual_bias_snake(*pick()[:2], bias, alpha[0]), 4),
        "branch_start": (lambda: ops.branch_start(*pick()[:2], *alpha), 6),
        "mean3": (lambda: ops.mean3(*pick()), 4),
    }
    res = {}
    for name, (fn, tensors) in cases.items():
        ms = time_launches(fn, max(args.steps, 10), dev)
        res[name] = {"us": round(ms * 1e3, 1), "gbs": round(tensors * 4 * n / (ms * 1e-3) / 1e9, 1)}
        log(f"{name}: {ms * 1e3:.1f} us, {res[name]['gbs']:.0f} GB/s")
    res["stitch"] = stitch_sample(args, dev, g)
    dom = res["residual_bias_snake"]
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "vocoder_residual_bias_snake_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("bytes_per_launch")
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import vocoder as OV
        # the whole workload, repeated until at least 10 s of single-threaded numpy (at most 8 passes)
        x, r = (t.cpu().numpy() for t in sets[0][:2])
        b_np, a_np = bias.cpu().numpy(), alpha[0].cpu().numpy()
        passes, t0 = 0, time.time()
        while passes < 8 and (passes == 0 or time.time() - t0 < 10.0):
            OV.residual_bias_snake(x, r, b_np, a_np)
            passes += 1
        dt = time.time() - t0
        cpu = {"value": round(passes * 4 * 4 * n / dt / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
               "sample": f"residual_bias_snake on [{B}, {C}, {T}] x {passes} with the numpy oracle (float64 Snake), "
                         f"one thread, {dt:.1f} s"}
    return {
        "metric": "HiFT vocoder elementwise HBM GB/s (residual_bias_snake)", "value": dom["gbs"], "unit": "GB/s",
        "n_gpus": 1, "ms_per_step": round(dom["us"] / 1e3, 4), "higher_is_better": True, "dtype": "f32",
        "data": "synthetic (N(0,1) activations, alpha U[0.2, 2.2], bias N(0, 0.01))",
        "config": {"workload": "HiFT last-stage elementwise ops", "batch": B, "channels": C, "samples": T},
        "roofline": {"bound": "hbm", "achieved": dom["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dom["gbs"] / HBM_PEAK_GBS, 4), "bytes_per_launch": 4 * 4 * n, "traffic": traffic},
        "kernels": res, "cpu_baseline": cpu}


def stitch_sample(args, dev, g):
    """Chunk stitching of the streaming vocoder (voc_stitch.hip) on a bulk micro-batch: 48 jobs,
    96-token windows (16 tokens of lookback + 80 emitted), each blending a 480-sample tail and
    withholding the next.  Bytes per job: the samples read (fp32), the tail read and written
    (fp32) and the PCM written (int16).  Also times the batch's copy to pinned host memory as
    int16 PCM against the fp32 waveforms a host-side stitch would copy."""
    from yapd_amd import kernels as K
    nj, ntok, emit_off, fade = 48, 96, 16, 480
    wav = torch.randn(nj, ntok * 960, generator=g, device=dev) * 0.5
    lo = emit_off * 960 - fade
    n_seg = ntok * 960 - lo
    n_out = n_seg - fade
    jobs = torch.tensor([[i, lo, n_seg, fade, 0, 0, n_out, i, i, i * n_out, 0, 0] for i in range(nj)],
                        dtype=torch.int32, device=dev)
    fin = torch.linspace(0, 1, fade, device=dev)
    fout = 1 - fin
    trim = torch.ones(960, device=dev)
    t_in = torch.randn(nj, fade, generator=g, device=dev)
    t_out = torch.empty_like(t_in)
    pcm = torch.empty(nj * n_out, dtype=torch.int16, device=dev)
    ms = time_launches(lambda: K.voc_stitch(wav, jobs, fin, fout, trim, t_in, t_out, pcm), max(args.steps, 10), dev)
    nbytes = nj * (4 * n_seg + 8 * fade + 2 * n_out)
    pin16 = torch.empty(pcm.numel(), dtype=torch.int16, pin_memory=True)
    pin32 = torch.empty(wav.shape, dtype=torch.float32, pin_memory=True)
    ms16 = time_launches(lambda: pin16.copy_(pcm, non_blocking=True), 10, dev)
    ms32 = time_launches(lambda: pin32.copy_(wav, non_blocking=True), 10, dev)
    out = {"us": round(ms * 1e3, 1), "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1), "bytes": nbytes,
           "jobs": nj, "samples_out": nj * n_out, "d2h_int16_us": round(ms16 * 1e3, 1),
           "d2h_fp32_us": round(ms32 * 1e3, 1)}
    log(f"stitch: {out['us']} us for {nj} jobs ({out['gbs']:.0f} GB/s); PCM to host {out['d2h_int16_us']} us "
        f"as int16 vs {out['d2h_fp32_us']} us for the fp32 waveforms")
    return out


def serve(args, dev, model=None):
    """Continuous batching (server/engine.py FlashEngine defaults): 128 slots, block 16,
    K = 10 denoise steps, temperature 0.6, position temperature 5.0, CFG 1.0, tau 0.1;
    requests with prefixes U[100, 300] and speech budgets of 208 tokens (13 blocks)
    arrive all at once; the timed window runs from the first tick to the last commit.
    ``model`` (the same seeded T3) is built when not given."""
    from yapd_amd.serve import HipFlashEngine, Request
    from yapd_amd.synthetic import MASK_ID, SOS_ID, STOP_ID, make_t3, uniform_lengths
    L, n_req, n_speech = args.layers, args.requests, 208
    if model is None:
        model = make_t3(n_layers=L, seed=args.seed, device=dev)
    V = model.speech_head.weight.shape[0]
    g = torch.Generator().manual_seed(args.seed + 1)
    prior = torch.distributions.Dirichlet(torch.full((V,), 0.1)).sample()
    log_prior = prior.clamp_min(1e-8).log()
    eng = HipFlashEngine(model, log_prior=log_prior, mask_id=MASK_ID, stop_id=STOP_ID, codec_vocab=SOS_ID,
                         max_active=128, max_prefix_tokens=320, max_speech_tokens=624, num_steps=10,
                         temperature=0.6, time_shift_tau=0.1, omnivoice_t_shift=0.5, cfg_scale=1.0,
                         position_temperature=5.0, prefill_max=16, block_size=16, page_table_seed=args.seed + 2)
    sos = model.speech_emb.weight[SOS_ID].detach().to(torch.bfloat16)
    lens = uniform_lengths(n_req, 100, 300, seed=args.seed + 3)
    reqs = []
    for i, lp in enumerate(lens):
        pre = (torch.randn(lp, model.speech_emb.weight.shape[1], generator=g) * 0.5).to(dev, torch.bfloat16)
        pre[-1] = sos
        reqs.append(Request(rid=i, prefix=pre, n_speech=n_speech))
    # warm-up: a few requests through the same engine (buffers, plans)
    for r in reqs[:8]:
        eng.submit(r)
    eng.run_until_idle()
    torch.cuda.synchronize(dev)
    eng.finished.clear()
    eng.commit_blocks = 0
    t0_tick = eng.tick_id
    t0 = time.perf_counter()
    for r in reqs[8:]:
        eng.submit(r)
    eng.run_until_idle()
    torch.cuda.synchronize(dev)
    secs = time.perf_counter() - t0
    done = [r for r in reqs[8:] if r.t3_done]
    toks = sum(len(r.committed) for r in done)
    ticks = eng.tick_id - t0_tick
    ttfc = sorted(r.t_first_commit - r.t_recv for r in done if r.t_first_commit > 0)
    log(f"serve: {len(done)} requests, {toks} committed tokens in {secs:.2f} s over {ticks} ticks "
        f"({secs / max(ticks, 1) * 1e3:.2f} ms/tick)")
    return {
        "metric": "committed speech tokens/sec, continuous batching (128 slots, 30 layers)",
        "value": round(toks / secs, 1), "unit": "committed speech tokens/s", "n_gpus": 1,
        "higher_is_better": True, "dtype": "bf16",
        "data": "synthetic (seeded random-init T3 weights, random prefixes, Dirichlet(0.1) prior)",
        "config": {"workload": "continuous-batching decode (admission, denoise, commit, retirement)",
                   "requests": len(done), "slots": 128, "block": 16, "K": 10, "layers": L,
                   "prefix_len": "U[100,300]", "n_speech": n_speech, "temperature": 0.6,
                   "position_temperature": 5.0, "cfg_w": 1.0},
        "ticks": ticks, "ms_per_tick": round(secs / max(ticks, 1) * 1e3, 3),
        "ttfc_s_median": round(ttfc[len(ttfc) // 2], 3) if ttfc else None,
        "commit_blocks": eng.commit_blocks, "wall_s": round(secs, 3)}


def quant_figures(args, dev):
    """The four projections of 30 layers (qkv 3072x1024, o 1024x1024, gate/up
    8192x1024, down 1024x4096) as 4-bit and 8-bit affine-quantised GEMMs
    (group 64, MLX layout, fp16 scales/biases) at M = 8192; weights N(0, 0.02).
    Each call dequantises its weight once into a bf16 scratch (inside the
    timing) and runs the bf16 GEMM, the route the library takes at this many
    rows; the fused kernel (dequantising every W tile again per tile row) is
    timed beside it.  Returns {bits: (ms, TFLOP/s, fused ms, fused TFLOP/s)}."""
    from yapd_amd.quant import qgemm_affine, quantize_affine
    M, L = 8192, args.layers
    shapes = [(3072, 1024), (1024, 1024), (8192, 1024), (1024, 4096)]
    g = torch.Generator(device=dev).manual_seed(args.seed)
    A = {k: torch.randn(M, k, generator=g, device=dev).to(torch.bfloat16) for k in (1024, 4096)}
    outs = {n: torch.empty(M, n, dtype=torch.bfloat16, device=dev) for n, _ in shapes}
    scratch = torch.empty(max(n * k for n, k in shapes), dtype=torch.bfloat16, device=dev)
    flops = 2.0 * M * sum(n * k for n, k in shapes) * L
    res = {}
    for bits in (4, 8):
        layers = [[quantize_affine(torch.randn(n, k, generator=g, device=dev) * 0.02, bits) for n, k in shapes]
                  for _ in range(L)]
        torch.cuda.synchronize(dev)

        def all_layers(scr):
            for lw in layers:
                for (n, k), (pk, sc, bi) in zip(shapes, lw):
                    qgemm_affine(A[k], pk, sc, bi, bits, out=outs[n], scratch=scr)
        ms = time_launches(lambda: all_layers(scratch), 5, dev)
        ms_f = time_launches(lambda: all_layers(None), 5, dev)
        res[bits] = (ms, flops / (ms * 1e-3) / 1e12, ms_f, flops / (ms_f * 1e-3) / 1e12)
        log(f"quant {bits}-bit: {L} layers {ms:.3f} ms, {res[bits][1]:.0f} TF/s dequantised once "
            f"(fused kernel {ms_f:.3f} ms, {res[bits][3]:.0f} TF/s)")
        del layers
    return res


def quant_projections(args, dev):
    res = quant_figures(args, dev)
    ms4, tf4, ms4_f, tf4_f = res[4]
    print(json.dumps({
        "metric": "affine-quantised projection TFLOP/s, 30 layers at M=8192", "value": round(tf4, 1),
        "unit": "TFLOP/s", "n_gpus": 1, "ms_per_step": round(ms4, 4), "higher_is_better": True, "dtype": "bf16",
        "data": "synthetic (weights N(0,0.02) quantised; A N(0,1))",
        "config": {"workload": "qkv/o/gate-up/down dequant GEMMs", "M": 8192, "layers": args.layers, "group": 64,
                   "bits": 4, "route": "W dequantised once into bf16 scratch (timed), then the bf16 GEMM"},
        "bits8": {"ms": round(res[8][0], 4), "tflops": round(res[8][1], 1),
                  "frac": round(res[8][1] / BF16_PEAK_TFLOPS, 4)},
        "fused_kernel": {"bits4_tflops": round(tf4_f, 1), "bits8_tflops": round(res[8][3], 1)},
        "roofline": {"bound": "mfma", "achieved": round(tf4, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tf4 / BF16_PEAK_TFLOPS, 4)}}), flush=True)


def quant_step(args, dev, model, prefixes, lps, sc_in, bits=4):
    """The benched step on ``bits``-bit weights: a quantised engine on the same model, prefixes and
    block (every layer projection affine-quantised, engines/mlx.py:221-255).  Returns ms per step."""
    from yapd_amd.engines.hip import HipEngine
    from yapd_amd.step import DecodeStep
    from yapd_amd.synthetic import MASK_ID, STOP_ID
    Bp, bl = args.pairs, args.block
    eng = HipEngine(model, max(lps) + 2 * bl, torch.bfloat16, batch_size=2 * Bp, page_table_seed=args.seed + 2,
                    quant_bits=bits)
    sos = eng.prefix_forward([p.to(dev) for p in prefixes + prefixes])
    step = DecodeStep(eng, model, n_pairs=Bp, block_size=bl, log_prior=sc_in.log_prior.to(dev), mask_id=MASK_ID,
                      stop_id=STOP_ID, num_steps=10, time_shift_tau=3.0, omnivoice_t_shift=0.5, cfg_scale=0.5)
    step.xt.copy_(sc_in.xt.to(dev))
    step.k_step.copy_(sc_in.k_step.to(dev))
    step.capture(lps, sos)
    for _ in range(3):
        step.replay()
    torch.cuda.synchronize(dev)
    st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    st.record()
    for _ in range(10):
        step.replay()
    en.record()
    torch.cuda.synchronize(dev)
    ms = st.elapsed_time(en) / 10
    log(f"{bits}-bit step {ms:.3f} ms")
    del step, eng
    torch.cuda.empty_cache()
    return ms


def kernel_sample(dev, Bp, bl):
    """Every kernel of the step at the bench shape, three dispatches each and in this order, for
    rocprofv3 --pmc (FETCH_SIZE / WRITE_SIZE / MFMA counters per dispatch): gate/up + SiLU, QKV +
    RoPE + KV write, o_proj + residual, down_proj + residual, RMSNorm, speech head (two launches
    per call), paged attention over three layers' pools (each ~0.9 GB of K/V, so no dispatch finds
    its pool in the 256 MB MALL), scoring on two alternating 268 MB logits sets, the 4-bit
    quantised gate/up and down projections at M = 8192, then a plain 1 GiB device copy (the
    counter calibration)."""
    from yapd_amd import kernels
    from yapd_amd.engines.hip import HipEngine
    from yapd_amd.paged import AttnPlan
    from yapd_amd.scoring import BlockScorer
    from yapd_amd.synthetic import MASK_ID, STOP_ID, make_t3, uniform_lengths
    B, D, H, F, V = 2 * Bp, 1024, 16, 4096, 8194
    N = B * bl
    model = make_t3(n_layers=3, seed=0, device=dev)
    lens = uniform_lengths(Bp, 150, 600, seed=1)
    starts = lens + lens
    eng = HipEngine(model, max(starts) + 2 * bl, torch.bfloat16, batch_size=B, page_table_seed=2)
    g = torch.Generator(device=dev).manual_seed(0)
    for pool in eng.kv.pools:
        pool.copy_(torch.randn(pool.shape, generator=g, device=dev, dtype=torch.bfloat16))
    buf = eng._buffers(B, bl)
    buf.pos0.copy_(torch.tensor(starts, dtype=torch.int32))
    normed = torch.randn(N, D, generator=g, device=dev).bfloat16()
    attn_in = torch.randn(N, D, generator=g, device=dev).bfloat16()
    act = torch.randn(N, F, generator=g, device=dev).bfloat16()
    resid = torch.randn(N, D, generator=g, device=dev).bfloat16()
    w = eng._w[0]
    head_w = model.speech_head.weight.detach().contiguous()
    ctx = torch.randn(B, 1, D, generator=g, device=dev).bfloat16()
    logits_buf = torch.zeros(B, bl, (V + 7) // 8 * 8, dtype=torch.bfloat16, device=dev)
    plan = AttnPlan([s + bl for s in starts], bl, H, dev)
    q = torch.randn(B, bl, H, 64, generator=g, device=dev).bfloat16()
    out = torch.empty_like(q)
    sets = [(torch.randn(B, bl, (V + 7) // 8 * 8, generator=g, device=dev) * 3).bfloat16() for _ in range(2)]
    log_prior = torch.log_softmax(torch.randn(V, generator=g, device=dev), 0)
    scorer = BlockScorer(n_pairs=Bp, block_size=bl, log_prior=log_prior, mask_id=MASK_ID, stop_id=STOP_ID,
                         num_steps=10, time_shift_tau=3.0, omnivoice_t_shift=0.5, cfg_scale=0.5, device=dev)
    xt = torch.full((Bp, bl), MASK_ID, dtype=torch.int64, device=dev)
    k_step = torch.zeros(Bp, dtype=torch.int64, device=dev)
    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize(dev)
    order = []

    def run(label, fn, reps=3):
        for i in range(reps):
            fn(i)
            order.append(label)
    run("gate_up_swiglu", lambda i: kernels.gemm_swiglu(normed, w["wgu"], buf.act))
    run("qkv_rope_kv", lambda i: kernels.gemm_qkv_rope_kv(normed, w["wqkv"], eng._cos, eng._sin, buf.pos0, bl, buf.q,
                                                          eng.kv.pools[0], eng.kv.table))
    run("o_proj_residual", lambda i: kernels.gemm_bf16_residual(attn_in, w["wo"], resid))
    run("down_proj_residual", lambda i: kernels.gemm_bf16_residual(act, w["wd"], resid))
    run("rmsnorm", lambda i: kernels.rmsnorm(resid, w["ln_in"], 1e-5, buf.normed))
    run("speech_head", lambda i: kernels.gemm_head_shift(normed.view(B, bl, D), ctx, head_w,
                                                         logits_buf[..., :V]))
    run("attention", lambda i: plan.run(q, eng.kv.pools[i], eng.kv.table, out, 0.125))
    run("scoring", lambda i: scorer(sets[i % 2][..., :V], xt, k_step, layout="stacked"))
    # the quantised projections at C5's M = 8192: 4-bit gate/up (N 8192, K 1024) and down (N 1024, K 4096)
    from yapd_amd.quant import qgemm_affine, quantize_affine
    q_gu, q_d = quantize_affine(w["wgu"], 4), quantize_affine(w["wd"], 4)
    out_gu = torch.empty(8192, 2 * F, dtype=torch.bfloat16, device=dev)
    out_d = torch.empty(8192, D, dtype=torch.bfloat16, device=dev)
    torch.cuda.synchronize(dev)
    run("qgemm4_gate_up", lambda i: qgemm_affine(normed[:8192], *q_gu, 4, out=out_gu))
    run("qgemm4_down", lambda i: qgemm_affine(act[:8192], *q_d, 4, out=out_d))
    run("copy_1GiB", lambda i: dst.copy_(src))
    torch.cuda.synchronize(dev)
    kv_len = plan.kv_len_host
    print(json.dumps({"kernel_sample": order, "M": N, "copy_bytes": COPY_BYTES,
                      "attention_bytes": sum(kv_len) * H * 64 * 2 * 2 + 2 * N * H * 64 * 2
                      + sum((k + 15) // 16 for k in kv_len) * 4,
                      "scoring_bytes": B * bl * V * 2 + V * 4 + Bp * bl * 29 + Bp * 13}), flush=True)


def host_cpu_info() -> dict:
    """The host's CPU model, sockets, threads per core (lscpu) and the thread counts used."""
    info = {"cpu_model": None, "sockets": None, "threads_per_core": None, "os_cpu_count": os.cpu_count(),
            "affinity_cpus": len(os.sched_getaffinity(0)), "torch_threads": torch.get_num_threads()}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
    except (OSError, subprocess.SubprocessError):
        out = ""
    for line in out.splitlines():
        key, _, val = line.partition(":")
        key, val = key.strip(), val.strip()
        if key == "Model name" and info["cpu_model"] is None:
            info["cpu_model"] = val
        elif key == "Socket(s)":
            info["sockets"] = int(val) if val.isdigit() else val
        elif key == "Thread(s) per core":
            info["threads_per_core"] = int(val) if val.isdigit() else val
    if info["cpu_model"] is None and os.path.exists("/proc/cpuinfo"):
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    info["cpu_model"] = line.split(":", 1)[1].strip()
                    break
    return info


def cpu_baseline(model, eng, lps, bl, sc_in, n_layers, L, runs=3):
    """Oracle (torch on the host) on a bounded sample of the same step, scaled to 30 layers:
    ``n_layers`` decoder layers at the full batch, the speech head and the scoring, each the
    median of ``runs`` timed runs after a warm-up, in bf16 (the step's dtype) and fp32."""
    from oracle import llama as OL
    from oracle import scoring as OS
    from oracle.schedule import omnivoice_unmask_schedule, quantile_fractions

    threads = len(os.sched_getaffinity(0)) or 1
    torch.set_num_threads(threads)
    B = len(lps)
    Bp = B // 2
    g = torch.Generator().manual_seed(99)
    kv = [([torch.randn(lp + bl, 16, 64, generator=g).bfloat16() for lp in lps],
           [torch.randn(lp + bl, 16, 64, generator=g).bfloat16() for lp in lps]) for _ in range(n_layers)]
    block = torch.randn(B, bl, 1024, generator=g).bfloat16()
    ctx = torch.randn(B, 1, 1024, generator=g).bfloat16()
    sched = torch.tensor(omnivoice_unmask_schedule(bl, 10, 0.5))
    q = torch.tensor(quantile_fractions(3.0, 10), dtype=torch.float32)
    w_head = model.speech_head.weight.detach().cpu()

    def median_time(fn):
        fn()  # warm-up
        ts = []
        for _ in range(runs):
            t = time.time()
            fn()
            ts.append(time.time() - t)
        return sorted(ts)[len(ts) // 2]

    per = {}
    for name, dt in (("bf16", torch.bfloat16), ("fp32", torch.float32)):
        bb = OL.backbone_from_model(model, max_pos=max(lps) + 2 * bl, dtype=dt)
        cache = OL.KVCache(k=[[t.to(dt) for t in k] for k, _ in kv], v=[[t.to(dt) for t in v] for _, v in kv])
        blk, cx, wh = block.to(dt), ctx.to(dt), w_head.to(dt)
        hid = OL.block_forward(bb, blk, cache, lps, n_layers=n_layers)
        t_layers = median_time(lambda: OL.block_forward(bb, blk, cache, lps, n_layers=n_layers))
        logits = OL.speech_head_shift(hid, cx, wh)
        t_head = median_time(lambda: OL.speech_head_shift(hid, cx, wh))
        lf = logits.float()
        t_score = median_time(lambda: OS.score_step(
            lf[:Bp], lf[Bp:], sc_in.xt.cpu(), sc_in.k_step.cpu(), sc_in.log_prior.cpu(), sched, q, K=10, cfg=0.5,
            tau=3.0, mask_id=8194, stop_id=6562))
        t_step = t_layers * L / n_layers + t_head + t_score
        per[name] = dict(t_layers=t_layers, t_head=t_head, t_score=t_score, t_step=t_step)
        log(f"cpu baseline {name}: {n_layers} layers {t_layers:.2f}s, head {t_head:.2f}s, score {t_score:.2f}s "
            f"(medians of {runs}) -> {t_step:.1f}s per step on {threads} threads")
    info = host_cpu_info()
    bf, fp = per["bf16"], per["fp32"]
    return {"value": round(Bp * bl / bf["t_step"], 2), "unit": "speech tokens/s", "cores": threads, "kind": "port",
            "sample": f"oracle torch-CPU block forward of {n_layers} of {L} layers at the full {B}-row batch "
                      f"(time x {L}/{n_layers}) + speech head + fp32 scoring, bf16; median of {runs} runs each "
                      f"after a warm-up; {bf['t_step']:.1f} s per step",
            "value_fp32": round(Bp * bl / fp["t_step"], 2),
            "layers_timed": n_layers, "layers_total": L, "rows": B, "layer_scale": L / n_layers, "runs": runs,
            "stat": "median", "seconds_per_step": {k: round(v["t_step"], 3) for k, v in per.items()},
            "seconds_layers_sample": {k: round(v["t_layers"], 3) for k, v in per.items()}, **info}


if __name__ == "__main__":
    main()
