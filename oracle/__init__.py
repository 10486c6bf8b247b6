"""CPU oracle for the T3 block-diffusion decode step.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (``yapd_amd``) imports,
links or runs anything under ``oracle/``.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
use it, and only as the reference that GPU results are compared against (or
as the timed CPU baseline), never as the thing measured or shipped.

Modules (each function cites the reference file:line it restates):

* :mod:`oracle.schedule` -- OmniVoice unmask-count schedule and the
  time-shifted quantile table (chatterbox_flash/model.py:133-177,
  server/engine.py:357-358).
* :mod:`oracle.scoring` -- CFG combine, prior-calibrated PMI, quantile
  threshold and top-n unmask rule in the fp32 op order of
  server/engine.py:532-593, plus the per-row model.py:185-311 variant.
* :mod:`oracle.pages` -- paged-KV index math (engines/flashinfer.py:318-411)
  generalised to an arbitrary page table, and the pool gather.
* :mod:`oracle.llama` -- the Llama backbone block forward with torch-SDPA
  semantics (engines/torch_sdpa.py:274-341, server/engine.py:133-176) with
  per-row cache starts, and the token-shifted speech head
  (engines/flashinfer.py:1452-1461).
* :mod:`oracle.quant` -- MLX affine group quantisation (engines/mlx.py:221-255
  calls ``mlx.nn.quantize``; the documented MLX formula is restated).
* :mod:`oracle.serve` -- the continuous-batching tick bookkeeping of
  server/engine.py:522-620 (commit / denoise transitions, clamps, flags).
* :mod:`oracle.vocoder` -- the HiFT vocoder's Snake / bias / residual /
  mean3 elementwise family of server/kernels.py:35-67.
"""
