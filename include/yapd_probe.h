/* Calibration kernels for the measurement harness (not part of the engine
 * boundary; they have no counterpart in the reference).
 *
 * yapd_mfma_peak_probe: `blocks` workgroups of 4 waves each run `iters`
 * rounds of 8 independent v_mfma_f32_32x32x16_bf16 on register operands and
 * store one float per thread to out[blocks * 256].  random_operands != 0: each
 * accumulator's operand pair holds random bf16 spread like activations (unit
 * scale) and weights (scale 0.02); 0: the same few-bit constants for all.
 * Work per call: blocks * 4 * iters * 8 * 32768 flops; the sustained bf16
 * MFMA rate is that divided by the launch time.
 *
 * yapd_hbm_read_probe: reads `bytes` (a multiple of 16) from the 16-byte
 * aligned `src` once with `blocks` workgroups of 256 threads: workgroup b
 * takes the contiguous 16-byte words [b P, (b + 1) P), P = ceil(bytes / 16 /
 * blocks) rounded up to a multiple of 256, and its thread t folds words
 * b P + t, b P + t + 256, ... by XOR into out[b * 256 + t] (out[blocks *
 * 256]).  The streaming read rate is bytes divided by the launch time. */
#ifndef YAPD_PROBE_H
#define YAPD_PROBE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

int yapd_mfma_peak_probe(int blocks, int iters, int random_operands, float* out, void* stream);
int yapd_hbm_read_probe(const void* src, int64_t bytes, int blocks, uint32_t* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif
