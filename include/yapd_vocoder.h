/* C ABI of the HiFT vocoder's fused elementwise family on gfx950.
 *
 * Drop-in for the HIP extension the reference builds at run time
 * (server/kernels.py:11-101, loaded by load_snake_extension() at
 * server/kernels.py:103-106 and installed into S3Gen's HiFT generator by
 * install_fused_snake() at server/kernels.py:154-165).  Every tensor is a
 * contiguous fp32 [B, C, T] array in device memory ("BCT"); per-channel
 * vectors (alpha, bias) have C entries.  Outputs are caller-allocated and may
 * not alias inputs.  Kernels run on `stream` (a hipStream_t; NULL = default
 * stream); nothing is allocated and the host never waits.  Return values and
 * yapd_last_error() are those of yapd_t3.h.
 *
 * Snake (HiFT / BigVGAN activation): snake(v, a) = v + (1 / (a + 1e-9)) *
 * sin(v * a)^2, with sin to within 2 ulp of the exact value. */
#ifndef YAPD_VOCODER_H_
#define YAPD_VOCODER_H_

#include <stdint.h>

#include "yapd_t3.h"

#ifdef __cplusplus
extern "C" {
#endif

/* out = snake(x + bias[c], alpha[c]); bias may be NULL (plain snake).
 * Replaces snake_hip / snake_bias_hip (server/kernels.py:35-47, 77-84). */
int yapd_snake(const float* x, const float* alpha, const float* bias, float* out, int64_t B, int C, int64_t T,
               void* stream);

/* out = (x + residual) + bias[c].
 * Replaces residual_bias_hip (server/kernels.py:48-51, 85-88). */
int yapd_residual_bias(const float* x, const float* residual, const float* bias, float* out, int64_t B, int C,
                       int64_t T, void* stream);

/* out = ((a + b) + c) * (float)(1/3) over n elements (any shape).
 * Replaces mean3_hip (server/kernels.py:52-55, 89-92). */
int yapd_mean3(const float* a, const float* b, const float* c, float* out, int64_t n, void* stream);

/* raw = (x + residual) + bias[c]; act = snake(raw, alpha[c]).
 * Replaces residual_bias_snake_hip (server/kernels.py:56-61, 93-96). */
int yapd_residual_bias_snake(const float* x, const float* residual, const float* bias, const float* alpha,
                             float* raw_out, float* act_out, int64_t B, int C, int64_t T, void* stream);

/* raw = x + source; out_j = snake(raw, alpha_j[c]) for j = 0, 1, 2.
 * Replaces branch_start_hip (server/kernels.py:62-67, 97-100). */
int yapd_branch_start(const float* x, const float* source, const float* alpha0, const float* alpha1,
                      const float* alpha2, float* raw_out, float* out0, float* out1, float* out2, int64_t B, int C,
                      int64_t T, void* stream);

/* Chunk stitching of the streaming vocoder for a whole micro-batch: replaces
 * the per-job numpy post-processing of Vocoder._postprocess
 * (server/vocoder.py:284-320) after the batch's HiFT pass (:271-279).
 *
 * wav: fp32 [rows][wav_stride] device array (the batch's waveforms, wav_cols
 * valid samples per row).  jobs: device int32 [n_jobs][YAPD_STITCH_JOB_INTS],
 * per job
 *   0 row      batch row of the job
 *   1 lo       first sample of the row the job uses
 *   2 n_seg    samples used from lo on
 *   3 n_blend  leading samples blended as tail * fade_out + x * fade_in with
 *              tails_in[tail_in] (0: none)
 *   4 trim     1: multiply the first min(n_trim, n_seg) samples by trim
 *   5 pre_roll zeros placed before the samples
 *   6 n_out    samples of the result written to pcm (pre_roll + n_seg, or
 *              that minus fade when the job withholds a tail)
 *   7 tail_in  row of tails_in for the blend (-1: none)
 *   8 tail_out row of tails_out that receives the last fade samples of the
 *              result, before clipping (-1: none)
 *   9 pcm_off  first pcm sample of the job
 *   10, 11     unused (0)
 * pcm = trunc(clip(result, -1, 1) * 32767), every product and sum rounded
 * separately as numpy does in float32.  A job that does not fit the buffers
 * it names is skipped.  fade_in / fade_out: fade floats each; trim: n_trim
 * floats. */
#define YAPD_STITCH_JOB_INTS 12
int yapd_voc_stitch(const float* wav, int64_t wav_stride, int64_t wav_cols, int rows, const int32_t* jobs,
                    int n_jobs, const float* fade_in, const float* fade_out, int fade, const float* trim, int n_trim,
                    const float* tails_in, int n_tails_in, float* tails_out, int n_tails_out, int16_t* pcm,
                    int64_t pcm_len, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* YAPD_VOCODER_H_ */
