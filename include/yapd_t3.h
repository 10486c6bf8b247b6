/*
 * yapd_t3.h -- C ABI of the MI355X (gfx950) T3 block-diffusion decode step.
 *
 * Every entry point takes raw device pointers, sizes/strides, scalars and a
 * hipStream_t passed as `void*` (NULL = the null stream).  Work is enqueued
 * on that stream and never synchronised; nothing here allocates device
 * memory or keeps hidden global state, so calls are re-entrant from one
 * host thread per stream.  Scratch memory is caller-owned ("workspace").
 *
 * Return value: YAPD_OK (0) or a nonzero YAPD_E* code; yapd_last_error()
 * then describes the failure (thread-local, valid until the next call).
 * Failed preconditions are errors -- there is no fallback path.
 *
 * bf16 tensors are raw 16-bit bfloat16 (the upper half of an IEEE fp32).
 */
#ifndef YAPD_T3_H
#define YAPD_T3_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define YAPD_OK 0
#define YAPD_EINVAL 1 /* bad argument (shape, stride, alignment, null pointer) */
#define YAPD_EHIP 2   /* the HIP runtime reported an error */

/* Message for the last nonzero return on this thread ("" if none). */
const char* yapd_last_error(void);

/* ABI revision of this library (bumped on any signature change). */
int yapd_abi_version(void);

/* ------------------------------------------------------------------------ *
 * (c) CFG + prior-calibrated PMI + time-shifted-quantile unmask scoring.
 *
 * Replaces the vectorised scorer of server/engine.py:532-593 (and the
 * per-row loop of chatterbox_flash/model.py:856-900 calling
 * _pmi_count_early_step_unmask, model.py:185-311, with compute_pmi at
 * chatterbox_flash/calibration.py:63-82 and the CFG combine at
 * chatterbox_flash/cfg_guidance.py:22-57).
 *
 * logits: bf16, element (row, pos, v) at row*seq_stride + pos*pos_stride + v
 *   (both strides even, base 4-byte aligned).  Pair p uses cond row
 *   cond_row0 + p*pair_row_step and, when has_uncond, null row
 *   cond + null_row_offset: generate() stacks [cond x B | null x B]
 *   (step 1, offset B, model.py:859-860); the server interleaves
 *   (cond_i, null_i) (step 2, offset 1, server/engine.py:534).
 * log_prior [vocab] fp32 = log(clamp(prior, 1e-8)) (server/engine.py:365-366).
 * xt_in [n_pairs, bl] int64 block tokens; k_step [n_pairs] int64 step index;
 * active [n_pairs] (NULL = all): inactive pairs keep their tokens.
 * sched [K] int32 OmniVoice counts, q_tab [K] fp32 quantile fractions.
 * temperature == 0: argmax of the guided distribution (bit-exact decisions);
 * > 0: Gumbel-max with Philox4x32-10 noise keyed by (seed, rng_offset).
 * pos_gumbel != 0 adds standard Gumbel noise to masked PMI
 * (server/engine.py:559-561; the reference adds it unscaled).
 * Outputs [n_pairs, bl]: sampled (int64), pmi (fp32), unmask (u8), xt_out
 * (int64); per pair: n_mask_after (int32), hit_eos (u8).  1 <= bl <= 64.
 * Two launches: a streaming pass per (pair, position), then one wave per pair.
 * ------------------------------------------------------------------------ */

int yapd_score_cfg_pmi_unmask(
    const void* logits, int64_t seq_stride, int64_t pos_stride,
    int n_pairs, int bl, int vocab,
    int cond_row0, int pair_row_step, int has_uncond, int null_row_offset,
    const float* log_prior, const int64_t* xt_in, const int64_t* k_step,
    const uint8_t* active, const int32_t* sched, const float* q_tab, int K,
    float cfg_w, int quantile_on, int64_t mask_id, int64_t stop_id,
    float temperature, int pos_gumbel, uint64_t seed, uint64_t rng_offset,
    int64_t* sampled_out, float* pmi_out, uint8_t* unmask_out, int64_t* xt_out,
    int32_t* n_mask_after_out, uint8_t* hit_eos_out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* YAPD_T3_H */
