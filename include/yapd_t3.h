/*
 * yapd_t3.h -- C ABI of the MI355X (gfx950) T3 block-diffusion decode step.
 *
 * Every entry point takes raw device pointers, sizes/strides, scalars and a
 * hipStream_t passed as `void*` (NULL = the null stream).  Work is enqueued
 * on that stream and never synchronised; nothing here allocates device
 * memory or keeps hidden global state, so calls are re-entrant from one
 * host thread per stream.  Scratch memory is caller-owned ("workspace"),
 * except in yapd_attn_paged_block_noalloc, whose split-KV partials live in a
 * static device array per GPU (see there).
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

/* ABI revision of this library (bumped on any signature or struct layout
 * change; 3 added the quantised-weight fields of yapd_t3_layer, 4 the wdq
 * buffer of yapd_t3_workspace). */
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
 * (int64); per pair: n_mask_after (int32), hit_eos (u8).  1 <= bl <= 64, 1 <= K <= 64.
 * One launch: a workgroup per pair, one wave per position, then the pair's
 * pmi and decision by one wave (lane = position) from LDS.
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


/* ------------------------------------------------------------------------ *
 * Paged KV pool (one per layer): bf16 [n_pages][2][H][16*64]; plane 0 holds
 * K (token-major inside a head), plane 1 holds V transposed inside a head.
 * Position p of row r lives on page page_table[r*table_stride + p/16], slot
 * p % 16.  Replaces the NHD pool + static page slices of
 * engines/flashinfer.py:104-116 and the index math of :318-344; any
 * permutation of pool pages is a valid table.  Table reads are clamped to
 * table_cols entries and page ids to n_pages, so a bad table cannot fault.
 * ------------------------------------------------------------------------ */

/* Scatter k, v ([rows*bl, H, 64] with token strides k_tok_stride,
 * v_tok_stride) at positions pos0[r] .. pos0[r]+bl-1 (device int32).
 * Replaces paged_kv[li][pw_idx, 0|1, pw_off] = k|v (engines/flashinfer.py:1034-1035). */
int yapd_kv_write(const void* k, const void* v, int64_t k_tok_stride, int64_t v_tok_stride, void* kv_pool,
                  int64_t n_pages, const int32_t* page_table, int table_stride, int table_cols,
                  const int32_t* pos0, int rows, int bl, int n_heads, void* stream);

/* Debug/test gather of one row's K and V, dense [kv_len, H, 64] each. */
int yapd_kv_gather(const void* kv_pool, int64_t n_pages, const int32_t* table_row, int table_len, int kv_len,
                   int n_heads, void* k_out, void* v_out, void* stream);

/* Host-side planner (CPU only, no GPU call): cuts each row's kv_len keys
 * into work items of whole 32-key chunks so that ~target_items items exist,
 * none shorter than min_split_keys (>= 32) unless the whole row is, longest
 * first.  work [n_work][4] = (row, key_begin, key_end, slot; slot -1
 * means the item writes the final output), merge [n_merge][3] = (row,
 * first_slot, n_slots).  Replaces the per-block plan() of
 * engines/flashinfer.py:346-411. */
int yapd_attn_plan(const int32_t* kv_len, int rows, int target_items, int min_split_keys, int32_t* work,
                   int work_cap, int32_t* merge, int merge_cap, int* n_work, int* n_merge, int* n_slots);

/* (a) Block attention over paged KV: out[r, i] = softmax(q[r, i] K_r^T *
 * scale) V_r over keys [0, kv_len[r]) -- bidirectional over the whole block
 * (causal = 0, the block step: engines/flashinfer.py:884-886, 1037-1039;
 * torch_sdpa.py:299-307), or causal inside the block (causal = 1, prefix
 * prefill).  q, out: bf16 [rows, bl, H, 64]; kv_len on the device.
 * n_work / n_merge size the grids; counts (device {n_work, n_merge}, may be
 * NULL) lets a captured graph replay with fewer items.  part_o [n_slots, bl,
 * H, 64] and part_ml [n_slots, bl, H, 2] fp32 are the split-KV workspace. */
int yapd_attn_paged_block(const void* q, const void* kv_pool, int64_t n_pages, const int32_t* page_table,
                          int table_stride, int table_cols, const int32_t* kv_len, int rows, int bl, int n_heads,
                          const int32_t* work, int n_work, const int32_t* merge, int n_merge,
                          const int32_t* counts, float* part_o, float* part_ml, int n_slots, float scale,
                          int causal, void* out, void* stream);

/* Variant of yapd_attn_paged_block that allocates nothing and takes no
 * workspace: the split-KV partials live in a file-scope device array of
 * 16 MiB per GPU (n_slots * bl * n_heads * 66 floats must fit, else
 * YAPD_EINVAL before any launch).  It has no counterpart in the reference;
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops).  Every call on one GPU shares that GPU's
 * array, so calls that overlap on one GPU race (use one stream per GPU or
 * order the streams).  The first call on a GPU that splits a row looks up
 * the array's device address (hipGetSymbolAddress, not a stream operation);
 * if `stream` is being captured then, the lookup runs in relaxed capture mode
 * for the calling thread.  Results equal yapd_attn_paged_block's bit for bit. */
int yapd_attn_paged_block_noalloc(const void* q, const void* kv_pool, int64_t n_pages, const int32_t* page_table,
                                  int table_stride, int table_cols, const int32_t* kv_len, int rows, int bl,
                                  int n_heads, const int32_t* work, int n_work, const int32_t* merge, int n_merge,
                                  const int32_t* counts, int n_slots, float scale, int causal, void* out,
                                  void* stream);

/* ------------------------------------------------------------------------ *
 * (b) bf16 MFMA projections (nn.Linear layout: C = A W^T, fp32 accumulate).
 * K must be a multiple of 64; A, W 16-byte aligned with leading dims
 * multiples of 8.
 * ------------------------------------------------------------------------ */

/* Plain projection: o_proj / down_proj (F.linear at engines/flashinfer.py:1041, 455). */
int yapd_gemm_bf16(const void* A, int64_t lda, const void* W, int64_t ldw, int M, int N, int K, void* C,
                   int64_t ldc, void* stream);

/* Projection into the residual stream: residual = bf16(residual + bf16(A*W^T))
 * (o_proj / down_proj + the residual add of fused_add_rmsnorm,
 * engines/flashinfer.py:1040-1060; the norm itself is yapd_rmsnorm). */
int yapd_gemm_bf16_residual(const void* A, int64_t lda, const void* W, int64_t ldw, int M, int N, int K,
                            void* residual, int64_t ld_res, void* stream);

/* Fused QKV + NeoX RoPE + paged KV write (engines/flashinfer.py:998-1035):
 * rows r*bl+j at position pos0[r]+j; cos/sin fp32 [max_pos, 64] hold the
 * model-dtype table (flashinfer.py:246-255) in HF's cat(freqs, freqs)
 * layout: column d + 32 must equal column d, and only columns 0..31 are
 * read.  q goes to q_out [M, H*64], k and v straight into the pool
 * (n_pages < 2^31). */
int yapd_gemm_qkv_rope_kv(const void* A, int64_t lda, const void* W_qkv, int M, int K, int n_heads,
                          const float* cos_t, const float* sin_t, int max_pos, const int32_t* pos0, int bl,
                          void* q_out, void* kv_pool, int64_t n_pages, const int32_t* page_table, int table_stride,
                          int table_cols, void* stream);

/* Input RMSNorm + QKV + NeoX RoPE + paged KV write on the residual stream
 * (engines/flashinfer.py:992-1035: input_layernorm, then the projections, RoPE
 * and the pool write): x [M, K] contiguous bf16 rows are normalised into the
 * caller's workspace normed [M, K] (HF LlamaRMSNorm, as yapd_rmsnorm with x),
 * then yapd_gemm_qkv_rope_kv runs on normed.  A composition, not a fused
 * kernel: two launches on `stream` (the norm is a separate row pass, as in the
 * step driver), every argument of both checked before the first (a rejected
 * call launches nothing). */
int yapd_gemm_rmsnorm_qkv_rope_kv(const void* x, const void* ln_w, float eps, void* normed, const void* W_qkv,
                                  int M, int K, int n_heads, const float* cos_t, const float* sin_t, int max_pos,
                                  const int32_t* pos0, int bl, void* q_out, void* kv_pool, int64_t n_pages,
                                  const int32_t* page_table, int table_stride, int table_cols, void* stream);

/* Fused gate/up + SiLU*up (engines/flashinfer.py:433-455): W rows are
 * [gate f..f+31; up f..f+31] for f = 0, 32, ...; act [M, F]. */
int yapd_gemm_swiglu(const void* A, int64_t lda, const void* W_gu_interleaved, int M, int F, int K, void* act,
                     int64_t ld_act, void* stream);

/* Token-shifted speech head (engines/flashinfer.py:1452-1461): logits row
 * (r, j) = W hidden[r, j-1], and (r, 0) = W shift_ctx[r]. */
int yapd_gemm_head_shift(const void* hidden, const void* shift_ctx, int rows, int bl, int K, const void* W,
                         int64_t ldw, int N, void* logits, int64_t ldc, void* stream);

/* HF LlamaRMSNorm rows (D multiple of 512, <= 2048): out = w * bf16(x *
 * rsqrt(mean(x^2) + eps)).  With delta: residual = bf16(residual + delta)
 * in place first (flashinfer fused_add_rmsnorm, engines/flashinfer.py:1043-1060);
 * with x and residual: residual = x (the clone of engines/flashinfer.py:992). */
int yapd_rmsnorm(const void* delta, void* residual, const void* x, const void* w, float eps, int M, int D,
                 void* out, void* stream);

/* (d) Affine group-quantised projection, MLX layout (engines/mlx.py:221-255
 * quantises with mlx.nn.quantize): w_packed uint32 [N, K*bits/32] holds
 * LSB-first codes, scales and biases fp16 [N, K/64]; W_hat = scale*q + bias
 * per group of 64 input features, dequantised into the MFMA B tile.
 * C[M, N] = A[M, K] W_hat^T in bf16 with fp32 accumulation; bits 4 or 8,
 * group_size 64. */
int yapd_qgemm_affine(const void* A, int64_t lda, const uint32_t* w_packed, const void* scales,
                      const void* biases, int bits, int group_size, int M, int N, int K, void* C, int64_t ldc,
                      void* stream);

/* (d) The weights yapd_qgemm_affine multiplies by: W_out[N, K] (bf16, row
 * pitch K, 16-byte aligned) = bf16(scale*q + bias), the dequantisation of
 * mlx.core.dequantize on the layout of engines/mlx.py:221-255 (the same
 * arithmetic as yapd_qgemm_affine's W loader, so yapd_gemm_bf16 on W_out
 * equals yapd_qgemm_affine bit for bit).  For many rows the dequantise-once
 * route is the faster one: the fused kernel dequantises each W tile again for
 * every tile row.  bits 4 or 8, group_size 64, K a multiple of 64. */
int yapd_dequant_affine(const uint32_t* w_packed, const void* scales, const void* biases, int bits,
                        int group_size, int N, int K, void* W_out, void* stream);

/* ------------------------------------------------------------------------ *
 * Whole block forward: one call runs the n_layers decoder layers and the
 * final norm (engines/flashinfer.py:_block_forward_fused :970-1065 /
 * _graph_body :1312-1461), optionally followed by the token-shifted head.
 * ------------------------------------------------------------------------ */
/* One affine-quantised projection weight in the MLX layout (as
 * yapd_qgemm_affine): packed uint32 [N, K*bits/32], LSB-first codes; scales
 * and biases fp16 [N, K/64]. */
typedef struct yapd_t3_qweight {
  const uint32_t* packed;
  const void* scales;
  const void* biases;
} yapd_t3_qweight;

typedef struct yapd_t3_layer {
  const void* w_qkv;     /* bf16 [3*H*64, D]: q, k, v rows */
  const void* w_o;       /* bf16 [D, H*64] */
  const void* w_gate_up; /* bf16 [2F, D], gate/up interleaved per 32 rows */
  const void* w_down;    /* bf16 [D, F] */
  const void* ln_in;     /* bf16 [D] */
  const void* ln_post;   /* bf16 [D] */
  float eps_in, eps_post;
  void* kv_pool;         /* this layer's pool */
  /* Weight-only quantisation of the layer's projections, as the reference's
   * Metal engine applies to its whole LLaMA stack when
   * CHATTERBOX_FLASH_MLX_QUANT_BITS is set (engines/mlx.py:221-255):
   * qbits = 4 or 8 runs the four projections on q_* (same row orders as the
   * bf16 weights; w_qkv .. w_down are then unused and may be NULL); qbits = 0
   * runs the bf16 weights.  The fused epilogues are the same, and the result
   * equals the bf16 path's on the dequantised weights bf16(scale*q + bias)
   * bit for bit. */
  int qbits;
  yapd_t3_qweight q_qkv, q_o, q_gate_up, q_down;
} yapd_t3_layer;

typedef struct yapd_t3_model {
  int n_layers, hidden, n_heads, ffn;
  const yapd_t3_layer* layers; /* host array [n_layers] */
  const void* final_norm;      /* bf16 [D] */
  float final_eps;
  const float* rope_cos;       /* fp32 [rope_positions, 64] */
  const float* rope_sin;
  int rope_positions;
  int64_t n_pages;
  const int32_t* page_table;
  int table_stride, table_cols;
} yapd_t3_model;

typedef struct yapd_t3_workspace {
  void* residual; /* bf16 [rows*bl, D] */
  void* q;        /* bf16 [rows*bl, H*64] */
  void* attn;     /* bf16 [rows*bl, H*64] */
  void* normed;   /* bf16 [rows*bl, D] */
  void* delta;    /* bf16 [rows*bl, D] */
  void* act;      /* bf16 [rows*bl, F] */
  const int32_t* work;   /* attention plan (yapd_attn_plan), device */
  int n_work;
  const int32_t* merge;
  int n_merge;
  const int32_t* counts; /* device {n_work, n_merge} or NULL */
  float* part_o;
  float* part_ml;
  int n_slots;
  /* Optional (NULL: unused), for quantised layers: bf16 scratch of wdq_elems
   * >= 3*H*64*D + D*H*64 + 2*F*D + D*F elements, 16-byte aligned.  With it,
   * a quantised layer over at least 4096 rows dequantises its four weights
   * into it (one yapd_dequant_affine pass) and runs the bf16 kernels, whose
   * results equal the fused quantised kernels' bit for bit; fewer rows, or
   * no buffer, run the fused kernels on the codes. */
  void* wdq;
  int64_t wdq_elems;
} yapd_t3_workspace;

/* block_emb [rows*bl, D] is not modified; pos0 [rows] (device) is each row's
 * first position, kv_len [rows] (device) = pos0 + bl.  hidden_out [rows*bl,
 * D] receives the final-normed hidden.  If head_w != NULL the logits [rows,
 * bl, vocab] (row pitch ld_logits) are computed from hidden and shift_ctx
 * [rows, D].  The shape rules of every per-layer call (D a multiple of 512
 * up to 2048, H a multiple of 4, F a multiple of 64, complete layers, tables,
 * attention plan and head arguments) are checked before the first launch: on
 * YAPD_EINVAL nothing has been launched. */
int yapd_t3_block_forward(const yapd_t3_model* model, const yapd_t3_workspace* ws, const void* block_emb,
                          int rows, int bl, const int32_t* pos0, const int32_t* kv_len, int causal,
                          void* hidden_out, const void* head_w, int vocab, const void* shift_ctx, void* logits,
                          int64_t ld_logits, void* stream);

/* One causal step of a prefix prefill (engines/flashinfer.py:prefix_forward
 * :678-854, the chunked causal forward that writes each row's prefix KV)
 * over packed rows: no row is padded to a chunk length.  A "row" here is a
 * segment of consecutive tokens of one sequence (its own page-table row);
 * several consecutive segments of one sequence may share a step, since all
 * keys of the step are written before any is attended.  Row r's tokens
 * are rows [row_start[r], row_start[r+1]) of tok_emb [n_tokens, D] (at most
 * max_q <= 64 per row), at positions pos0[r], pos0[r] + 1, ...; tok_row
 * [n_tokens] names each token's row; kv_len[r] = pos0[r] + the row's token
 * count (row_start, tok_row, pos0, kv_len: device int32).  The workspace's
 * activations hold n_tokens rows, its attention plan is yapd_attn_plan over
 * kv_len with bl = max_q, and its partials are [n_slots, max_q, H, ...].
 * hidden_out [n_tokens, D] receives the final-normed hidden.  The row map's
 * indices are clamped on the device (a bad map cannot fault); the layer and
 * workspace rules of yapd_t3_block_forward are checked before any launch. */
int yapd_t3_prefill_packed(const yapd_t3_model* model, const yapd_t3_workspace* ws, const void* tok_emb,
                           int n_tokens, int rows, int max_q, const int32_t* row_start, const int32_t* tok_row,
                           const int32_t* pos0, const int32_t* kv_len, void* hidden_out, void* stream);

/* ------------------------------------------------------------------------ *
 * Continuous-batching tick bookkeeping (server/engine.py:522-612, the state
 * updates of FlashEngine._step_gpu after the scorer).  For slots s <
 * n_slots, with commit = is_commit[s] on entry:
 *   xt_final[s][j] = commit ? xt_blk[s][j] : xt_new[s][j], scattered into
 *   xt[s][blk_start[s] + j];  n_mask_after / hit_eos over xt_final;
 *   k_step    = commit ? 0 : k_step + 1;
 *   cache_len = commit ? min(cache_len + bl, max_len - bl) : cache_len;
 *   blk_start = commit ? min(blk_start + bl, n_max - bl) : blk_start;
 *   is_commit = !commit && !hit_eos && (n_mask_after == 0 || k_step >= K);
 *   flags[s] = {commit, n_mask_after, hit_eos, k_step, blk_start, n_speech};
 *   the n_branch shift_ctx rows of a committing slot take the block's last
 *   hidden row (server/engine.py:522-527).
 * hidden [n_slots * n_branch * bl, D] and shift_ctx [n_slots * n_branch, D]
 * are bf16; every other array is int64 except is_commit (uint8). */
int yapd_tick_update(int n_slots, int bl, int n_branch, int D, int K, int64_t mask_id, int64_t stop_id,
                     int64_t max_len, int64_t n_max, int64_t* xt, int64_t xt_stride, const int64_t* xt_blk,
                     const int64_t* xt_new, int64_t* k_step, int64_t* cache_len, int64_t* blk_start,
                     uint8_t* is_commit, const int64_t* n_speech, const void* hidden, void* shift_ctx,
                     int64_t* flags, int64_t* xt_final, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* YAPD_T3_H */
