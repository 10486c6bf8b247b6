// Whole-block forward of the T3 backbone: the layer loop of
// engines/flashinfer.py:_block_forward_fused (:970-1065) / _graph_body
// (:1312-1461) driven from native code, one FFI call per step.  Every launch
// goes to the caller's stream, so the whole call can be captured in a HIP
// graph.
//
// Per layer:  qkv+rope+kv-write GEMM -> paged attention -> o_proj GEMM
//             adding into the residual -> post-attention RMSNorm ->
//             gate/up+SiLU GEMM -> down GEMM adding into the residual ->
//             next input RMSNorm (final norm after the last layer).
#include "common.h"

#define YAPD_TRY(expr)            \
  do {                            \
    const int _rc = (expr);       \
    if (_rc != YAPD_OK) return _rc; \
  } while (0)

extern "C" int yapd_t3_block_forward(const yapd_t3_model* m, const yapd_t3_workspace* ws, const void* block_emb,
                                     int rows, int bl, const int32_t* pos0, const int32_t* kv_len, int causal,
                                     void* hidden_out, const void* head_w, int vocab, const void* shift_ctx,
                                     void* logits, int64_t ld_logits, void* stream) {
  YAPD_REQUIRE(m && ws && block_emb && pos0 && kv_len && hidden_out, "t3_block_forward: NULL pointer");
  YAPD_REQUIRE(m->n_layers >= 1 && m->layers, "t3_block_forward: no layers");
  YAPD_REQUIRE(rows >= 1 && bl >= 1 && bl <= 64, "t3_block_forward: need rows >= 1, 1 <= bl <= 64");
  YAPD_REQUIRE(ws->residual && ws->q && ws->attn && ws->normed && ws->delta && ws->act && ws->work,
               "t3_block_forward: incomplete workspace");
  const int D = m->hidden, H = m->n_heads, F = m->ffn, HD = H * 64;
  const int M = rows * bl;
  // The shape rules of every per-layer call, checked before the first launch,
  // so that a rejected call leaves the residual, the KV pools and the outputs
  // untouched (the calls below check them again).
  YAPD_REQUIRE(D % 512 == 0 && D >= 512 && D <= 2048, "t3_block_forward: hidden must be 512, 1024, 1536 or 2048 (got %d)",
               D);
  // attention covers 4 heads per workgroup
  YAPD_REQUIRE(H % 4 == 0 && H >= 4, "t3_block_forward: n_heads must be a multiple of 4 (got %d)", H);
  YAPD_REQUIRE(F % 64 == 0 && F >= 64, "t3_block_forward: ffn must be a multiple of 64 (got %d)", F);
  YAPD_REQUIRE(m->rope_cos && m->rope_sin && m->rope_positions >= 1 && m->final_norm,
               "t3_block_forward: missing RoPE tables or final norm");
  YAPD_REQUIRE(m->page_table && m->n_pages >= 1 && m->table_cols >= 1 && m->table_stride >= m->table_cols,
               "t3_block_forward: bad page table");
  for (int li = 0; li < m->n_layers; ++li) {
    const yapd_t3_layer& L = m->layers[li];
    YAPD_REQUIRE(L.w_qkv && L.w_o && L.w_gate_up && L.w_down && L.ln_in && L.ln_post && L.kv_pool,
                 "t3_block_forward: layer %d has a NULL weight or KV pool", li);
  }
  YAPD_REQUIRE(ws->n_work >= 1 && (ws->n_merge == 0 || (ws->merge && ws->part_o && ws->part_ml && ws->n_slots >= 1)),
               "t3_block_forward: bad attention plan in the workspace");
  YAPD_REQUIRE(!head_w || (shift_ctx && logits && vocab >= 1 && ld_logits >= vocab),
               "t3_block_forward: head needs shift_ctx, logits, vocab >= 1 and ld_logits >= vocab");
  const float scale = 0.125f;  // head_dim ** -0.5 for head_dim 64
  void* st = stream;
  auto* res = ws->residual;
  auto* xn = ws->normed;

  YAPD_TRY(yapd_rmsnorm(nullptr, res, block_emb, m->layers[0].ln_in, m->layers[0].eps_in, M, D, xn, st));
  for (int li = 0; li < m->n_layers; ++li) {
    const yapd_t3_layer& L = m->layers[li];
    YAPD_TRY(yapd_gemm_qkv_rope_kv(xn, D, L.w_qkv, M, D, H, m->rope_cos, m->rope_sin, m->rope_positions, pos0, bl,
                                   ws->q, L.kv_pool, m->n_pages, m->page_table, m->table_stride, m->table_cols, st));
    YAPD_TRY(yapd_attn_paged_block(ws->q, L.kv_pool, m->n_pages, m->page_table, m->table_stride, m->table_cols,
                                   kv_len, rows, bl, H, ws->work, ws->n_work, ws->merge, ws->n_merge, ws->counts,
                                   ws->part_o, ws->part_ml, ws->n_slots, scale, causal, ws->attn, st));
    YAPD_TRY(yapd_gemm_bf16_residual(ws->attn, HD, L.w_o, HD, M, D, HD, res, D, st));
    YAPD_TRY(yapd_rmsnorm(nullptr, nullptr, res, L.ln_post, L.eps_post, M, D, xn, st));
    YAPD_TRY(yapd_gemm_swiglu(xn, D, L.w_gate_up, M, F, D, ws->act, F, st));
    YAPD_TRY(yapd_gemm_bf16_residual(ws->act, F, L.w_down, F, M, D, F, res, D, st));
    const bool last = li + 1 == m->n_layers;
    const void* wn = last ? m->final_norm : m->layers[li + 1].ln_in;
    const float eps = last ? m->final_eps : m->layers[li + 1].eps_in;
    YAPD_TRY(yapd_rmsnorm(nullptr, nullptr, res, wn, eps, M, D, last ? hidden_out : xn, st));
  }
  if (head_w != nullptr) {
    YAPD_TRY(yapd_gemm_head_shift(hidden_out, shift_ctx, rows, bl, D, head_w, D, vocab, logits, ld_logits, st));
  }
  return YAPD_OK;
}
