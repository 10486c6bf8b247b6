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
#include "attention.h"
#include "common.h"
#include "packed.h"
#include "quant.h"

#define YAPD_TRY(expr)            \
  do {                            \
    const int _rc = (expr);       \
    if (_rc != YAPD_OK) return _rc; \
  } while (0)

namespace {

// Rows of a packed prefill chunk (NULL in a block step): row r's tokens are
// rows [row_start[r], row_start[r+1]) of the activations, tok_row names each
// token's row.
struct PackedRows {
  const int32_t* row_start;
  const int32_t* tok_row;
};

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Quantised layers at this many rows or more, given the workspace's wdq
// buffer, dequantise their four weights once into it and run the bf16
// kernels: the fused kernels redo the dequantisation for every row tile,
// while here it is one pass over the weights per layer.  Below, the fused
// kernels read the 4- or 8-bit codes themselves (a quarter or half of the
// bf16 bytes), which is what pays at few rows.
constexpr int kDequantMinRows = 4096;

// bf16 elements of one layer's dequantised projections: qkv, o, gate/up, down.
int64_t layer_weight_elems(int D, int HD, int F) {
  return static_cast<int64_t>(3 * HD) * D + static_cast<int64_t>(D) * HD + static_cast<int64_t>(2 * F) * D +
         static_cast<int64_t>(D) * F;
}

yapd::QWeight qw(const yapd_t3_qweight& w, int bits) {
  return yapd::QWeight{w.packed, static_cast<const uint16_t*>(w.scales), static_cast<const uint16_t*>(w.biases),
                       bits};
}

// The rules of every per-layer call (shapes, pointers, alignment, the
// attention plan), checked before the first launch, so that a rejected call
// leaves the residual, the KV pools and the outputs untouched (the calls below
// check them again).
int model_checks(const yapd_t3_model* m, const yapd_t3_workspace* ws, int rows, int bl, const int32_t* pos0,
                 const int32_t* kv_len) {
  YAPD_REQUIRE(m->n_layers >= 1 && m->layers, "t3_block_forward: no layers");
  YAPD_REQUIRE(ws->residual && ws->q && ws->attn && ws->normed && ws->delta && ws->act && ws->work,
               "t3_block_forward: incomplete workspace");
  YAPD_REQUIRE(al16(ws->residual) && al16(ws->q) && al16(ws->attn) && al16(ws->normed) && al16(ws->delta) &&
                   al16(ws->act),
               "t3_block_forward: workspace activations must be 16-byte aligned");
  const int D = m->hidden, H = m->n_heads, F = m->ffn;
  YAPD_REQUIRE(D % 512 == 0 && D >= 512 && D <= 2048, "t3_block_forward: hidden must be 512, 1024, 1536 or 2048 (got %d)",
               D);
  // attention covers 4 heads per workgroup
  YAPD_REQUIRE(H % 4 == 0 && H >= 4, "t3_block_forward: n_heads must be a multiple of 4 (got %d)", H);
  YAPD_REQUIRE(F % 64 == 0 && F >= 64, "t3_block_forward: ffn must be a multiple of 64 (got %d)", F);
  YAPD_REQUIRE(m->rope_cos && m->rope_sin && m->rope_positions >= 1 && m->final_norm,
               "t3_block_forward: missing RoPE tables or final norm");
  YAPD_REQUIRE(al16(m->rope_cos) && al16(m->rope_sin), "t3_block_forward: RoPE tables must be 16-byte aligned");
  YAPD_REQUIRE(m->page_table && m->n_pages >= 1 && m->n_pages <= INT32_MAX && m->table_cols >= 1 &&
                   m->table_stride >= m->table_cols,
               "t3_block_forward: bad page table");
  const int HD = H * 64;
  for (int li = 0; li < m->n_layers; ++li) {
    const yapd_t3_layer& L = m->layers[li];
    YAPD_REQUIRE(L.ln_in && L.ln_post && L.kv_pool, "t3_block_forward: layer %d has a NULL norm or KV pool", li);
    YAPD_REQUIRE(al16(L.kv_pool), "t3_block_forward: layer %d KV pool must be 16-byte aligned", li);
    if (L.qbits == 0) {
      YAPD_REQUIRE(L.w_qkv && L.w_o && L.w_gate_up && L.w_down, "t3_block_forward: layer %d has a NULL weight", li);
      YAPD_REQUIRE(al16(L.w_qkv) && al16(L.w_o) && al16(L.w_gate_up) && al16(L.w_down),
                   "t3_block_forward: layer %d weights must be 16-byte aligned", li);
    } else {
      YAPD_REQUIRE(!ws->wdq || (al16(ws->wdq) && ws->wdq_elems >= layer_weight_elems(D, HD, F)),
                   "t3_block_forward: wdq must be 16-byte aligned and hold %lld bf16 (got %lld)",
                   static_cast<long long>(layer_weight_elems(D, HD, F)), static_cast<long long>(ws->wdq_elems));
      YAPD_TRY(yapd::qweight_checks(qw(L.q_qkv, L.qbits), 3 * HD, D, "t3_block_forward q_qkv"));
      YAPD_TRY(yapd::qweight_checks(qw(L.q_o, L.qbits), D, HD, "t3_block_forward q_o"));
      YAPD_TRY(yapd::qweight_checks(qw(L.q_gate_up, L.qbits), 2 * F, D, "t3_block_forward q_gate_up"));
      YAPD_TRY(yapd::qweight_checks(qw(L.q_down, L.qbits), D, F, "t3_block_forward q_down"));
    }
    YAPD_TRY(yapd::attn_checks(ws->q, L.kv_pool, m->n_pages, m->page_table, m->table_stride, m->table_cols, kv_len,
                               rows, bl, H, ws->work, ws->n_work, ws->attn));
  }
  YAPD_REQUIRE(ws->n_work >= 1 && (ws->n_merge == 0 || (ws->merge && ws->part_o && ws->part_ml && ws->n_slots >= 1)),
               "t3_block_forward: bad attention plan in the workspace");
  YAPD_REQUIRE(ws->n_merge == 0 || al16(ws->part_o), "t3_block_forward: part_o must be 16-byte aligned");
  YAPD_REQUIRE(pos0 != nullptr, "t3_block_forward: NULL pos0");
  return YAPD_OK;
}

// The layer loop over M activation rows (rows x bl, or a packed chunk's
// tokens), ending in the final norm into hidden_out.
int run_layers(const yapd_t3_model* m, const yapd_t3_workspace* ws, const void* emb, int M, int rows, int bl,
               const int32_t* pos0, const int32_t* kv_len, int causal, const PackedRows* pk, void* hidden_out,
               void* st) {
  const int D = m->hidden, H = m->n_heads, F = m->ffn, HD = H * 64;
  const float scale = 0.125f;  // head_dim ** -0.5 for head_dim 64
  auto* res = ws->residual;
  auto* xn = ws->normed;
  YAPD_TRY(yapd_rmsnorm(nullptr, res, emb, m->layers[0].ln_in, m->layers[0].eps_in, M, D, xn, st));
  const hipStream_t hst = static_cast<hipStream_t>(st);
  for (int li = 0; li < m->n_layers; ++li) {
    const yapd_t3_layer& L = m->layers[li];
    // q: the fused quantised kernels; with dq the weights are dequantised
    // into wdq first and the bf16 kernels run on them
    const bool dq = L.qbits != 0 && ws->wdq != nullptr && M >= kDequantMinRows;
    const bool q = L.qbits != 0 && !dq;
    const void* w_qkv = L.w_qkv;
    const void* w_o = L.w_o;
    const void* w_gate_up = L.w_gate_up;
    const void* w_down = L.w_down;
    if (dq) {
      uint16_t* out[4];
      out[0] = static_cast<uint16_t*>(ws->wdq);
      out[1] = out[0] + static_cast<int64_t>(3 * HD) * D;
      out[2] = out[1] + static_cast<int64_t>(D) * HD;
      out[3] = out[2] + static_cast<int64_t>(2 * F) * D;
      const yapd::QWeight w[4] = {qw(L.q_qkv, L.qbits), qw(L.q_o, L.qbits), qw(L.q_gate_up, L.qbits),
                                  qw(L.q_down, L.qbits)};
      const int N[4] = {3 * HD, D, 2 * F, D}, K[4] = {D, HD, D, F};
      YAPD_TRY(yapd::dequant_affine(w, N, K, out, 4, hst));
      w_qkv = out[0];
      w_o = out[1];
      w_gate_up = out[2];
      w_down = out[3];
    }
    if (q) {
      YAPD_TRY(yapd::qgemm_qkv_rope_kv(xn, D, qw(L.q_qkv, L.qbits), M, D, H, m->rope_cos, m->rope_sin,
                                       m->rope_positions, pos0, bl, rows, pk ? pk->row_start : nullptr,
                                       pk ? pk->tok_row : nullptr, ws->q, L.kv_pool, m->n_pages, m->page_table,
                                       m->table_stride, m->table_cols, hst));
    }
    if (pk == nullptr) {
      if (!q)
        YAPD_TRY(yapd_gemm_qkv_rope_kv(xn, D, w_qkv, M, D, H, m->rope_cos, m->rope_sin, m->rope_positions, pos0,
                                       bl, ws->q, L.kv_pool, m->n_pages, m->page_table, m->table_stride,
                                       m->table_cols, st));
      YAPD_TRY(yapd_attn_paged_block(ws->q, L.kv_pool, m->n_pages, m->page_table, m->table_stride, m->table_cols,
                                     kv_len, rows, bl, H, ws->work, ws->n_work, ws->merge, ws->n_merge, ws->counts,
                                     ws->part_o, ws->part_ml, ws->n_slots, scale, causal, ws->attn, st));
    } else {
      if (!q)
        YAPD_TRY(yapd::gemm_qkv_rope_kv_packed(xn, D, w_qkv, M, D, H, m->rope_cos, m->rope_sin, m->rope_positions,
                                               pos0, rows, pk->row_start, pk->tok_row, ws->q, L.kv_pool, m->n_pages,
                                               m->page_table, m->table_stride, m->table_cols, hst));
      YAPD_TRY(yapd::attn_launch(ws->q, L.kv_pool, m->n_pages, m->page_table, m->table_stride, m->table_cols, kv_len,
                                 rows, bl, H, ws->work, ws->n_work, ws->merge, ws->n_merge, ws->counts, ws->part_o,
                                 ws->part_ml, ws->n_slots, scale, causal, ws->attn, st, pk->row_start, M));
    }
    if (q) {
      YAPD_TRY(yapd::qgemm_residual(ws->attn, HD, qw(L.q_o, L.qbits), M, D, HD, res, D, hst));
    } else {
      YAPD_TRY(yapd_gemm_bf16_residual(ws->attn, HD, w_o, HD, M, D, HD, res, D, st));
    }
    YAPD_TRY(yapd_rmsnorm(nullptr, nullptr, res, L.ln_post, L.eps_post, M, D, xn, st));
    if (q) {
      YAPD_TRY(yapd::qgemm_swiglu(xn, D, qw(L.q_gate_up, L.qbits), M, F, D, ws->act, F, hst));
      YAPD_TRY(yapd::qgemm_residual(ws->act, F, qw(L.q_down, L.qbits), M, D, F, res, D, hst));
    } else {
      YAPD_TRY(yapd_gemm_swiglu(xn, D, w_gate_up, M, F, D, ws->act, F, st));
      YAPD_TRY(yapd_gemm_bf16_residual(ws->act, F, w_down, F, M, D, F, res, D, st));
    }
    const bool last = li + 1 == m->n_layers;
    const void* wn = last ? m->final_norm : m->layers[li + 1].ln_in;
    const float eps = last ? m->final_eps : m->layers[li + 1].eps_in;
    YAPD_TRY(yapd_rmsnorm(nullptr, nullptr, res, wn, eps, M, D, last ? hidden_out : xn, st));
  }
  return YAPD_OK;
}

}  // namespace

extern "C" int yapd_t3_block_forward(const yapd_t3_model* m, const yapd_t3_workspace* ws, const void* block_emb,
                                     int rows, int bl, const int32_t* pos0, const int32_t* kv_len, int causal,
                                     void* hidden_out, const void* head_w, int vocab, const void* shift_ctx,
                                     void* logits, int64_t ld_logits, void* stream) {
  YAPD_REQUIRE(m && ws && block_emb && pos0 && kv_len && hidden_out, "t3_block_forward: NULL pointer");
  YAPD_REQUIRE(rows >= 1 && bl >= 1 && bl <= 64, "t3_block_forward: need rows >= 1, 1 <= bl <= 64");
  YAPD_TRY(model_checks(m, ws, rows, bl, pos0, kv_len));
  YAPD_REQUIRE(!head_w || (shift_ctx && logits && vocab >= 1 && ld_logits >= vocab),
               "t3_block_forward: head needs shift_ctx, logits, vocab >= 1 and ld_logits >= vocab");
  YAPD_TRY(run_layers(m, ws, block_emb, rows * bl, rows, bl, pos0, kv_len, causal, nullptr, hidden_out, stream));
  if (head_w != nullptr) {
    YAPD_TRY(yapd_gemm_head_shift(hidden_out, shift_ctx, rows, bl, m->hidden, head_w, m->hidden, vocab, logits,
                                  ld_logits, stream));
  }
  return YAPD_OK;
}

extern "C" int yapd_t3_prefill_packed(const yapd_t3_model* m, const yapd_t3_workspace* ws, const void* tok_emb,
                                      int n_tokens, int rows, int max_q, const int32_t* row_start,
                                      const int32_t* tok_row, const int32_t* pos0, const int32_t* kv_len,
                                      void* hidden_out, void* stream) {
  YAPD_REQUIRE(m && ws && tok_emb && row_start && tok_row && pos0 && kv_len && hidden_out,
               "t3_prefill_packed: NULL pointer");
  YAPD_REQUIRE(rows >= 1 && max_q >= 1 && max_q <= 64 && n_tokens >= 1 &&
                   static_cast<int64_t>(n_tokens) <= static_cast<int64_t>(rows) * max_q,
               "t3_prefill_packed: need rows >= 1, 1 <= max_q <= 64, 1 <= n_tokens <= rows * max_q");
  YAPD_TRY(model_checks(m, ws, rows, max_q, pos0, kv_len));
  const PackedRows pk{row_start, tok_row};
  return run_layers(m, ws, tok_emb, n_tokens, rows, max_q, pos0, kv_len, 1, &pk, hidden_out, stream);
}
