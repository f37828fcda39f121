/*
 * oracle.h -- CPU restatement of the reference's decode math (TEST INFRASTRUCTURE).
 *
 * This library is the checker, never the product.  Only tests/, the smoke()
 * entry of __graft_entry__.py and the cpu_baseline leg of bench.py may load it.
 * The product path (ai-research_amd/) never links or calls it.
 *
 * Every function restates one piece of the reference (Sullux/ai-research, Zig)
 * and cites the file:line it follows.  The reference itself is Zig and cannot
 * be built here (no zig toolchain), so there is no oracle/_ref build; the
 * restatement is pinned instead by known answers, invariants and an
 * independent numpy restatement (tests/test_oracle.py, tests/numpy_ref.py).
 *
 * Parity status per function (what pins it):
 *   orc_bf16_*                 pinned: tensor.zig:30-41 KAT + RNE tie cases
 *   orc_quantize_row_q4_0/q8_0 pinned: hand-derived known answers, invariants,
 *                              independent numpy restatement (bit-exact)
 *   orc_gemv_q4 / q8 / bf16    pinned: kernels.zig:176-183 KAT, constant-weight
 *                              closed form, fp64 brute force
 *   orc_rmsnorm / unit         pinned: closed form (output RMS = 1)
 *   orc_gelu_tanh              pinned: fp64 closed form (tolerance only; the
 *                              reference's std.math.tanh is ulp-level unpinned)
 *   orc_rope_partial           pinned: pos 0 identity, pair norms, angle
 *                              additivity, suffix pass-through
 *   orc_softmax / orc_argmax   pinned: sum to 1; lowest index on ties
 *   orc_ring_*                 pinned: ring_buffer.zig:149-187 KATs + wraparound
 *   orc_attention              pinned: equal scores -> mean(V), S=1 -> V,
 *                              dominant score -> that V, fp64 brute force
 *   orc_forward_layer_batch    pinned: bit-identical to orc_forward_token run
 *                              token by token on the layer (tests/test_oracle.py)
 *   orc_forward_token          pinned: an independent fp64 numpy forward
 *                              (tests/numpy_ref.forward64) within 1e-5, with
 *                              planted mistakes in it shown to miss by >1e-3
 *   orc_embed                  pinned: bit-exact vs a numpy restatement
 *   orc_gate_up_geglu_q4 /     pinned: fp64 brute force; gate/up swap caught
 *   orc_gated_mlp_q4
 *   orc_gate_mean_sq           pinned: fp64 closed form; x_prev update
 *   orc_forward_token_gated    pinned: with every gate open it equals
 *                              orc_forward_token; gated-off layers are the
 *                              identity and write no K/V (checked against
 *                              orc_forward_token on the remaining layers)
 *   orc_qtracker_*             pinned: src/quiescence.zig:63-77 KAT
 */
#ifndef ORACLE_H
#define ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- bf16 (src/tensor.zig:7-18) ---------------------------------------- */
uint16_t orc_bf16_from_f32(float v);
float orc_bf16_to_f32(uint16_t b);
void orc_bf16_from_f32_n(const float *src, uint16_t *dst, size_t n);

/* ---- quantizers (src/quant.zig) ----------------------------------------- */
enum { ORC_QUANT_NONE = 0, ORC_QUANT_Q8 = 1, ORC_QUANT_Q4 = 2 };
void orc_quantize_row_q8_0(uint32_t *dst, const uint16_t *src, size_t n);
void orc_quantize_row_q4_0(uint32_t *dst, const uint16_t *src, size_t n);
size_t orc_quantized_row_words(size_t cols, int mode);
size_t orc_quantized_size_bytes(size_t rows, size_t cols, int mode);
void orc_quantize_matrix(uint32_t *dst, const uint16_t *src, size_t rows,
                         size_t cols, int mode, int nthreads);

/* ---- GEMVs -------------------------------------------------------------- */
void orc_gemv_q4(const uint32_t *w, const float *x, float *y, size_t rows,
                 size_t cols, int nthreads);
void orc_gemv_q8(const uint32_t *w, const float *x, float *y, size_t rows,
                 size_t cols, int nthreads);
void orc_gemv_bf16(const uint16_t *w, const float *x, float *y, size_t rows,
                   size_t cols);

/* ---- elementwise / reductions (src/kernels.zig) ------------------------- */
float orc_dot_f32(const float *a, const float *b, size_t n);
void orc_rmsnorm(float *out, const float *in, const float *w, size_t n, float eps);
void orc_unit_rmsnorm(float *out, const float *in, size_t n, float eps);
float orc_gelu_tanh(float x);
void orc_gate_up_geglu_q4(float *act, const float *x, const uint32_t *wg,
                          const uint32_t *wu, size_t inter, size_t h, int nthreads);
void orc_gated_mlp_q4(float *out, float *act, const float *x,
                      const uint32_t *wg, const uint32_t *wu, const uint32_t *wd,
                      size_t h, size_t inter, int nthreads);
void orc_rope_partial(float *vec, size_t len, size_t pos, size_t head_dim,
                      size_t rotary_dim, float theta);
void orc_softmax(float *v, size_t n);
uint32_t orc_argmax(const float *v, size_t n);

/* ---- ring buffer (src/ring_buffer.zig) ---------------------------------- */
typedef struct orc_ring {
  size_t num_layers, max_kv_dim, num_anchors, window_size, num_recall, total_slots;
  float *k, *v;
  uint64_t *clocks;
  uint8_t *active;
  uint64_t total_ingested;
} orc_ring;
int orc_ring_init(orc_ring *r, size_t num_layers, size_t max_kv_dim,
                  size_t num_anchors, size_t window_size, size_t num_recall);
void orc_ring_deinit(orc_ring *r);
size_t orc_ring_slot_index(const orc_ring *r, uint64_t clock);
size_t orc_ring_activate_slot(orc_ring *r, size_t layer, uint64_t clock);
void orc_ring_write_kv(orc_ring *r, size_t layer, uint64_t clock,
                       const float *k, const float *v, size_t len);
void orc_ring_clear_recall(orc_ring *r);
void orc_ring_write_recall_kv(orc_ring *r, size_t layer, size_t rank,
                              const float *k, const float *v, size_t len, uint64_t clock);
size_t orc_ring_active_slots(const orc_ring *r, size_t layer, uint64_t clock,
                             uint32_t *out);

/* ---- attention pieces (src/model/forward.zig) --------------------------- */
void orc_qkv_norm_rope(float *q, float *k, float *v, const float *q_norm,
                       const float *k_norm, size_t nq, size_t nkv, size_t head_dim,
                       size_t rotary_dim, int k_eq_v, float theta, float eps,
                       uint64_t clock);
void orc_attention(const float *q, const float *k_cache, const float *v_cache,
                   size_t slot_stride, const uint32_t *active, size_t n_active,
                   size_t nq, size_t nkv, size_t head_dim, float *out);

/* ---- one decode step (src/gpu/model_dispatch.zig op order) -------------- */
typedef struct orc_layer {
  int full_attention;
  size_t head_dim, rotary_dim, num_kv_heads;
  int k_eq_v;
  const float *input_norm, *q_norm, *k_norm, *post_attn_norm, *pre_ffn_norm,
      *post_ffn_norm; /* post_* may be NULL */
  float layer_scalar;
  /* Q4_0 or Q8_0 rows; in mode none the bf16 rows (uint16 pairs per word) */
  const uint32_t *wq, *wk, *wv, *wo, *wg, *wu, *wd;
  float *k_cache, *v_cache; /* [total_slots][num_kv_heads*head_dim] */
} orc_layer;

typedef struct orc_model {
  size_t hidden, intermediate, vocab, num_q_heads, num_layers;
  int layer_mode; /* ORC_QUANT_Q4, ORC_QUANT_Q8 or ORC_QUANT_NONE (bf16) */
  float eps, rope_theta, rope_theta_full;
  const uint32_t *lm_head; /* Q8_0 rows; bf16 rows in mode none */
  const float *final_norm;
  const orc_layer *layers;
} orc_model;

void orc_embed(const uint16_t *embed_bf16, uint32_t token, size_t hidden, float *x);
uint32_t orc_forward_token(const orc_model *m, float *x, uint64_t clock,
                           size_t slot_idx, const uint32_t *active, size_t n_active,
                           int want_logits, float *logits, int nthreads);

/* Layer `layer` of the step above for T tokens in order: token t with clock
 * clocks[t], slot slots[t] and the active list active[t * stride ..] of
 * n_active[t] entries; X [T][H] is updated in place, the layer's caches as T
 * calls of orc_forward_token on that one layer would leave them, and every
 * output bit-identical to those calls (the GEMVs become row-tile x token-tile
 * products with the same per-dot summation order).  Returns 0, or -1 when
 * out of memory. */
int orc_forward_layer_batch(const orc_model *m, size_t layer, float *X, size_t T,
                            const uint64_t *clocks, const uint32_t *slots, const uint32_t *active,
                            size_t stride, const uint32_t *n_active, int nthreads);

/* ---- layer gating ------------------------------------------------------- */
/* quiescence_gate.wgsl: mean (x - x_prev)^2 in the shader's order; x_prev <- x */
float orc_gate_mean_sq(const float *x, float *x_prev, size_t H);
/* model_dispatch.zig:45-101: layers >= L/3 gated against x_prev [L][H] */
uint32_t orc_forward_token_gated(const orc_model *m, float *x, uint64_t clock,
                                 size_t slot_idx, const uint32_t *active, size_t n_active,
                                 int want_logits, float *logits, int nthreads,
                                 float *x_prev, float thresh, uint32_t *run);
/* QuiescenceTracker (src/quiescence.zig:3-61), the CPU path's gating */
typedef struct orc_qtracker {
  int enabled;
  float split_ratio, threshold;
  size_t forced_cadence, num_layers;
  uint64_t total_evals, skipped_evals;
} orc_qtracker;
int orc_qtracker_should_execute(orc_qtracker *t, size_t layer, uint64_t clock, const float *x,
                                const float *prev_x, size_t n);

#ifdef __cplusplus
}
#endif
#endif
