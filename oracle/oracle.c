/*
 * oracle.c -- CPU restatement of the reference decode path (TEST INFRASTRUCTURE).
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * this library, as the checker.  Citations are file:line in Sullux/ai-research.
 *
 * Float semantics follow the reference's Zig code: strict IEEE f32, no
 * contraction (built with -ffp-contract=off), left-to-right evaluation.
 */
#include "oracle.h"

#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* bf16: src/tensor.zig:7-18                                                */
/* ------------------------------------------------------------------------ */
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* fromF32: bits + 0x7FFF + ((bits >> 16) & 1), then >> 16 (tensor.zig:9-12).
 * No NaN special case, exactly like the reference. */
uint16_t orc_bf16_from_f32(float v) {
  uint32_t b = f2u(v);
  uint32_t bias = 0x7FFFu + ((b >> 16) & 1u);
  return (uint16_t)((b + bias) >> 16);
}

/* toF32: bits << 16 (tensor.zig:15-18). */
float orc_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

void orc_bf16_from_f32_n(const float *src, uint16_t *dst, size_t n) {
  for (size_t i = 0; i < n; i++) dst[i] = orc_bf16_from_f32(src[i]);
}

/* ------------------------------------------------------------------------ */
/* quantizers: src/quant.zig                                                */
/* ------------------------------------------------------------------------ */
#define QK 32

/* std.math.round: half away from zero.  roundf is exactly that. */
static inline int32_t round_clamp(float p, int32_t lo, int32_t hi) {
  float r = roundf(p);
  /* clamp in float first so the int conversion is always defined; for every
   * finite in-range input this equals clamp(@intFromFloat(round(p))). */
  if (!(r >= (float)lo)) r = (float)lo;
  if (r > (float)hi) r = (float)hi;
  return (int32_t)r;
}

/* quantizeRowQ8_0 (quant.zig:20-51): block = 9 words, word 0 = f32 scale
 * d = amax/127, then 32 int8 little-endian, 4 per word. */
void orc_quantize_row_q8_0(uint32_t *dst, const uint16_t *src, size_t n) {
  size_t nb = n / QK;
  for (size_t b = 0; b < nb; b++) {
    const uint16_t *s = src + b * QK;
    uint32_t *d = dst + b * 9;
    float vals[QK];
    float amax = 0.0f;
    for (int i = 0; i < QK; i++) {
      vals[i] = orc_bf16_to_f32(s[i]);
      float a = fabsf(vals[i]);
      if (a > amax) amax = a;
    }
    float scale = amax / 127.0f;                  /* quant.zig:36 */
    float id = amax > 0.0f ? 127.0f / amax : 0.0f; /* quant.zig:37 */
    d[0] = f2u(scale);
    uint8_t bytes[QK];
    for (int i = 0; i < QK; i++)
      bytes[i] = (uint8_t)(int8_t)round_clamp(vals[i] * id, -128, 127); /* :42 */
    for (int w = 0; w < 8; w++)
      d[1 + w] = (uint32_t)bytes[4 * w] | ((uint32_t)bytes[4 * w + 1] << 8) |
                 ((uint32_t)bytes[4 * w + 2] << 16) | ((uint32_t)bytes[4 * w + 3] << 24);
  }
}

/* quantizeRowQ4_0 (quant.zig:55-90): block = 5 words, word 0 = f32 scale
 * d = amax/7; nibble = clamp(round(v*id), -8, 7) + 8; element j goes to word
 * 1 + j/8 at bit 4*(j%8) (sequential packing, not ggml's lo/hi split). */
void orc_quantize_row_q4_0(uint32_t *dst, const uint16_t *src, size_t n) {
  size_t nb = n / QK;
  for (size_t b = 0; b < nb; b++) {
    const uint16_t *s = src + b * QK;
    uint32_t *d = dst + b * 5;
    float vals[QK];
    float amax = 0.0f;
    for (int i = 0; i < QK; i++) {
      vals[i] = orc_bf16_to_f32(s[i]);
      float a = fabsf(vals[i]);
      if (a > amax) amax = a;
    }
    float scale = amax / 7.0f;                  /* quant.zig:71 */
    float id = amax > 0.0f ? 7.0f / amax : 0.0f; /* quant.zig:72 */
    d[0] = f2u(scale);
    uint32_t nib[QK];
    for (int i = 0; i < QK; i++)
      nib[i] = (uint32_t)(round_clamp(vals[i] * id, -8, 7) + 8); /* :77-78 */
    for (int w = 0; w < 4; w++) {
      uint32_t word = 0;
      for (int k = 0; k < 8; k++) word |= nib[w * 8 + k] << (4 * k); /* :81-88 */
      d[1 + w] = word;
    }
  }
}

/* getQuantizedRowWords (quant.zig:164-171): ceil(cols/32) blocks per row. */
size_t orc_quantized_row_words(size_t cols, int mode) {
  size_t nb = (cols + QK - 1) / QK;
  if (mode == ORC_QUANT_Q8) return nb * 9;
  if (mode == ORC_QUANT_Q4) return nb * 5;
  return cols / 2;
}

size_t orc_quantized_size_bytes(size_t rows, size_t cols, int mode) {
  return rows * orc_quantized_row_words(cols, mode) * 4;
}

/* ---- a minimal row-parallel helper (the reference splits rows into
 * contiguous chunks: quant.zig:135-157, kernels.zig:76-92) ---------------- */
typedef void (*row_fn)(void *ctx, size_t r0, size_t r1);
typedef struct { row_fn fn; void *ctx; size_t r0, r1; } par_task;
static void *par_entry(void *p) {
  par_task *t = (par_task *)p;
  t->fn(t->ctx, t->r0, t->r1);
  return NULL;
}
static void par_rows(size_t rows, int nthreads, row_fn fn, void *ctx) {
  if (nthreads <= 1 || rows < (size_t)nthreads * 4) { fn(ctx, 0, rows); return; }
  if (nthreads > 256) nthreads = 256;
  pthread_t th[256];
  par_task tasks[256];
  size_t chunk = (rows + (size_t)nthreads - 1) / (size_t)nthreads;
  int spawned = 0;
  for (int t = 0; t < nthreads; t++) {
    size_t a = (size_t)t * chunk;
    if (a >= rows) break;
    size_t b = a + chunk < rows ? a + chunk : rows;
    tasks[t] = (par_task){fn, ctx, a, b};
    if (pthread_create(&th[spawned], NULL, par_entry, &tasks[t]) != 0) {
      fn(ctx, a, b);
      continue;
    }
    spawned++;
  }
  for (int t = 0; t < spawned; t++) pthread_join(th[t], NULL);
}

typedef struct { uint32_t *dst; const uint16_t *src; size_t cols, wpr; int mode; } qm_ctx;
static void qm_rows(void *p, size_t r0, size_t r1) {
  qm_ctx *c = (qm_ctx *)p;
  for (size_t r = r0; r < r1; r++) {
    if (c->mode == ORC_QUANT_Q8)
      orc_quantize_row_q8_0(c->dst + r * c->wpr, c->src + r * c->cols, c->cols);
    else
      orc_quantize_row_q4_0(c->dst + r * c->wpr, c->src + r * c->cols, c->cols);
  }
}

/* quantizeMatrix (quant.zig:92-162).  Threading never changes the bytes. */
void orc_quantize_matrix(uint32_t *dst, const uint16_t *src, size_t rows,
                         size_t cols, int mode, int nthreads) {
  if (rows == 0 || cols == 0 || (mode != ORC_QUANT_Q4 && mode != ORC_QUANT_Q8)) return;
  qm_ctx c = {dst, src, cols, orc_quantized_row_words(cols, mode), mode};
  par_rows(rows, nthreads, qm_rows, &c);
}

/* ------------------------------------------------------------------------ */
/* GEMVs                                                                    */
/* ------------------------------------------------------------------------ */
/* Q4_0 dequant dot, the CPU formula of src/test_q4_exec.zig:56-74:
 * weight = (f32(nib) - 8) * d, row_sum += weight * x, sequential. */
static float q4_row_dot(const uint32_t *row, const float *x, size_t cols) {
  float sum = 0.0f;
  size_t nb = cols / QK;
  for (size_t b = 0; b < nb; b++) {
    const uint32_t *blk = row + b * 5;
    float d = u2f(blk[0]);
    for (int w = 0; w < 4; w++) {
      uint32_t p = blk[1 + w];
      for (int n = 0; n < 8; n++) {
        uint32_t nib = (p >> (4 * n)) & 0xFu;
        float weight = ((float)nib - 8.0f) * d;
        sum += weight * x[b * QK + (size_t)w * 8 + (size_t)n];
      }
    }
  }
  return sum;
}

/* Q8_0 dequant dot, shaders/gemv_q8.wgsl:23-37: f32(q) * s * x, in element order. */
static float q8_row_dot(const uint32_t *row, const float *x, size_t cols) {
  float sum = 0.0f;
  size_t nb = cols / QK;
  for (size_t b = 0; b < nb; b++) {
    const uint32_t *blk = row + b * 9;
    float s = u2f(blk[0]);
    for (int j = 0; j < QK; j++) {
      int8_t q = (int8_t)((blk[1 + (j >> 2)] >> (8 * (j & 3))) & 0xFFu);
      sum += (float)q * s * x[b * QK + (size_t)j];
    }
  }
  return sum;
}

typedef struct { const uint32_t *w; const float *x; float *y; size_t cols, wpr; int q8; } gv_ctx;
static void gv_rows(void *p, size_t r0, size_t r1) {
  gv_ctx *c = (gv_ctx *)p;
  for (size_t r = r0; r < r1; r++)
    c->y[r] = c->q8 ? q8_row_dot(c->w + r * c->wpr, c->x, c->cols)
                    : q4_row_dot(c->w + r * c->wpr, c->x, c->cols);
}

void orc_gemv_q4(const uint32_t *w, const float *x, float *y, size_t rows,
                 size_t cols, int nthreads) {
  gv_ctx c = {w, x, y, cols, orc_quantized_row_words(cols, ORC_QUANT_Q4), 0};
  par_rows(rows, nthreads, gv_rows, &c);
}

void orc_gemv_q8(const uint32_t *w, const float *x, float *y, size_t rows,
                 size_t cols, int nthreads) {
  gv_ctx c = {w, x, y, cols, orc_quantized_row_words(cols, ORC_QUANT_Q8), 1};
  par_rows(rows, nthreads, gv_rows, &c);
}

/* dotBf16 (kernels.zig:25-43): 8 lane accumulators, ordered reduce, tail. */
static float dot_bf16(const uint16_t *w, const float *x, size_t n) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  size_t i = 0;
  for (; i + 8 <= n; i += 8)
    for (int l = 0; l < 8; l++) acc[l] += orc_bf16_to_f32(w[i + l]) * x[i + l];
  float sum = acc[0];
  for (int l = 1; l < 8; l++) sum += acc[l];
  for (; i < n; i++) sum += orc_bf16_to_f32(w[i]) * x[i];
  return sum;
}

/* gemv (kernels.zig:68-73) on bf16 rows. */
void orc_gemv_bf16(const uint16_t *w, const float *x, float *y, size_t rows, size_t cols) {
  for (size_t r = 0; r < rows; r++) y[r] = dot_bf16(w + r * cols, x, cols);
}

/* gemvParallel (kernels.zig:76-92): the same rows split over threads. */
typedef struct { const uint16_t *w; const float *x; float *y; size_t cols; } gvb_ctx;
static void gvb_rows(void *p, size_t r0, size_t r1) {
  gvb_ctx *c = (gvb_ctx *)p;
  for (size_t r = r0; r < r1; r++) c->y[r] = dot_bf16(c->w + r * c->cols, c->x, c->cols);
}
static void gemv_bf16_par(const uint16_t *w, const float *x, float *y, size_t rows, size_t cols,
                          int nthreads) {
  gvb_ctx c = {w, x, y, cols};
  par_rows(rows, nthreads, gvb_rows, &c);
}

/* ------------------------------------------------------------------------ */
/* kernels.zig                                                              */
/* ------------------------------------------------------------------------ */
/* dotF32 (kernels.zig:6-22). */
float orc_dot_f32(const float *a, const float *b, size_t n) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  size_t i = 0;
  for (; i + 8 <= n; i += 8)
    for (int l = 0; l < 8; l++) acc[l] += a[i + l] * b[i + l];
  float sum = acc[0];
  for (int l = 1; l < 8; l++) sum += acc[l];
  for (; i < n; i++) sum += a[i] * b[i];
  return sum;
}

/* rmsNorm (kernels.zig:46-52); w holds the bf16 weights widened to f32, as
 * the GPU path stores them (src/gpu/model_gpu.zig:64-73).  In place is OK. */
void orc_rmsnorm(float *out, const float *in, const float *w, size_t n, float eps) {
  float ss = 0.0f;
  for (size_t i = 0; i < n; i++) ss += in[i] * in[i];
  float r = 1.0f / sqrtf(ss / (float)n + eps);
  for (size_t i = 0; i < n; i++) out[i] = in[i] * r * w[i];
}

/* unitRmsNorm (kernels.zig:55-61). */
void orc_unit_rmsnorm(float *out, const float *in, size_t n, float eps) {
  float ss = 0.0f;
  for (size_t i = 0; i < n; i++) ss += in[i] * in[i];
  float r = 1.0f / sqrtf(ss / (float)n + eps);
  for (size_t i = 0; i < n; i++) out[i] = in[i] * r;
}

/* geluTanh (kernels.zig:94-97), constants as in shaders/fused_mlp_q4.wgsl:15-18. */
float orc_gelu_tanh(float x) {
  float inner = 0.7978845608f * (x + 0.044715f * x * x * x);
  return 0.5f * x * (1.0f + tanhf(inner));
}

typedef struct { float *act; const float *x; const uint32_t *wg, *wu; size_t h, wpr; } gu_ctx;
static void gu_rows(void *p, size_t r0, size_t r1) {
  gu_ctx *c = (gu_ctx *)p;
  for (size_t r = r0; r < r1; r++) {
    float g = q4_row_dot(c->wg + r * c->wpr, c->x, c->h);
    float u = q4_row_dot(c->wu + r * c->wpr, c->x, c->h);
    c->act[r] = orc_gelu_tanh(g) * u; /* kernels.zig:112-114 */
  }
}

/* gate+up half of gatedMlp (kernels.zig:100-119) on Q4_0 rows. */
void orc_gate_up_geglu_q4(float *act, const float *x, const uint32_t *wg,
                          const uint32_t *wu, size_t inter, size_t h, int nthreads) {
  gu_ctx c = {act, x, wg, wu, h, orc_quantized_row_words(h, ORC_QUANT_Q4)};
  par_rows(inter, nthreads, gu_rows, &c);
}

/* gatedMlp (kernels.zig:100-129): act = gelu(Wg x) * (Wu x); out = Wd act. */
void orc_gated_mlp_q4(float *out, float *act, const float *x,
                      const uint32_t *wg, const uint32_t *wu, const uint32_t *wd,
                      size_t h, size_t inter, int nthreads) {
  orc_gate_up_geglu_q4(act, x, wg, wu, inter, h, nthreads);
  orc_gemv_q4(wd, act, out, h, inter, nthreads);
}

/* applyRopePartial (kernels.zig:132-150): per head, pairs (i, i + rot/2) for
 * i < rot/2 with freq = 1 / theta^(2i/rot); dims >= rot untouched. */
void orc_rope_partial(float *vec, size_t len, size_t pos, size_t head_dim,
                      size_t rotary_dim, float theta) {
  size_t nh = len / head_dim, half = rotary_dim / 2;
  for (size_t h = 0; h < nh; h++) {
    float *v = vec + h * head_dim;
    for (size_t i = 0; i < half; i++) {
      float freq = 1.0f / powf(theta, (float)(2 * i) / (float)rotary_dim);
      float angle = (float)pos * freq;
      float c = cosf(angle), s = sinf(angle);
      float v0 = v[i], v1 = v[i + half];
      v[i] = v0 * c - v1 * s;
      v[i + half] = v0 * s + v1 * c;
    }
  }
}

/* softmax (kernels.zig:152-162). */
void orc_softmax(float *v, size_t n) {
  float mx = -INFINITY;
  for (size_t i = 0; i < n; i++) mx = fmaxf(mx, v[i]);
  float sum = 0.0f;
  for (size_t i = 0; i < n; i++) { v[i] = expf(v[i] - mx); sum += v[i]; }
  float inv = 1.0f / sum;
  for (size_t i = 0; i < n; i++) v[i] *= inv;
}

/* sampleArgmax (kernels.zig:164-174): strict '>' so the lowest index wins ties. */
uint32_t orc_argmax(const float *v, size_t n) {
  uint32_t best = 0;
  float bv = v[0];
  for (size_t i = 1; i < n; i++)
    if (v[i] > bv) { bv = v[i]; best = (uint32_t)i; }
  return best;
}

/* ------------------------------------------------------------------------ */
/* ring buffer: src/ring_buffer.zig                                         */
/* ------------------------------------------------------------------------ */
int orc_ring_init(orc_ring *r, size_t num_layers, size_t max_kv_dim,
                  size_t num_anchors, size_t window_size, size_t num_recall) {
  memset(r, 0, sizeof(*r));
  r->num_layers = num_layers; r->max_kv_dim = max_kv_dim;
  r->num_anchors = num_anchors; r->window_size = window_size; r->num_recall = num_recall;
  r->total_slots = num_anchors + window_size + num_recall; /* ring_buffer.zig:23 */
  size_t ne = num_layers * r->total_slots * max_kv_dim;
  r->k = (float *)calloc(ne ? ne : 1, sizeof(float));
  r->v = (float *)calloc(ne ? ne : 1, sizeof(float));
  r->clocks = (uint64_t *)calloc(num_layers * r->total_slots + 1, sizeof(uint64_t));
  r->active = (uint8_t *)calloc(num_layers * r->total_slots + 1, 1);
  if (!r->k || !r->v || !r->clocks || !r->active) { orc_ring_deinit(r); return -1; }
  return 0;
}

void orc_ring_deinit(orc_ring *r) {
  free(r->k); free(r->v); free(r->clocks); free(r->active);
  r->k = r->v = NULL; r->clocks = NULL; r->active = NULL;
}

/* getSlotIndex (ring_buffer.zig:56-59). */
size_t orc_ring_slot_index(const orc_ring *r, uint64_t clock) {
  if (clock < r->num_anchors) return (size_t)clock;
  return r->num_anchors + (size_t)((clock - r->num_anchors) % r->window_size);
}

/* activateSlot (ring_buffer.zig:61-68). */
size_t orc_ring_activate_slot(orc_ring *r, size_t layer, uint64_t clock) {
  size_t slot = orc_ring_slot_index(r, clock);
  size_t gi = layer * r->total_slots + slot;
  r->clocks[gi] = clock;
  r->active[gi] = 1;
  if (layer == 0 && clock >= r->total_ingested) r->total_ingested = clock + 1;
  return slot;
}

/* writeKV (ring_buffer.zig:70-80). */
void orc_ring_write_kv(orc_ring *r, size_t layer, uint64_t clock,
                       const float *k, const float *v, size_t len) {
  size_t slot = orc_ring_slot_index(r, clock);
  size_t gi = layer * r->total_slots + slot;
  memcpy(r->k + gi * r->max_kv_dim, k, len * sizeof(float));
  memcpy(r->v + gi * r->max_kv_dim, v, len * sizeof(float));
  r->clocks[gi] = clock;
  r->active[gi] = 1;
  if (layer == 0 && clock >= r->total_ingested) r->total_ingested = clock + 1;
}

/* clearRecall (ring_buffer.zig:82-88). */
void orc_ring_clear_recall(orc_ring *r) {
  size_t start = r->num_anchors + r->window_size;
  for (size_t l = 0; l < r->num_layers; l++)
    memset(r->active + l * r->total_slots + start, 0, r->num_recall);
}

/* writeRecallKV (ring_buffer.zig:90-99). */
void orc_ring_write_recall_kv(orc_ring *r, size_t layer, size_t rank,
                              const float *k, const float *v, size_t len, uint64_t clock) {
  size_t slot = r->num_anchors + r->window_size + rank;
  size_t gi = layer * r->total_slots + slot;
  memcpy(r->k + gi * r->max_kv_dim, k, len * sizeof(float));
  memcpy(r->v + gi * r->max_kv_dim, v, len * sizeof(float));
  r->clocks[gi] = clock;
  r->active[gi] = 1;
}

/* getActiveSlots (ring_buffer.zig:101-136): anchors first, then live window
 * slots in slot order, then recall slots whose clock <= now. */
size_t orc_ring_active_slots(const orc_ring *r, size_t layer, uint64_t clock, uint32_t *out) {
  size_t base = layer * r->total_slots, n = 0;
  size_t alim = clock + 1 < r->num_anchors ? (size_t)clock + 1 : r->num_anchors;
  for (size_t s = 0; s < alim; s++)
    if (r->active[base + s]) out[n++] = (uint32_t)s;
  size_t rstart = r->num_anchors + r->window_size;
  if (clock >= r->num_anchors) {
    uint64_t minc = clock >= r->window_size ? clock - r->window_size + 1 : r->num_anchors;
    for (size_t s = r->num_anchors; s < rstart; s++) {
      if (!r->active[base + s]) continue;
      uint64_t c = r->clocks[base + s];
      if (c >= minc && c <= clock) out[n++] = (uint32_t)s;
    }
  }
  for (size_t s = rstart; s < r->total_slots; s++) {
    if (!r->active[base + s]) continue;
    if (r->clocks[base + s] <= clock) out[n++] = (uint32_t)s;
  }
  return n;
}

/* ------------------------------------------------------------------------ */
/* attention pieces: src/model/forward.zig                                  */
/* ------------------------------------------------------------------------ */
/* forward.zig:125-143: v <- k when k_eq_v; per-head q RMSNorm(q_norm) + RoPE;
 * per-head k RMSNorm(k_norm), v unit RMS, k RoPE.  All in place. */
void orc_qkv_norm_rope(float *q, float *k, float *v, const float *q_norm,
                       const float *k_norm, size_t nq, size_t nkv, size_t head_dim,
                       size_t rotary_dim, int k_eq_v, float theta, float eps,
                       uint64_t clock) {
  size_t kv_dim = nkv * head_dim;
  if (k_eq_v) memcpy(v, k, kv_dim * sizeof(float));
  for (size_t h = 0; h < nq; h++)
    orc_rmsnorm(q + h * head_dim, q + h * head_dim, q_norm, head_dim, eps);
  orc_rope_partial(q, nq * head_dim, (size_t)clock, head_dim, rotary_dim, theta);
  for (size_t h = 0; h < nkv; h++) {
    orc_rmsnorm(k + h * head_dim, k + h * head_dim, k_norm, head_dim, eps);
    orc_unit_rmsnorm(v + h * head_dim, v + h * head_dim, head_dim, eps);
  }
  orc_rope_partial(k, kv_dim, (size_t)clock, head_dim, rotary_dim, theta);
}

/* runAttentionHeads (forward.zig:77-104): scale 1.0 (forward.zig:80),
 * kv head = h / (nq / nkv), softmax over the active slots, out = sum p * V. */
void orc_attention(const float *q, const float *k_cache, const float *v_cache,
                   size_t slot_stride, const uint32_t *active, size_t n_active,
                   size_t nq, size_t nkv, size_t head_dim, float *out) {
  size_t group = nq / nkv;
  float *sc = (float *)malloc((n_active ? n_active : 1) * sizeof(float));
  for (size_t h = 0; h < nq; h++) {
    size_t kh = h / group;
    const float *qh = q + h * head_dim;
    for (size_t i = 0; i < n_active; i++)
      sc[i] = orc_dot_f32(qh, k_cache + (size_t)active[i] * slot_stride + kh * head_dim,
                          head_dim) * 1.0f;
    orc_softmax(sc, n_active);
    float *oh = out + h * head_dim;
    memset(oh, 0, head_dim * sizeof(float));
    for (size_t i = 0; i < n_active; i++) {
      const float *vh = v_cache + (size_t)active[i] * slot_stride + kh * head_dim;
      for (size_t d = 0; d < head_dim; d++) oh[d] += sc[i] * vh[d];
    }
  }
  free(sc);
}

/* ------------------------------------------------------------------------ */
/* one decode step                                                          */
/* ------------------------------------------------------------------------ */
/* forward.zig:33-37: x = bf16(E[token]) * sqrt(H). */
void orc_embed(const uint16_t *embed_bf16, uint32_t token, size_t hidden, float *x) {
  float scale = sqrtf((float)hidden);
  const uint16_t *row = embed_bf16 + (size_t)token * hidden;
  for (size_t i = 0; i < hidden; i++) x[i] = orc_bf16_to_f32(row[i]) * scale;
}

/* Mode none (the reference's --gpu bf16 mode, src/gpu/model_gpu.zig:51-57)
 * keeps the checkpoint's bf16 rows: the layer pointers then address bf16
 * elements, two per word.  The CPU forward uses the same bf16 rows
 * (src/model/forward.zig:112-124). */
static void layer_gemv(const orc_model *m, const uint32_t *w, const float *x,
                       float *y, size_t rows, size_t cols, int nt) {
  if (m->layer_mode == ORC_QUANT_Q8) orc_gemv_q8(w, x, y, rows, cols, nt);
  else if (m->layer_mode == ORC_QUANT_Q4) orc_gemv_q4(w, x, y, rows, cols, nt);
  else gemv_bf16_par((const uint16_t *)w, x, y, rows, cols, nt);
}

/* one row of gate or up in the layer mode */
static float mode_row_dot(int mode, const uint32_t *w, size_t r, size_t wpr, const float *x,
                          size_t h) {
  if (mode == ORC_QUANT_Q8) return q8_row_dot(w + r * wpr, x, h);
  if (mode == ORC_QUANT_Q4) return q4_row_dot(w + r * wpr, x, h);
  return dot_bf16((const uint16_t *)w + r * h, x, h);
}

typedef struct { float *act; const float *x; const uint32_t *wg, *wu; size_t h, wpr; int mode; } gum_ctx;
static void gum_rows(void *p, size_t r0, size_t r1) {
  gum_ctx *c = (gum_ctx *)p;
  for (size_t r = r0; r < r1; r++) {
    float g = mode_row_dot(c->mode, c->wg, r, c->wpr, c->x, c->h);
    float u = mode_row_dot(c->mode, c->wu, r, c->wpr, c->x, c->h);
    c->act[r] = orc_gelu_tanh(g) * u;
  }
}

/* One token through every layer in the order the GPU graph records it
 * (src/gpu/model_dispatch.zig:10-43, 103-129), which equals the CPU forward
 * (src/model/forward.zig:49-70) with quantized weights:
 *   normed = RMSNorm(x, input_norm); q,k,v = W normed
 *   q/k norm + RoPE, v unit RMS, K/V -> cache[slot_idx]; attention over active
 *   o = Wo attn; [o = RMSNorm(o, post_attn)]; x = x + o
 *   normed = RMSNorm(x, pre_ffn); act = gelu(Wg normed) * (Wu normed); m = Wd act
 *   [m = RMSNorm(m, post_ffn)]; x = (x + m) * layer_scalar
 * tail: logits = Q8 head . RMSNorm(x, final_norm); token = argmax (raw logits).
 * x is updated in place; returns the greedy token when want_logits. */
typedef struct {
  float *normed, *q, *k, *v, *attn, *o, *act;
} orc_scratch;

static int scratch_init(const orc_model *m, orc_scratch *s) {
  size_t H = m->hidden, I = m->intermediate, nq = m->num_q_heads, maxq = 0, maxkv = 0;
  for (size_t l = 0; l < m->num_layers; l++) {
    const orc_layer *L = &m->layers[l];
    if (nq * L->head_dim > maxq) maxq = nq * L->head_dim;
    if (L->num_kv_heads * L->head_dim > maxkv) maxkv = L->num_kv_heads * L->head_dim;
  }
  if (!maxq) maxq = 1;
  if (!maxkv) maxkv = 1;
  s->normed = (float *)malloc(H * sizeof(float));
  s->q = (float *)malloc(maxq * sizeof(float));
  s->k = (float *)malloc(maxkv * sizeof(float));
  s->v = (float *)malloc(maxkv * sizeof(float));
  s->attn = (float *)malloc(maxq * sizeof(float));
  s->o = (float *)malloc(H * sizeof(float));
  s->act = (float *)malloc(I * sizeof(float));
  return s->normed && s->q && s->k && s->v && s->attn && s->o && s->act;
}

static void scratch_free(orc_scratch *s) {
  free(s->normed); free(s->q); free(s->k); free(s->v); free(s->attn); free(s->o); free(s->act);
}

/* One layer (the op order above), x updated in place. */
static void forward_layer(const orc_model *m, const orc_layer *L, orc_scratch *s, float *x,
                          uint64_t clock, size_t slot_idx, const uint32_t *active,
                          size_t n_active, int nt) {
  size_t H = m->hidden, I = m->intermediate, nq = m->num_q_heads;
  size_t wpr_h = orc_quantized_row_words(H, m->layer_mode);
  size_t hd = L->head_dim, qd = nq * hd, kvd = L->num_kv_heads * hd;
  float theta = L->full_attention ? m->rope_theta_full : m->rope_theta;
  orc_rmsnorm(s->normed, x, L->input_norm, H, m->eps);
  layer_gemv(m, L->wq, s->normed, s->q, qd, H, nt);
  layer_gemv(m, L->wk, s->normed, s->k, kvd, H, nt);
  if (!L->k_eq_v) layer_gemv(m, L->wv, s->normed, s->v, kvd, H, nt);
  orc_qkv_norm_rope(s->q, s->k, s->v, L->q_norm, L->k_norm, nq, L->num_kv_heads, hd,
                    L->rotary_dim, L->k_eq_v, theta, m->eps, clock);
  memcpy(L->k_cache + slot_idx * kvd, s->k, kvd * sizeof(float));
  memcpy(L->v_cache + slot_idx * kvd, s->v, kvd * sizeof(float));
  orc_attention(s->q, L->k_cache, L->v_cache, kvd, active, n_active, nq, L->num_kv_heads, hd,
                s->attn);
  layer_gemv(m, L->wo, s->attn, s->o, H, qd, nt);
  if (L->post_attn_norm) orc_rmsnorm(s->o, s->o, L->post_attn_norm, H, m->eps);
  for (size_t i = 0; i < H; i++) x[i] = (x[i] + s->o[i]) * 1.0f;
  orc_rmsnorm(s->normed, x, L->pre_ffn_norm, H, m->eps);
  gum_ctx gc = {s->act, s->normed, L->wg, L->wu, H, wpr_h, m->layer_mode};
  par_rows(I, nt, gum_rows, &gc);
  layer_gemv(m, L->wd, s->act, s->o, H, I, nt);
  if (L->post_ffn_norm) orc_rmsnorm(s->o, s->o, L->post_ffn_norm, H, m->eps);
  for (size_t i = 0; i < H; i++) x[i] = (x[i] + s->o[i]) * L->layer_scalar;
}

static uint32_t forward_tail(const orc_model *m, orc_scratch *s, const float *x, float *logits,
                             int nt) {
  orc_rmsnorm(s->normed, x, m->final_norm, m->hidden, m->eps);
  if (m->layer_mode == ORC_QUANT_NONE)  /* the bf16 embedding (model_gpu.zig:160-161) */
    gemv_bf16_par((const uint16_t *)m->lm_head, s->normed, logits, m->vocab, m->hidden, nt);
  else
    orc_gemv_q8(m->lm_head, s->normed, logits, m->vocab, m->hidden, nt);
  return orc_argmax(logits, m->vocab);
}

uint32_t orc_forward_token(const orc_model *m, float *x, uint64_t clock,
                           size_t slot_idx, const uint32_t *active, size_t n_active,
                           int want_logits, float *logits, int nt) {
  orc_scratch s;
  uint32_t tok = 0;
  if (scratch_init(m, &s)) {
    for (size_t l = 0; l < m->num_layers; l++)
      forward_layer(m, &m->layers[l], &s, x, clock, slot_idx, active, n_active, nt);
    if (want_logits) tok = forward_tail(m, &s, x, logits, nt);
  }
  scratch_free(&s);
  return tok;
}

/* ------------------------------------------------------------------------ */
/* one layer over a batch of tokens                                         */
/* ------------------------------------------------------------------------ */
/* The row dots of a batch: Y[t][r] = the dot of row r of W (Q4_0 or Q8_0)
 * with token t's vector, for rows [r0, r1).  Each dot takes the per-token
 * GEMV's weights (q4_row_dot: (f32(nib) - 8) * d; q8_row_dot: f32(q) * s)
 * and its sequential sum from element 0, so Y[t][r] is bit-identical to
 * orc_gemv_q4 / orc_gemv_q8 on token t alone.  The batch only changes the
 * loop nest: a tile of BR rows is dequantized once and meets BT tokens per
 * pass (xt is the batch transposed, [cols][T]), with one accumulator per
 * (row, token). */
#define BR 4
#define BT 16
typedef struct {
  const uint32_t *w;
  const float *xt;
  float *y;
  size_t cols, wpr, T, ystride;
  int mode;
} bg_ctx;

static void dequant_row(int mode, const uint32_t *row, size_t cols, float *out) {
  size_t nb = cols / QK;
  for (size_t b = 0; b < nb; b++) {
    if (mode == ORC_QUANT_Q4) {
      const uint32_t *blk = row + b * 5;
      float d = u2f(blk[0]);
      for (int w = 0; w < 4; w++)
        for (int n = 0; n < 8; n++)
          out[b * QK + (size_t)w * 8 + (size_t)n] = ((float)((blk[1 + w] >> (4 * n)) & 0xFu) - 8.0f) * d;
    } else {
      const uint32_t *blk = row + b * 9;
      float sc = u2f(blk[0]);
      for (int j = 0; j < QK; j++)
        out[b * QK + (size_t)j] = (float)(int8_t)((blk[1 + (j >> 2)] >> (8 * (j & 3))) & 0xFFu) * sc;
    }
  }
}

/* A full BR x BT tile (4 rows x 16 tokens) in AVX2 registers: per element
 * j, acc[i][t] = acc[i][t] + w[i][j] * x[t][j] as one multiply and one add
 * (no fused multiply-add), the same two roundings as the scalar loop. */
static void bg_tile_full(const float *wt, size_t cols, const float *xt, size_t T,
                         float acc[BR][BT]) {
  __m256 a00 = _mm256_setzero_ps(), a01 = _mm256_setzero_ps();
  __m256 a10 = _mm256_setzero_ps(), a11 = _mm256_setzero_ps();
  __m256 a20 = _mm256_setzero_ps(), a21 = _mm256_setzero_ps();
  __m256 a30 = _mm256_setzero_ps(), a31 = _mm256_setzero_ps();
  const float *w0 = wt, *w1 = wt + cols, *w2 = wt + 2 * cols, *w3 = wt + 3 * cols;
  for (size_t j = 0; j < cols; j++) {
    const __m256 x0 = _mm256_loadu_ps(xt + j * T), x1 = _mm256_loadu_ps(xt + j * T + 8);
    __m256 w = _mm256_broadcast_ss(w0 + j);
    a00 = _mm256_add_ps(a00, _mm256_mul_ps(w, x0));
    a01 = _mm256_add_ps(a01, _mm256_mul_ps(w, x1));
    w = _mm256_broadcast_ss(w1 + j);
    a10 = _mm256_add_ps(a10, _mm256_mul_ps(w, x0));
    a11 = _mm256_add_ps(a11, _mm256_mul_ps(w, x1));
    w = _mm256_broadcast_ss(w2 + j);
    a20 = _mm256_add_ps(a20, _mm256_mul_ps(w, x0));
    a21 = _mm256_add_ps(a21, _mm256_mul_ps(w, x1));
    w = _mm256_broadcast_ss(w3 + j);
    a30 = _mm256_add_ps(a30, _mm256_mul_ps(w, x0));
    a31 = _mm256_add_ps(a31, _mm256_mul_ps(w, x1));
  }
  _mm256_storeu_ps(acc[0], a00);
  _mm256_storeu_ps(acc[0] + 8, a01);
  _mm256_storeu_ps(acc[1], a10);
  _mm256_storeu_ps(acc[1] + 8, a11);
  _mm256_storeu_ps(acc[2], a20);
  _mm256_storeu_ps(acc[2] + 8, a21);
  _mm256_storeu_ps(acc[3], a30);
  _mm256_storeu_ps(acc[3] + 8, a31);
}

static void bg_rows(void *p, size_t r0, size_t r1) {
  bg_ctx *c = (bg_ctx *)p;
  float *wt = (float *)malloc(BR * c->cols * sizeof(float));
  if (!wt) return;
  float acc[BR][BT];
  for (size_t rb = r0; rb < r1; rb += BR) {
    size_t nr = r1 - rb < BR ? r1 - rb : BR;
    for (size_t i = 0; i < nr; i++) dequant_row(c->mode, c->w + (rb + i) * c->wpr, c->cols, wt + i * c->cols);
    for (size_t t0 = 0; t0 < c->T; t0 += BT) {
      size_t nt = c->T - t0 < BT ? c->T - t0 : BT;
      if (nr == BR && nt == BT) {
        bg_tile_full(wt, c->cols, c->xt + t0, c->T, acc);
      } else {
        memset(acc, 0, sizeof(acc));
        for (size_t j = 0; j < c->cols; j++) {
          const float *xj = c->xt + j * c->T + t0;
          for (size_t i = 0; i < nr; i++) {
            const float w = wt[i * c->cols + j];
            for (size_t t = 0; t < nt; t++) acc[i][t] = acc[i][t] + w * xj[t];
          }
        }
      }
      for (size_t t = 0; t < nt; t++)
        for (size_t i = 0; i < nr; i++) c->y[(t0 + t) * c->ystride + rb + i] = acc[i][t];
    }
  }
  free(wt);
}

/* out[c][t] = in[t][c] */
static void transpose(const float *in, size_t T, size_t cols, float *out) {
  for (size_t t = 0; t < T; t++)
    for (size_t c = 0; c < cols; c++) out[c * T + t] = in[t * cols + c];
}

static void batch_gemm(int mode, const uint32_t *w, const float *xt, float *y, size_t rows,
                       size_t cols, size_t T, int nt) {
  bg_ctx c = {w, xt, y, cols, orc_quantized_row_words(cols, mode), T, rows, mode};
  par_rows(rows, nt, bg_rows, &c);
}

typedef struct {
  const float *q;
  const orc_layer *L;
  size_t kvd, qd, nq, stride;
  const uint32_t *active, *n_active;
  float *out;
} ba_ctx;
static void ba_tokens(void *p, size_t t0, size_t t1) {
  ba_ctx *c = (ba_ctx *)p;
  for (size_t t = t0; t < t1; t++)
    orc_attention(c->q + t * c->qd, c->L->k_cache, c->L->v_cache, c->kvd, c->active + t * c->stride,
                  c->n_active[t], c->nq, c->L->num_kv_heads, c->L->head_dim, c->out + t * c->qd);
}

int orc_forward_layer_batch(const orc_model *m, size_t layer, float *X, size_t T,
                            const uint64_t *clocks, const uint32_t *slots, const uint32_t *active,
                            size_t stride, const uint32_t *n_active, int nt) {
  const orc_layer *L = &m->layers[layer];
  size_t H = m->hidden, I = m->intermediate, nq = m->num_q_heads;
  size_t hd = L->head_dim, qd = nq * hd, kvd = L->num_kv_heads * hd;
  float theta = L->full_attention ? m->rope_theta_full : m->rope_theta;
  if (T == 0) return 0;
  if (m->layer_mode != ORC_QUANT_Q4 && m->layer_mode != ORC_QUANT_Q8) {
    /* bf16 rows: the per-token layer, token by token */
    orc_scratch s;
    if (!scratch_init(m, &s)) { scratch_free(&s); return -1; }
    for (size_t t = 0; t < T; t++)
      forward_layer(m, L, &s, X + t * H, clocks[t], slots[t], active + t * stride, n_active[t], nt);
    scratch_free(&s);
    return 0;
  }
  size_t maxk = H > I ? H : I;
  if (qd > maxk) maxk = qd;
  float *xn = (float *)malloc(T * H * sizeof(float));
  float *xt = (float *)malloc(T * maxk * sizeof(float));
  float *q = (float *)malloc(T * qd * sizeof(float));
  float *k = (float *)malloc(T * kvd * sizeof(float));
  float *v = (float *)malloc(T * kvd * sizeof(float));
  float *at = (float *)malloc(T * qd * sizeof(float));
  float *o = (float *)malloc(T * H * sizeof(float));
  float *g = (float *)malloc(T * I * sizeof(float));
  float *u = (float *)malloc(T * I * sizeof(float));
  int ok = xn && xt && q && k && v && at && o && g && u;
  if (ok) {
    /* normed = RMSNorm(x, input_norm); q, k, v = W normed */
    for (size_t t = 0; t < T; t++) orc_rmsnorm(xn + t * H, X + t * H, L->input_norm, H, m->eps);
    transpose(xn, T, H, xt);
    batch_gemm(m->layer_mode, L->wq, xt, q, qd, H, T, nt);
    batch_gemm(m->layer_mode, L->wk, xt, k, kvd, H, T, nt);
    if (!L->k_eq_v) batch_gemm(m->layer_mode, L->wv, xt, v, kvd, H, T, nt);
    for (size_t t = 0; t < T; t++)
      orc_qkv_norm_rope(q + t * qd, k + t * kvd, v + t * kvd, L->q_norm, L->k_norm, nq,
                        L->num_kv_heads, hd, L->rotary_dim, L->k_eq_v, theta, m->eps, clocks[t]);
    /* K/V into the cache and attention, in token order.  When no slot is
     * written twice and no token lists a slot a later token writes, writing
     * every row first leaves each token the cache it sees in order, and the
     * tokens attend in parallel. */
    int in_order = 1;
    for (size_t t = 0; t < T && in_order; t++) {
      for (size_t t2 = t + 1; t2 < T && in_order; t2++) in_order = slots[t2] != slots[t];
      for (size_t i = 0; i < n_active[t] && in_order; i++)
        for (size_t t2 = t + 1; t2 < T && in_order; t2++)
          in_order = active[t * stride + i] != slots[t2];
    }
    ba_ctx bc = {q, L, kvd, qd, nq, stride, active, n_active, at};
    if (in_order) {
      for (size_t t = 0; t < T; t++) {
        memcpy(L->k_cache + slots[t] * kvd, k + t * kvd, kvd * sizeof(float));
        memcpy(L->v_cache + slots[t] * kvd, v + t * kvd, kvd * sizeof(float));
      }
      par_rows(T, nt, ba_tokens, &bc);
    } else {
      for (size_t t = 0; t < T; t++) {
        memcpy(L->k_cache + slots[t] * kvd, k + t * kvd, kvd * sizeof(float));
        memcpy(L->v_cache + slots[t] * kvd, v + t * kvd, kvd * sizeof(float));
        ba_tokens(&bc, t, t + 1);
      }
    }
    /* o = Wo attn; [RMSNorm(o, post_attn)]; x = x + o */
    transpose(at, T, qd, xt);
    batch_gemm(m->layer_mode, L->wo, xt, o, H, qd, T, nt);
    for (size_t t = 0; t < T; t++) {
      float *xr = X + t * H, *orow = o + t * H;
      if (L->post_attn_norm) orc_rmsnorm(orow, orow, L->post_attn_norm, H, m->eps);
      for (size_t i = 0; i < H; i++) xr[i] = (xr[i] + orow[i]) * 1.0f;
      orc_rmsnorm(xn + t * H, xr, L->pre_ffn_norm, H, m->eps);
    }
    /* act = gelu(Wg normed) * (Wu normed); m = Wd act */
    transpose(xn, T, H, xt);
    batch_gemm(m->layer_mode, L->wg, xt, g, I, H, T, nt);
    batch_gemm(m->layer_mode, L->wu, xt, u, I, H, T, nt);
    for (size_t i = 0; i < T * I; i++) g[i] = orc_gelu_tanh(g[i]) * u[i];
    transpose(g, T, I, xt);
    batch_gemm(m->layer_mode, L->wd, xt, o, H, I, T, nt);
    /* [RMSNorm(m, post_ffn)]; x = (x + m) * layer_scalar */
    for (size_t t = 0; t < T; t++) {
      float *xr = X + t * H, *orow = o + t * H;
      if (L->post_ffn_norm) orc_rmsnorm(orow, orow, L->post_ffn_norm, H, m->eps);
      for (size_t i = 0; i < H; i++) xr[i] = (xr[i] + orow[i]) * L->layer_scalar;
    }
  }
  free(xn); free(xt); free(q); free(k); free(v); free(at); free(o); free(g); free(u);
  return ok ? 0 : -1;
}

/* quiescence_gate.wgsl:16-62: the mean over H of (x - x_prev)^2, summed the
 * way the shader sums it (32 lanes, lane k over elements k, k + 32, ...; then
 * s[l] += s[l + 16], s[l + 8], s[l + 4], s[l + 2] and s[0] + s[1]), and
 * x_prev <- x. */
float orc_gate_mean_sq(const float *x, float *x_prev, size_t H) {
  float s[32];
  for (size_t lane = 0; lane < 32; lane++) {
    float acc = 0.0f;
    for (size_t i = lane; i < H; i += 32) {
      float d = x[i] - x_prev[i];
      acc = acc + d * d;
    }
    s[lane] = acc;
  }
  for (size_t i = 0; i < H; i++) x_prev[i] = x[i];
  for (size_t w = 16; w >= 2; w /= 2)
    for (size_t l = 0; l < w; l++) s[l] = s[l] + s[l + w];
  return (s[0] + s[1]) / (float)H;
}

/* The GPU graph with layer gating (src/gpu/model_dispatch.zig:45-101,
 * 103-129): layers l < L/3 always run; a layer l >= L/3 first runs the gate
 * (orc_gate_mean_sq against x_prev[l], which it then overwrites) and runs
 * only when the mean square is >= thresh or thresh <= 0.  A gated-off layer
 * is skipped whole: no K/V write, x unchanged.  run[l] gets 1 or 0. */
uint32_t orc_forward_token_gated(const orc_model *m, float *x, uint64_t clock, size_t slot_idx,
                                 const uint32_t *active, size_t n_active, int want_logits,
                                 float *logits, int nt, float *x_prev, float thresh,
                                 uint32_t *run) {
  orc_scratch s;
  uint32_t tok = 0;
  size_t dense_limit = m->num_layers / 3;
  if (scratch_init(m, &s)) {
    for (size_t l = 0; l < m->num_layers; l++) {
      int go = 1;
      if (l >= dense_limit) {
        float ms = orc_gate_mean_sq(x, x_prev + l * m->hidden, m->hidden);
        go = (ms >= thresh) || (thresh <= 0.0f);
      }
      if (run) run[l] = (uint32_t)go;
      if (go) forward_layer(m, &m->layers[l], &s, x, clock, slot_idx, active, n_active, nt);
    }
    if (want_logits) tok = forward_tail(m, &s, x, logits, nt);
  }
  scratch_free(&s);
  return tok;
}

/* QuiescenceTracker.shouldExecute (src/quiescence.zig:29-55), the CPU
 * path's layer gating: lower layers (l < split_ratio * L) and clocks on the
 * forced cadence always run; otherwise a layer runs unless the relative
 * velocity sqrt(sum (x - prev)^2 / sum x^2) (0 when sum x^2 <= 1e-12) is
 * below the threshold. */
int orc_qtracker_should_execute(orc_qtracker *t, size_t layer, uint64_t clock, const float *x,
                                const float *prev_x, size_t n) {
  if (!t->enabled) return 1;
  size_t split = (size_t)((float)t->num_layers * t->split_ratio);
  if (layer < split) return 1;
  if (clock % t->forced_cadence == 0) return 1;
  t->total_evals++;
  float dsum = 0.0f, nsum = 0.0f;
  for (size_t i = 0; i < n; i++) {
    float d = x[i] - prev_x[i];
    dsum += d * d;
    nsum += x[i] * x[i];
  }
  float vel = nsum > 1e-12f ? sqrtf(dsum / nsum) : 0.0f;
  if (vel < t->threshold) {
    t->skipped_evals++;
    return 0;
  }
  return 1;
}
