/* decode_host.c -- a plain C host of the backend's C ABI, driving a model
 * the way the Zig engine does through its shim: GpuContext.init,
 * GpuModelContext.init from borrowed bf16 host tensors, the host ring
 * (DynamicRingBuffer) for slot numbers and active lists, and
 * gpuDispatchForwardToken per token: the prompt token by token without
 * logits except for its last token, then greedy decode
 * (src/interactive.zig:33-48, src/model/forward.zig:33-45,
 * src/gpu/model_dispatch.zig:131-147).
 *
 * Usage: decode_host MODEL_FILE.  The file (little-endian, written by
 * tests/test_gpu_c_host.py):
 *   "GHH1"; u32 vocab, hidden, intermediate, layers, heads, kv_heads,
 *   global_kv_heads, head_dim, global_head_dim, k_eq_v, max_slots, mode,
 *   anchors, window, recall, n_prompt, n_decode; f32 eps, theta, theta_full;
 *   u8 layer_types[64];
 *   per layer: u32 count[13] (bf16 elements of input_layernorm, q_proj,
 *   k_proj, v_proj, o_proj, q_norm, k_norm, post_attention_layernorm,
 *   pre_feedforward_layernorm, gate_proj, up_proj, down_proj,
 *   post_feedforward_layernorm; 0 = absent), f32 layer_scalar, then the
 *   present tensors' bf16 data in that order;
 *   bf16 embed [vocab][hidden]; bf16 final_norm [hidden]; u32 prompt[n_prompt].
 * Prints "tokens:" and the greedy tokens (the last prompt token's, then one
 * per decode step) on one line.  Then runs the engine's --bench sequence
 * (src/model/bench.zig:12-21: one warm-up submitPreRecorded of the decode
 * graph, 20 timed with a host clock) through gh_model_submit_prerecorded,
 * and prints "bench:" with the ms per token and the token the last replay
 * left.  Exits 1 with the backend's message on any failure. */
#define _POSIX_C_SOURCE 199309L
#include <math.h>
#include <stdint.h>
#include <time.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "gemma_hip.h"

static const uint8_t* cur;
static const uint8_t* end;

static int take(void* dst, size_t n) {
  if ((size_t)(end - cur) < n) return 0;
  memcpy(dst, cur, n);
  cur += n;
  return 1;
}

static const uint16_t* take_bf16(size_t n) {
  if ((size_t)(end - cur) < 2 * n) return NULL;
  const uint16_t* p = (const uint16_t*)cur;
  cur += 2 * n;
  return p;
}

static int fail_with(const char* what, gh_status st) {
  fprintf(stderr, "%s failed (status %d): %s\n", what, (int)st, gh_last_error());
  return 1;
}

/* src/model/forward.zig:33-37: x = bf16(E[token]) * sqrt(hidden) */
static void embed_row(const uint16_t* embed, uint32_t token, uint32_t hidden, float* x) {
  const float scale = sqrtf((float)hidden);
  const uint16_t* row = embed + (size_t)token * hidden;
  for (uint32_t i = 0; i < hidden; i++) {
    uint32_t bits = (uint32_t)row[i] << 16;
    float f;
    memcpy(&f, &bits, 4);
    x[i] = f * scale;
  }
}

int main(int argc, char** argv) {
  if (argc != 2) {
    fprintf(stderr, "usage: %s MODEL_FILE\n", argv[0]);
    return 2;
  }
  FILE* f = fopen(argv[1], "rb");
  if (!f) {
    perror(argv[1]);
    return 1;
  }
  fseek(f, 0, SEEK_END);
  const long size = ftell(f);
  fseek(f, 0, SEEK_SET);
  uint8_t* blob = (uint8_t*)malloc((size_t)size);
  if (!blob || fread(blob, 1, (size_t)size, f) != (size_t)size) {
    fprintf(stderr, "cannot read %s\n", argv[1]);
    return 1;
  }
  fclose(f);
  cur = blob;
  end = blob + size;

  char magic[4];
  uint32_t h[17];
  float hf[3];
  gh_model_config cfg;
  memset(&cfg, 0, sizeof cfg);
  if (!take(magic, 4) || memcmp(magic, "GHH1", 4) != 0 || !take(h, sizeof h) ||
      !take(hf, sizeof hf) || !take(cfg.layer_types, 64)) {
    fprintf(stderr, "bad model file header\n");
    return 1;
  }
  cfg.vocab_size = h[0];
  cfg.hidden_size = h[1];
  cfg.intermediate_size = h[2];
  cfg.num_hidden_layers = h[3];
  cfg.num_attention_heads = h[4];
  cfg.num_key_value_heads = h[5];
  cfg.num_global_key_value_heads = h[6];
  cfg.head_dim = h[7];
  cfg.global_head_dim = h[8];
  cfg.attention_k_eq_v = h[9];
  cfg.max_slots = h[10];
  const gh_quant_mode mode = (gh_quant_mode)h[11];
  const uint32_t anchors = h[12], window = h[13], recall = h[14];
  const uint32_t n_prompt = h[15], n_decode = h[16];
  cfg.rms_norm_eps = hf[0];
  cfg.rope_theta = hf[1];
  cfg.rope_theta_full = hf[2];
  if (cfg.num_hidden_layers == 0 || cfg.num_hidden_layers > 64 || n_prompt == 0) {
    fprintf(stderr, "bad model file configuration\n");
    return 1;
  }

  gh_layer_weights* layers =
      (gh_layer_weights*)calloc(cfg.num_hidden_layers, sizeof(gh_layer_weights));
  for (uint32_t l = 0; l < cfg.num_hidden_layers; l++) {
    uint32_t count[13];
    float scalar;
    if (!take(count, sizeof count) || !take(&scalar, 4)) {
      fprintf(stderr, "bad layer %u record\n", l);
      return 1;
    }
    const uint16_t** slot[13] = {
        &layers[l].input_layernorm,          &layers[l].q_proj,
        &layers[l].k_proj,                   &layers[l].v_proj,
        &layers[l].o_proj,                   &layers[l].q_norm,
        &layers[l].k_norm,                   &layers[l].post_attention_layernorm,
        &layers[l].pre_feedforward_layernorm, &layers[l].gate_proj,
        &layers[l].up_proj,                  &layers[l].down_proj,
        &layers[l].post_feedforward_layernorm};
    for (int t = 0; t < 13; t++) {
      *slot[t] = count[t] ? take_bf16(count[t]) : NULL;
      if (count[t] && !*slot[t]) {
        fprintf(stderr, "layer %u tensor %d truncated\n", l, t);
        return 1;
      }
    }
    layers[l].layer_scalar = scalar;
  }
  const uint32_t H = cfg.hidden_size;
  const uint16_t* embed = take_bf16((size_t)cfg.vocab_size * H);
  const uint16_t* final_norm = take_bf16(H);
  uint32_t* prompt = (uint32_t*)malloc((size_t)n_prompt * 4);
  if (!embed || !final_norm || !take(prompt, (size_t)n_prompt * 4)) {
    fprintf(stderr, "model file truncated\n");
    return 1;
  }

  /* GpuContext.init, GpuModelContext.init (the weights are borrowed for the
   * duration of the call only) */
  gh_context* ctx = NULL;
  gh_status st = gh_context_init(NULL, &ctx);
  if (st != GH_OK) return fail_with("gh_context_init", st);
  gh_model* m = NULL;
  st = gh_model_init(ctx, &cfg, layers, embed, final_norm, mode, 0.0f, &m);
  if (st != GH_OK) return fail_with("gh_model_init", st);
  gh_ring* ring = NULL;
  st = gh_ring_create(1, anchors, window, recall, &ring);
  if (st != GH_OK) return fail_with("gh_ring_create", st);
  const uint32_t total = gh_ring_total_slots(ring);
  uint32_t* active = (uint32_t*)malloc((size_t)total * 4);
  float* x = (float*)malloc((size_t)H * 4);

  printf("tokens:");
  uint64_t clock = 0;
  uint32_t token = 0;
  for (uint32_t i = 0; i < n_prompt + n_decode; i++, clock++) {
    const int want_logits = i + 1 >= n_prompt;
    embed_row(embed, i < n_prompt ? prompt[i] : token, H, x);
    const uint32_t slot = gh_ring_activate_slot(ring, 0, clock);
    const uint32_t n = gh_ring_active_slots(ring, 0, clock, active, total);
    st = gh_dispatch_forward_token(m, x, want_logits, clock, slot, active, n, &token);
    if (st != GH_OK) return fail_with("gh_dispatch_forward_token", st);
    if (want_logits) printf(" %u", token);
  }
  printf("\n");

  /* --bench: g.engine.submitPreRecorded(g.cmd_buf_decode), 1 + 20 times */
  st = gh_model_submit_prerecorded(m, GH_GRAPH_DECODE);
  if (st != GH_OK) return fail_with("gh_model_submit_prerecorded", st);
  struct timespec t0, t1;
  clock_gettime(CLOCK_MONOTONIC, &t0);
  for (int i = 0; i < 20; i++) {
    st = gh_model_submit_prerecorded(m, GH_GRAPH_DECODE);
    if (st != GH_OK) return fail_with("gh_model_submit_prerecorded", st);
  }
  clock_gettime(CLOCK_MONOTONIC, &t1);
  const double ms = ((double)(t1.tv_sec - t0.tv_sec) * 1e3 + (double)(t1.tv_nsec - t0.tv_nsec) / 1e6) / 20.0;
  const size_t vocab_bytes = (size_t)cfg.vocab_size * 4;
  float* logits = (float*)malloc(vocab_bytes);
  st = gh_model_read_tensor(m, -1, GH_T_LOGITS, logits, vocab_bytes);
  if (st != GH_OK) return fail_with("gh_model_read_tensor", st);
  uint32_t best = 0;
  for (uint32_t i = 1; i < cfg.vocab_size; i++)
    if (logits[i] > logits[best]) best = i;
  printf("bench: %.4f ms / token, token %u\n", ms, best);
  free(logits);

  gh_ring_destroy(ring);
  gh_model_deinit(m);
  gh_context_deinit(ctx);
  free(x);
  free(active);
  free(prompt);
  free(layers);
  free(blob);
  return 0;
}
