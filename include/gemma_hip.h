/*
 * gemma_hip.h -- C ABI of the MI355X (gfx950) decode backend.
 *
 * This is the drop-in boundary for the Vulkan backend of Sullux/ai-research
 * (src/gpu.zig, the src/gpu/ directory and the WGSL shaders under shaders/).
 * A Zig host binds it with
 * @cImport; every entry point names the reference interface it replaces.
 *
 * Conventions
 *  - Plain pointers and sizes only.  "dev" pointers are device (HBM)
 *    addresses, from gh_buffer_alloc or any HIP allocator on the same device.
 *  - Every call returns gh_status; GH_OK is 0.  Nothing is swallowed (the
 *    reference returns token 0 on a failed submit, model_dispatch.zig:145).
 *    gh_last_error() gives the message of the calling thread's last failure.
 *  - Kernel entry points (gh_gemv_*, ...) are enqueued on the context's single
 *    in-order stream and return at once, like recording into the reference's
 *    command buffer; gh_sync waits, like submitPreRecorded (kernels.zig:147).
 *  - Weight layouts are the reference's, unchanged (src/quant.zig):
 *      Q4_0 row = ceil(K/32) blocks x 5 u32  {f32 d, 4 words of 8 nibbles}
 *      Q8_0 row = ceil(K/32) blocks x 9 u32  {f32 d, 8 words of 4 int8}
 *    KV caches are [slot][kv_heads*head_dim] f32 per layer, slots numbered as
 *    src/ring_buffer.zig numbers them ([anchors | window | recall]).
 */
#ifndef GEMMA_HIP_H
#define GEMMA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum gh_status {
  GH_OK = 0,
  GH_ERR_NO_DEVICE = 1,      /* NoVulkanDevices / NoComputeDeviceFound (context.zig:24-68) */
  GH_ERR_CODE_OBJECT = 2,    /* a gfx950 code object failed to load */
  GH_ERR_ALLOC = 3,          /* device or host allocation failed (buffer.zig:20-44) */
  GH_ERR_INVALID = 4,        /* bad argument (null pointer, zero size, ...) */
  GH_ERR_UNSUPPORTED = 5,    /* shape outside what the kernels handle */
  GH_ERR_HIP = 6             /* a HIP runtime call failed (launch, copy, sync) */
} gh_status;

/* QuantMode (src/quant.zig:3-13). */
typedef enum gh_quant_mode { GH_QUANT_NONE = 0, GH_QUANT_Q8 = 1, GH_QUANT_Q4 = 2 } gh_quant_mode;

typedef struct gh_context gh_context;

/* ---- context: GpuContext (src/gpu/context.zig:13-104) -------------------- */
/* Number of visible HIP devices (0 when none); never fails. */
int gh_device_count(void);
/* GpuContext.init (context.zig:17): picks device 0, loads the gfx950 code
 * objects from code_object_dir (NULL = the directory holding this library). */
gh_status gh_context_init(const char *code_object_dir, gh_context **out);
/* GpuContext.deinit (context.zig:104). */
void gh_context_deinit(gh_context *ctx);
/* GpuContext.device_name (context.zig:15). */
const char *gh_context_device_name(const gh_context *ctx);
const char *gh_last_error(void);
/* Waits for all work enqueued on the context (submitPreRecorded's fence wait,
 * src/gpu/kernels.zig:147-157). */
gh_status gh_sync(gh_context *ctx);

/* ---- buffers: GpuBuffer (src/gpu/buffer.zig:13-53) ------------------------ */
/* GpuBuffer.init: 256-byte aligned device memory. */
gh_status gh_buffer_alloc(gh_context *ctx, size_t bytes, void **dev);
/* GpuBuffer.deinit. */
gh_status gh_buffer_free(gh_context *ctx, void *dev);
/* The reference writes through a mapped pointer (asSlice); here copies are
 * explicit and synchronous with the context stream. */
gh_status gh_buffer_write(gh_context *ctx, void *dev_dst, const void *host_src, size_t bytes);
gh_status gh_buffer_read(gh_context *ctx, void *host_dst, const void *dev_src, size_t bytes);
gh_status gh_buffer_copy(gh_context *ctx, void *dev_dst, const void *dev_src, size_t bytes);
gh_status gh_buffer_fill_u32(gh_context *ctx, void *dev, uint32_t value, size_t count);

/* HBM read-bandwidth probe (no reference counterpart; measurement only: the
 * attainable read rate the GEMV streams are judged against).  Reads `bytes` of
 * dev once with 16-byte loads, per_lane (1, 2, 4 or 8) loads in flight per
 * lane, over `grid` workgroups of 256 threads (0: 4 per CU); contiguous = 0
 * strides the grid over the whole buffer, 1 gives each workgroup its own
 * contiguous share.  bytes must be a multiple of 16 * 256 * per_lane * grid.
 * Writes one float per workgroup (the sum of what it read) to sums. */
gh_status gh_read_probe(gh_context *ctx, const void *dev, size_t bytes, uint32_t per_lane,
                        uint32_t contiguous, uint32_t grid, float *sums);

/* ---- timing on the context stream (no reference counterpart: the reference
 * times with host clocks, src/model/bench.zig:14-21) ------------------------ */
gh_status gh_event_create(gh_context *ctx, void **ev);
gh_status gh_event_record(gh_context *ctx, void *ev);
gh_status gh_event_elapsed_ms(void *ev_start, void *ev_end, float *ms);
gh_status gh_event_destroy(void *ev);

/* ---- pre-recorded work: recordForwardGraph + submitPreRecorded
 * (src/gpu/model_dispatch.zig:103-129, src/gpu/kernels.zig:147-157).  Work
 * enqueued on the context between begin and end is captured into a HIP graph
 * instead of running; gh_graph_launch replays it on the context stream. ---- */
gh_status gh_graph_begin(gh_context *ctx);
gh_status gh_graph_end(gh_context *ctx, void **graph);
gh_status gh_graph_launch(gh_context *ctx, void *graph);
gh_status gh_graph_destroy(void *graph);

/* ---- quantization: src/quant.zig ------------------------------------------ */
/* getQuantizedRowWords (quant.zig:164-171). */
size_t gh_quantized_row_words(size_t cols, gh_quant_mode mode);
/* getQuantizedSizeBytes (quant.zig:173-175). */
size_t gh_quantized_size_bytes(size_t rows, size_t cols, gh_quant_mode mode);
/* quantizeMatrix (quant.zig:92-162) on the host, nthreads <= 0 means 16. */
gh_status gh_quantize_matrix(uint32_t *dst, const uint16_t *src_bf16, size_t rows,
                             size_t cols, gh_quant_mode mode, int nthreads);
/* quantizeMatrix on the device: bf16 [rows][cols] in HBM -> blocks in HBM,
 * byte-identical to the host routine.  cols % 32 == 0. */
gh_status gh_quantize_matrix_dev(gh_context *ctx, void *dst_dev, const void *src_bf16_dev,
                                 size_t rows, size_t cols, gh_quant_mode mode);

/* ---- synthetic inputs (no reference counterpart) --------------------------
 * Deterministic N(mean, std) draws: element i of (seed, stream) has the same
 * bits on the host and on the device.  Used for random-init weights and
 * inputs; bf16 variants round with src/tensor.zig's RNE. */
gh_status gh_synth_normal_f32(float *dst, size_t n, uint64_t seed, uint64_t stream,
                              double mean, double stddev, uint64_t offset);
gh_status gh_synth_normal_bf16(uint16_t *dst, size_t n, uint64_t seed, uint64_t stream,
                               double mean, double stddev, uint64_t offset);
gh_status gh_synth_normal_f32_dev(gh_context *ctx, float *dst_dev, size_t n, uint64_t seed,
                                  uint64_t stream, double mean, double stddev, uint64_t offset);
gh_status gh_synth_normal_bf16_dev(gh_context *ctx, uint16_t *dst_dev, size_t n, uint64_t seed,
                                   uint64_t stream, double mean, double stddev, uint64_t offset);
gh_status gh_synth_uniform_u32(uint32_t *dst, size_t n, uint64_t seed, uint64_t stream,
                               uint32_t bound);

/* ---- engine kernels: GpuEngine.record* (src/gpu/kernels.zig:80-142) ------ */
/* recordGemv (kernels.zig:80-83), shaders/gemv_q4.wgsl: Y[M] = deq(W)[M x K] . X[K].
 * K % 128 == 0 (the reference's 4-block unroll), W 16-byte aligned. */
gh_status gh_gemv_q4(gh_context *ctx, const void *W, const float *X, float *Y,
                     uint32_t M, uint32_t K);
/* recordGemvLogits / Q8 pipeline (kernels.zig:88-91), shaders/gemv_q8.wgsl. */
gh_status gh_gemv_q8(gh_context *ctx, const void *W, const float *X, float *Y,
                     uint32_t M, uint32_t K);
/* recordGemv in mode none (the --gpu flag; kernels.zig:36 selects
 * shaders/gemv_bf16.wgsl:1-63): Y[M] = W[M x K] . X[K] with W row-major bf16
 * widened exactly to f32.  K % 128 == 0, W 16-byte aligned. */
gh_status gh_gemv_bf16(gh_context *ctx, const void *W, const float *X, float *Y,
                       uint32_t M, uint32_t K);
/* recordGateUpSwiGlu (kernels.zig:92-95), shaders/fused_mlp_q4.wgsl:
 * Y[r] = gelu_tanh(Wg[r] . X) * (Wu[r] . X) for r < M. */
gh_status gh_gate_up_geglu_q4(gh_context *ctx, const void *Wg, const void *Wu,
                              const float *X, float *Y, uint32_t M, uint32_t K);

/* ---- fused decode building blocks (no single reference counterpart: each
 * fuses a norm dispatch into the GEMV that consumes it) ---------------------
 * The x prologue every workgroup applies before the GEMV:
 *   mode 0: x as given
 *   mode 1: RMSNorm(x) * norm                               (recordRmsNorm)
 *   mode 2: xn = (x + r') * scalar, r' = RMSNorm(r) * r_norm (r as given when
 *           r_norm is null), xn written to x_out, then RMSNorm(xn) * norm
 *           (recordRmsNorm of the post norm + recordAddRmsNorm,
 *            src/gpu/model_dispatch.zig:32-34,39-41)
 * All vectors have K floats, 16-byte aligned; x_out must not alias x or r. */
typedef struct gh_xprologue {
  const float *x, *r, *r_norm, *norm;
  float *x_out;
  float scalar, eps;
  uint32_t mode;
} gh_xprologue;
/* Y = W . prologue(x) with Q4_0, Q8_0 or (GH_QUANT_NONE) bf16 rows
 * (recordRmsNorm + recordGemv). */
gh_status gh_norm_gemv(gh_context *ctx, gh_quant_mode mode, const void *W, float *Y, uint32_t M,
                       uint32_t K, const gh_xprologue *pro);
/* Y = gelu_tanh(Wg . x) * (Wu . x), x = prologue (recordAddRmsNorm +
 * recordGateUpSwiGlu); Q4_0, Q8_0 or bf16 rows.  (For mode none the
 * reference binds the Q4 shader to bf16 rows, kernels.zig:41; the bf16 form
 * computes the CPU path's gatedMlp, src/kernels.zig:100-129.) */
gh_status gh_norm_gate_up_geglu(gh_context *ctx, gh_quant_mode mode, const void *Wg,
                                const void *Wu, float *Y, uint32_t M, uint32_t K,
                                const gh_xprologue *pro);
/* Q8_0 vocab projection of prologue(x) with the greedy argmax fused in
 * (recordRmsNorm + recordGemvLogits + recordArgmax, model_dispatch.zig:121-127);
 * *token (device u32) gets the lowest index of the largest logit; logits
 * (device, M floats) are written when non-null. */
gh_status gh_norm_gemv_argmax_q8(gh_context *ctx, const void *W, float *logits, uint32_t *token,
                                 uint32_t M, uint32_t K, const gh_xprologue *pro);
/* The same with the bf16 head of mode none (the embedding itself,
 * model_gpu.zig:160-161; gemv_logits = the bf16 GEMV, kernels.zig:38). */
gh_status gh_norm_gemv_argmax_bf16(gh_context *ctx, const void *W, float *logits,
                                   uint32_t *token, uint32_t M, uint32_t K,
                                   const gh_xprologue *pro);

/* recordRmsNorm (kernels.zig:108-111), shaders/rmsnorm.wgsl:
 * Y = X * (mean(X^2) + eps)^-1/2 * W.  Y may alias X. */
gh_status gh_rmsnorm(gh_context *ctx, const float *X, const float *W, float *Y, uint32_t dim,
                     float eps);
/* recordAddRmsNorm (kernels.zig:100-103), shaders/add_rmsnorm.wgsl:
 * X <- (X + R) * scalar in place, then Y = RMSNorm(X) * W. */
gh_status gh_add_rmsnorm(gh_context *ctx, float *X, const float *R, const float *W, float *Y,
                         uint32_t dim, float eps, float scalar);
/* recordQkvRope (kernels.zig:124-129), shaders/qkv_rope.wgsl: per-head
 * RMSNorm(q_norm) + split-half RoPE on the first rotary_dim dims of every
 * query head (into Q_out, which may be Q_in); RMSNorm(k_norm) + RoPE of each
 * key head into K_cache and unit-RMS of each value head (the raw key head when
 * k_eq_v) into V_cache, both at row step_params[1] of [slot][num_kv*head_dim].
 * step_params (device, u32) = {clock, slot_idx, S, 0}. */
gh_status gh_qkv_rope(gh_context *ctx, const float *Q_in, const float *K_in, const float *V_in,
                      const float *Q_norm, const float *K_norm, float *Q_out, float *K_cache,
                      float *V_cache, const uint32_t *step_params, uint32_t num_q,
                      uint32_t num_kv, uint32_t head_dim, uint32_t rotary_dim, uint32_t k_eq_v,
                      float theta, float eps);
/* recordDecodeAttn (kernels.zig:116-119), shaders/decode_attn.wgsl: for
 * every query head h (kv head h / gqa_ratio), softmax over the S =
 * step_params[2] active slots of inv_sqrt_dim * (Q[h] . K[slot]), then the
 * weighted sum of V[slot].  The reference passes inv_sqrt_dim = 1.0
 * (model/forward.zig:80).  step_params[3] bit 1 (value 2; the reference
 * writes 0) declares the active list to be 0 .. S-1, which spares reading it.
 * kv_dim = (num_q_heads / gqa_ratio) * head_dim;
 * head_dim % 4 == 0, <= 512; gqa_ratio <= 4.  The first call allocates the
 * context's split-K scratch (do not make that call inside graph capture). */
gh_status gh_decode_attn(gh_context *ctx, const float *Q, const float *K_cache,
                         const float *V_cache, const uint32_t *active_slots, float *out,
                         const uint32_t *step_params, uint32_t head_dim, uint32_t kv_dim,
                         uint32_t gqa_ratio, float inv_sqrt_dim, uint32_t num_q_heads);
/* recordQkvRope + recordDecodeAttn (kernels.zig:116-129) as the decode graph
 * runs them back to back (model_dispatch.zig:22-25), in one split-K launch
 * plus the split merge: per-head RMSNorm(q_norm) + RoPE of the query heads,
 * RMSNorm(k_norm) + RoPE of the key heads and unit-RMS of the value heads
 * (the raw key heads when k_eq_v) written to K_cache / V_cache at row
 * step_params[1], then attention of every query head (kv head h / (num_q /
 * num_kv), scale 1.0, model/forward.zig:80) over the step_params[2] active
 * slots into out [num_q][head_dim].  Q_in is left unchanged.  max_slots sets
 * the split count as the model's ring does.  rope_table (nullable) holds the
 * angles as gh_rope_table writes them; null computes them in the kernel.
 * step_params[3] bit 1 (value 2) may declare the active list to be 0 .. S-1,
 * which spares reading it.  The first call allocates the context's split
 * scratch (not inside graph capture). */
gh_status gh_qkv_rope_attn(gh_context *ctx, const float *Q_in, const float *K_in,
                           const float *V_in, const float *Q_norm, const float *K_norm,
                           float *K_cache, float *V_cache, const uint32_t *active_slots,
                           const uint32_t *step_params, float *out, uint32_t num_q,
                           uint32_t num_kv, uint32_t head_dim, uint32_t rotary_dim,
                           uint32_t k_eq_v, float theta, float eps, uint32_t max_slots,
                           const float *rope_table);
/* The RoPE angles of the clock step_params[0] for one (rotary_dim, theta)
 * into table (device, 512 floats: cos of pairs 0 .. rotary_dim/2 - 1 from
 * index 0, their sin from index 256), computed as the attention prologue
 * computes them (applyRopePartial, src/kernels.zig:132-150).  The decode
 * graph builds the tables of both layer types once per token; passing one
 * to gh_qkv_rope_attn spares each launch the powf/cosf/sinf work. */
gh_status gh_rope_table(gh_context *ctx, const uint32_t *step_params, uint32_t rotary_dim,
                        float theta, float *table);
/* gh_qkv_rope_attn without any allocation (no reference counterpart: it is
 * for callers that cannot allocate -- code under HIP graph capture, serving
 * loops or harnesses that forbid hipMalloc).  Same arguments, kernels and
 * results; the split partials live in a fixed 1 MiB device array of this
 * library (one per GPU, held until the process ends) instead of context
 * scratch that the first call allocates.  Shapes whose partials need more
 * (num_kv * splits * (num_q / num_kv) * (head_dim + 4) * 4 bytes; 332,800
 * for 8 kv heads of 256 with 2 query heads each at 640 slots) are refused
 * with GH_ERR_UNSUPPORTED.  All calls on one GPU share the array: calls that
 * overlap on one GPU (other streams or threads) race. */
gh_status gh_qkv_rope_attn_noalloc(gh_context *ctx, const float *Q_in, const float *K_in,
                                   const float *V_in, const float *Q_norm, const float *K_norm,
                                   float *K_cache, float *V_cache, const uint32_t *active_slots,
                                   const uint32_t *step_params, float *out, uint32_t num_q,
                                   uint32_t num_kv, uint32_t head_dim, uint32_t rotary_dim,
                                   uint32_t k_eq_v, float theta, float eps, uint32_t max_slots,
                                   const float *rope_table);
/* recordArgmax (kernels.zig:139-142), shaders/argmax.wgsl, with the CPU
 * path's tie rule (sampleArgmax, src/kernels.zig:164-174): the lowest index
 * of the largest value.  out_token is a device u32. */
gh_status gh_argmax(gh_context *ctx, const float *logits, uint32_t *out_token, uint32_t vocab);

/* ---- batched prefill GEMMs (no reference counterpart: the reference
 * prefills token by token through its decode graph, src/interactive.zig:33-37,
 * src/gpu/model_dispatch.zig:144).  One projection of T prompt tokens on the
 * matrix cores: C[T][N] = A[T][K] . deq(W)[N][K]^T with A f32 row-major
 * (16-byte aligned) and W in the quant.zig row layout of mode (Q4 or Q8), or
 * bf16 rows in mode GH_QUANT_NONE (16-byte aligned); the weights enter
 * exactly (integer values with f32 block scales applied to the block sums,
 * or the bf16 values), the activations as two fp16 halves of a / s with s a
 * power of two per row (no fp16 overflow; bf16 halves for bf16 weights),
 * fp32 accumulation; K % 32 == 0 and K <= 16384.  All pointers are device
 * pointers. */
gh_status gh_prefill_gemm(gh_context *ctx, gh_quant_mode mode, const void *W, const float *A,
                          float *C, uint32_t T, uint32_t N, uint32_t K);
/* act[T][N] = gelu_tanh(A . deq(Wg)^T) * (A . deq(Wu)^T): the batched form of
 * shaders/fused_mlp_q4.wgsl. */
gh_status gh_prefill_gate_up_geglu(gh_context *ctx, gh_quant_mode mode, const void *Wg,
                                   const void *Wu, const float *A, float *act, uint32_t T,
                                   uint32_t N, uint32_t K);

/* ---- ring bookkeeping: DynamicRingBuffer (src/ring_buffer.zig:7-147) -------
 * The host side of the [anchors | window | recall] ring: which slot a clock
 * maps to and which slots a token attends over.  The K/V values live in the
 * model's device caches; these calls produce the slot_idx / active list that
 * gh_dispatch_forward_token takes. */
typedef struct gh_ring gh_ring;
/* DynamicRingBuffer.init (ring_buffer.zig:19-36); total = A + W + R slots. */
gh_status gh_ring_create(uint32_t num_layers, uint32_t num_anchors, uint32_t window_size,
                         uint32_t num_recall, gh_ring **out);
void gh_ring_destroy(gh_ring *r);
uint32_t gh_ring_total_slots(const gh_ring *r);
/* getSlotIndex (ring_buffer.zig:56-59). */
uint32_t gh_ring_slot_index(const gh_ring *r, uint64_t clock);
/* activateSlot (ring_buffer.zig:61-68). */
uint32_t gh_ring_activate_slot(gh_ring *r, uint32_t layer, uint64_t clock);
/* clearRecall (ring_buffer.zig:82-88). */
void gh_ring_clear_recall(gh_ring *r);
/* writeRecallKV's slot bookkeeping (ring_buffer.zig:90-99); returns the slot. */
uint32_t gh_ring_activate_recall(gh_ring *r, uint32_t layer, uint32_t rank, uint64_t clock);
/* getActiveSlots (ring_buffer.zig:101-136): writes up to cap slots, returns
 * the full count. */
uint32_t gh_ring_active_slots(const gh_ring *r, uint32_t layer, uint64_t clock, uint32_t *out,
                              uint32_t cap);

/* ---- model: GpuModelContext + gpuDispatchForwardToken ---------------------
 * (src/gpu/model_gpu.zig:35-197, src/gpu/model_dispatch.zig:103-147) */
typedef struct gh_model gh_model;

/* ModelConfig (src/model/types.zig:43-61) fields the device path uses.
 * Per-layer shapes follow src/model/loader.zig:36-42: full-attention layers
 * use global_head_dim, rotary_dim = head_dim / 4, num_global_key_value_heads,
 * rope_theta_full and k_eq_v = attention_k_eq_v; sliding layers use head_dim,
 * rotary_dim = head_dim, num_key_value_heads, rope_theta.  max_slots is the
 * ring size (anchors + window + recall) of the per-layer K/V caches. */
typedef struct gh_model_config {
  uint32_t vocab_size, hidden_size, intermediate_size, num_hidden_layers;
  uint32_t num_attention_heads, num_key_value_heads, num_global_key_value_heads;
  uint32_t head_dim, global_head_dim, attention_k_eq_v, max_slots;
  float rms_norm_eps, rope_theta, rope_theta_full;
  uint8_t layer_types[64]; /* 1 = full_attention, 0 = sliding_attention */
} gh_model_config;

/* LayerWeights (src/model/types.zig:13-41): borrowed bf16 host pointers,
 * row-major [out][in]; v_proj, post_* and k_norm may be null (k_norm null =
 * ones, v_proj null = the key projection is used as value, as
 * src/gpu/model_gpu.zig:124 does). */
typedef struct gh_layer_weights {
  const uint16_t *input_layernorm, *q_proj, *k_proj, *v_proj, *o_proj, *q_norm, *k_norm;
  const uint16_t *post_attention_layernorm, *pre_feedforward_layernorm;
  const uint16_t *gate_proj, *up_proj, *down_proj, *post_feedforward_layernorm;
  float layer_scalar; /* 1.0 when the checkpoint has none */
} gh_layer_weights;

/* GpuModelContext.init (model_gpu.zig:75): quantizes every layer matrix with
 * quantizeMatrix's bytes (Q4_0 or Q8_0 per mode), or keeps the bf16 rows in
 * mode GH_QUANT_NONE (createWeightBuffer, model_gpu.zig:51-57); the tied LM
 * head is Q8_0 in the quantized modes and bf16 in mode none (model_gpu.zig:
 * 160-161).  Widens norms to f32, allocates the K/V ring caches and records
 * the decode and prefill graphs.  embed_tokens is
 * [vocab][hidden] bf16.  quiescence_thresh != 0 records the decode graph
 * with layer gating, as gh_model_set_quiescence describes; 0 records it
 * ungated (the reference's default). */
gh_status gh_model_init(gh_context *ctx, const gh_model_config *cfg,
                        const gh_layer_weights *layers, const uint16_t *embed_tokens,
                        const uint16_t *final_norm, gh_quant_mode mode,
                        float quiescence_thresh, gh_model **out);
/* Random-init model of the same architecture (no reference counterpart):
 * every matrix N(0, 0.02) and every norm 1 + N(0, 0.1), drawn on the device
 * with the synthetic generator, rounded to bf16 and quantized exactly as
 * gh_model_init would; layer_scalar 1.  The bf16 embedding stays on the device
 * for gh_model_embed. */
gh_status gh_model_init_synthetic(gh_context *ctx, const gh_model_config *cfg,
                                  gh_quant_mode mode, uint64_t seed, gh_model **out);
/* GpuModelContext.deinit (model_gpu.zig:187). */
void gh_model_deinit(gh_model *m);

/* gpuDispatchForwardToken (model_dispatch.zig:131-147): x = the token's
 * embedding [hidden] (host), clock, slot_idx = ring.activateSlot(0, clock)
 * and the active slots from ring.getActiveSlots (u32, host).  When want_logits
 * the decode graph runs and *out_token receives the greedy token; otherwise
 * the prefill graph (no LM head) runs and *out_token is 0.  Every layer writes
 * this token's K/V into its cache at slot_idx.  x, the step record and the
 * list go up in one copy before the graph replays (the graph holds kernels
 * only).  After gh_model_ring_init, slot_idx must be the ring's slot for the
 * clock, and the call also records the activation in the device ring. */
gh_status gh_dispatch_forward_token(gh_model *m, const float *x, int want_logits, uint64_t clock,
                                    uint32_t slot_idx, const uint32_t *active_slots,
                                    uint32_t n_active, uint32_t *out_token);
/* T prompt tokens in one call: the result of calling gh_dispatch_forward_token
 * for each token in order (want_logits only on the last), computed layer by
 * layer over the whole batch with the prefill GEMMs (no reference
 * counterpart; the reference has no batched prefill).  x is [T][hidden]
 * (host); token t has position clocks[t], ring slot slot_idx[t] and active
 * list active[t * active_stride ..] of n_active[t] entries (host, as
 * ring.activateSlot / getActiveSlots give them).  Every layer writes each
 * token's K/V at its slot.  A batch that writes one slot twice, or in which
 * a token's active list holds a slot that a later token of the batch writes
 * (any prompt after the window has wrapped), writes its K/V to staging rows
 * past the ring slots (min(max_slots, 256) per cache) and moves them into
 * the slots after the layers (longer such batches run as consecutive chunks
 * of that many tokens).  A batch of at most 2 tokens (Q4 weights) or 1
 * token (Q8, bf16) runs token by token through the recorded graphs, which is
 * faster at that size (environment GH_PF_SEQ_MAX at model init overrides
 * it).  With layer gating on, a
 * last token with logits runs the gated decode graph after the others (see
 * gh_model_set_quiescence).  Otherwise the first call allocates the model's
 * prefill buffers for T tokens, and a call that needs more of the context's
 * scratch (split-K planes, split attention partials) grows it; so a prefill
 * is not to be recorded inside graph capture. */
gh_status gh_model_prefill(gh_model *m, const float *x, uint32_t T, const uint64_t *clocks,
                           const uint32_t *slot_idx, const uint32_t *active,
                           uint32_t active_stride, const uint32_t *n_active, int want_logits,
                           uint32_t *out_token);
/* x = bf16(E[token]) * sqrt(hidden) (src/model/forward.zig:33-37) for a
 * synthetic model, whose bf16 embedding lives on the device. */
gh_status gh_model_embed(gh_model *m, uint32_t token, float *x_host);

/* ---- device-resident ring bookkeeping ------------------------------------
 * The model keeps layer 0's DynamicRingBuffer state (src/ring_buffer.zig:
 * 7-147: a clock and an active flag per slot) in HBM, plus a host mirror.  A
 * token then needs only x and its clock: the decode graph's first kernel
 * activates the clock's slot (activateSlot, ring_buffer.zig:61-68) and builds
 * slot_idx, S and the active list (getSlotIndex / getActiveSlots,
 * ring_buffer.zig:56-59,101-136), which the host computes per token in the
 * reference (src/model/forward.zig:42-43, src/gpu/model_dispatch.zig:136-142).
 * DynamicRingBuffer.init for the device state (ring_buffer.zig:19-36): A
 * anchors, W window slots (> 0), R recall slots, A + W + R <= max_slots; all
 * slots start inactive. */
gh_status gh_model_ring_init(gh_model *m, uint32_t num_anchors, uint32_t window_size,
                             uint32_t num_recall);
/* forwardToken's GPU branch (src/model/forward.zig:41-45) with the ring on
 * the device: only x (host) and the clock go up. */
gh_status gh_model_forward_clock(gh_model *m, const float *x, int want_logits, uint64_t clock,
                                 uint32_t *out_token);
/* T prompt tokens at clocks first_clock .. first_clock + T - 1 through the
 * batched prefill, their slots and lists taken from the device ring (as T
 * calls of gh_model_forward_clock would see them).  A call that fails
 * leaves the ring unchanged. */
gh_status gh_model_ring_prefill(gh_model *m, const float *x, uint32_t T, uint64_t first_clock,
                                int want_logits, uint32_t *out_token);
/* GpuEngine.submitPreRecorded (src/gpu/kernels.zig:147-157) on the model's
 * own graphs, as src/model/bench.zig:12-15 calls it with cmd_buf_decode:
 * replays the recorded decode graph (GH_GRAPH_DECODE: layers, LM head and
 * argmax, gated at the model's threshold) or prefill graph (GH_GRAPH_PREFILL)
 * on the inputs the device already holds -- x, the step record and the list
 * of the last forward call -- with no host copy in or out, and waits for it.
 * Before any forward call those inputs are x = 0 at clock 0, slot 0, the
 * one-slot list {0}.  The passes keep the caller's x as sent, so without
 * layer gating a replay recomputes the last forward call's step bit for bit
 * (its K/V row rewritten with the same values); with gating on, a replay
 * also moves each gated layer's previous input, as every pass does.  After
 * gh_model_ring_init a replay records the step's activation in the device
 * ring again. */
typedef enum gh_graph_kind { GH_GRAPH_DECODE = 0, GH_GRAPH_PREFILL = 1 } gh_graph_kind;
gh_status gh_model_submit_prerecorded(gh_model *m, gh_graph_kind which);
/* clearRecall (ring_buffer.zig:82-88) on the device ring. */
gh_status gh_model_ring_clear_recall(gh_model *m);
/* writeRecallKV (ring_buffer.zig:90-99) into the device caches: layer's
 * [kv_dim] key and value rows (host f32) go to recall slot A + W + rank; for
 * layer 0 the slot becomes active with `clock`, the bookkeeping the device
 * path lists every layer by (forward.zig:42-43).  The reference's GPU path
 * activates recall slots without uploading their K/V
 * (src/model/memory_inject.zig:38-45 writes the host ring only); this call
 * uploads both. */
gh_status gh_model_write_recall_kv(gh_model *m, uint32_t layer, uint32_t rank, const float *k,
                                   const float *v, uint64_t clock);

/* Layer gating ("quiescence", the threshold GpuModelContext.init takes,
 * src/gpu/model_gpu.zig:75,182; src/gpu/model_dispatch.zig:45-101,
 * shaders/quiescence_gate.wgsl:16-62).  With threshold != 0 every layer l >=
 * num_layers / 3 of the decode graph first compares its input residual x
 * with the input it saw on the previous call, mean((x - x_prev)^2) over
 * hidden, stores x as x_prev, and runs only when that mean is >= threshold
 * (or threshold <= 0); a gated-off layer is skipped whole -- x passes
 * through, and its K/V row of this token is not written.  The prefill graph
 * (want_logits 0) runs every layer but records x_prev as the reference's
 * prefill graph does (gates at threshold 0); so does gh_model_prefill for
 * every prompt token except a last one with logits, which runs the gated
 * decode graph, as forwardToken sends it (compute_logits,
 * src/model/forward.zig:41-45).  threshold 0 turns gating off.  Resets
 * every x_prev to 0 and records the graphs again. */
gh_status gh_model_set_quiescence(gh_model *m, float threshold);

/* Per-layer residual trace (no reference counterpart; for checking): when
 * enabled, every forward call also copies the residual stream at each
 * layer's input into row l of a [num_layers + 1][hidden] buffer, and with
 * logits the final residual into row num_layers (GH_T_TRACE); a batched
 * prefill does the same for its last token.  Enabling or disabling records
 * the graphs again. */
gh_status gh_model_set_trace(gh_model *m, int enable);

/* Tensor access for checking and cache set-up (no reference counterpart). */
typedef enum gh_tensor {
  GH_T_QKV = 0,        /* layer: [q_dim + kv_dim (+ kv_dim)] quantized rows */
  GH_T_O_PROJ = 1,     /* layer: [hidden] rows over q_dim */
  GH_T_GATE = 2,       /* layer: [intermediate] rows over hidden */
  GH_T_UP = 3,
  GH_T_DOWN = 4,       /* layer: [hidden] rows over intermediate */
  GH_T_INPUT_NORM = 5, /* layer: f32 vectors ... */
  GH_T_Q_NORM = 6,
  GH_T_K_NORM = 7,
  GH_T_POST_ATTN_NORM = 8,
  GH_T_PRE_FFN_NORM = 9,
  GH_T_POST_FFN_NORM = 10,
  GH_T_K_CACHE = 11,   /* layer: f32 [max_slots][kv_dim] */
  GH_T_V_CACHE = 12,
  GH_T_LM_HEAD = 20,   /* global (layer ignored): Q8_0 [vocab] rows over hidden */
  GH_T_FINAL_NORM = 21,
  GH_T_EMBED = 22,     /* synthetic models: bf16 [vocab][hidden] */
  GH_T_LOGITS = 23,    /* f32 [vocab] of the last decode step */
  GH_T_HIDDEN = 24,    /* f32 [hidden]: the final residual of the last call that
                          computed logits (absent after a call without logits) */
  GH_T_STEP = 25,      /* u32 [4]: {clock, slot_idx, S, mode} of the last step */
  GH_T_ACTIVE = 26,    /* u32 [max_slots]: the last step's active list (S entries) */
  GH_T_RING_CLOCKS = 27, /* u32 [max_slots]: device ring clock per slot */
  GH_T_RING_FLAGS = 28,  /* u32 [max_slots]: device ring active flag per slot */
  GH_T_TRACE = 29,     /* f32 [hidden]: trace row `layer` (0 .. num_layers) */
  GH_T_GATE_FLAGS = 30, /* u32 [num_layers]: 1 where the last step ran the layer */
  GH_T_GATE_PREV = 31, /* f32 [num_layers][hidden]: each gated layer's previous input */
  GH_T_PREFILL_TRACE = 32 /* f32 [T][hidden]: with the trace on, layer `layer`'s input
                             rows (0 .. num_layers - 1) of every token of the last
                             batched gh_model_prefill call (or chunk) */
} gh_tensor;
/* Byte size of a tensor (0 when it does not exist). */
size_t gh_model_tensor_bytes(const gh_model *m, int layer, gh_tensor t);
gh_status gh_model_read_tensor(gh_model *m, int layer, gh_tensor t, void *host, size_t bytes);
gh_status gh_model_write_tensor(gh_model *m, int layer, gh_tensor t, const void *host,
                                size_t bytes);

#ifdef __cplusplus
}
#endif
#endif
