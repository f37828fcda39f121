// model.cpp -- the model-level C ABI: GpuModelContext.init/deinit and
// gpuDispatchForwardToken (src/gpu/model_gpu.zig:35-197,
// src/gpu/model_dispatch.zig:103-147) on one MI355X.
//
// HBM layout: one arena holding, per layer, the concatenated [q | k | v]
// rows (one GEMV for the three projections), o, gate, up and down in the
// reference's quant.zig blocks, the norms widened to f32, and the per-layer
// K/V caches [max_slots ring rows + stage_rows prefill staging rows][kv_dim];
// then the Q8_0 LM head, the final
// norm and the activations.  Each forward pass is recorded once as a HIP
// graph of kernels only -- the ring step, then 6 launches a layer (QKV
// stream, attention, attention merge, o stream, gate+up stream, down stream),
// then the LM head and its argmax -- and replayed per token; the host copies
// x (and, on the host-list entry, the step record and the active list) in
// before the replay and the token out after it.
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <cmath>
#include <string>
#include <vector>

#include "../common/attn_args.h"
#include "../common/stream_args.h"
#include "../common/synth.h"
#include "runtime.hpp"

using gh::fail;
using gh::hip_fail;

namespace {

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

struct Layer {
  bool full;
  uint32_t head_dim, rot, nkv, q_dim, kv_dim, qkv_rows;
  bool k_eq_v;
  float theta, scalar;
  size_t qkv, o, gate, up, down;                   // arena offsets (bytes)
  size_t input_norm, q_norm, k_norm, post_attn, pre_ffn, post_ffn;  // SIZE_MAX = absent
  size_t k_cache, v_cache;
};

constexpr size_t kNone = ~(size_t)0;
// Staging rows per K/V cache (at most max_slots): a prefill batch that
// overwrites slots it also attends to stages at most this many tokens per
// chunk.  256 keeps a 640-slot ring's staging at 40% of its ring rows.
constexpr uint32_t kStageRowsMax = 256;
constexpr uint32_t kPfGroup = 4;  // tokens per gh_pf_attn_g_* workgroup (PF_GT in attn.hip)

}  // namespace

struct gh_model {
  gh_context* ctx = nullptr;
  gh_model_config cfg{};
  gh_quant_mode mode = GH_QUANT_Q4;
  std::vector<Layer> layers;
  uint8_t* arena = nullptr;
  size_t arena_bytes = 0;
  size_t lm_head = 0, final_norm = 0;
  // x0 is the caller's x (in the io region); the residual stream runs in x1
  // and x2, so a replay of a recorded graph sees the same x
  size_t x0 = 0, x1 = 0, x2 = 0, qkv_out = 0, attn_out = 0, o_out = 0, act = 0, m_out = 0,
         logits = 0;
  size_t token = 0, step = 0, active = 0, attn_part = 0, amax = 0;
  // The per-token inputs sit in one region, [x0: hidden f32 | step: 4 u32 |
  // active list], so that one host->device copy carries them (x alone and the
  // step record when the device ring computes the list).
  size_t io = 0, io_bytes = 0;
  // device-resident ring bookkeeping (layer 0): clock and active flag per slot
  size_t ring_clock = 0, ring_flag = 0;
  // per-token RoPE tables (cos, sin) of the sliding (0) and full (1) layers
  size_t rope_tab = 0;
  uint32_t rope_rot[2] = {0, 0};
  float rope_theta[2] = {0.f, 0.f};
  uint32_t ring_a = 0, ring_w = 0, ring_r = 0;
  gh_ring* ring = nullptr;  // host mirror of the same state (batched prefill lists)
  uint32_t nsplit = 1, max_q = 0, max_kv = 0;
  uint32_t stage_rows = 0;  // staging rows after the ring rows of each K/V cache
  size_t hidden_decode = 0;      // where the decode graph leaves the final residual
  size_t hidden_final = 0;       // where the last call left it (kNone: not computed)
  uint16_t* embed_dev = nullptr; // synthetic models only
  // pinned host staging of the io region and the token read-back
  uint8_t* h_io = nullptr;
  float* h_x = nullptr;
  uint32_t* h_active = nullptr;
  uint32_t* h_step = nullptr;
  uint32_t* h_token = nullptr;
  void* graph_decode = nullptr;
  void* graph_prefill = nullptr;
  // per-layer residual trace: row l = layer l's input, row L = the final residual
  float* trace = nullptr;
  bool trace_on = false;
  // the batched prefill's trace: [L][T][hidden], layer l's input rows of
  // every token of the last traced batch (pf_trace_T tokens)
  float* pf_trace = nullptr;
  uint32_t pf_trace_cap = 0, pf_trace_T = 0;
  // GH_EAGER_DECODE=1 (read at init): each token launches its kernels
  // directly instead of replaying the recorded graph (for kernel tracing).
  bool eager = false;
  // GH_QGATE_KERNEL=1 (read at init): gated layers start with the separate
  // gh_qgate_k launch instead of gating in their QKV stream's prologue
  bool qgate_kernel = false;
  // A prompt of at most this many tokens runs token by token through the
  // decode graphs: at the 12B shape in Q4, 1-2 tokens take 2.6 / 5.1 ms that
  // way against 5.8 / 6.0 ms for one batched call (whose projections stream
  // the weights once for all tokens), and 3 tokens 7.5 against 6.1.  Q8 and
  // bf16 decode steps take 3.7 and 5.0 ms, and one batched call 6.9 and
  // 8.3 ms, so there only a single token runs that way.  Set at init from the
  // weight mode; GH_PF_SEQ_MAX (read at init) overrides it, and 0 sends every
  // prompt to the batched kernels.
  uint32_t seq_prefill_max = 2;
  // layer gating (quiescence): layers >= num_layers / 3 are gated when on
  bool q_on = false;
  float q_thr = 0.f;
  size_t xprev = 0, gate_flags = 0;  // [L][hidden] f32 previous layer inputs, [L] u32 ran flags
  // batched prefill buffers (gh_model_prefill), sized for pf_cap tokens
  uint32_t pf_cap = 0, pf_stride = 0;
  uint8_t* pf_arena = nullptr;
  float *pf_x = nullptr, *pf_qkv = nullptr, *pf_o = nullptr, *pf_m = nullptr;
  float *pf_xn = nullptr, *pf_attn = nullptr, *pf_act = nullptr;
  float* pf_rs = nullptr;  // row scales of the normed rows (pf_xn holds their fp16 hi/lo planes)
  uint32_t *pf_meta = nullptr, *pf_active = nullptr;
  // grouped prefill attention: per group of pf_gtok consecutive tokens, the
  // union of their active lists as (slot, token mask) pairs, and its length
  uint32_t *pf_union = nullptr, *pf_ucount = nullptr, *pf_scatter = nullptr;
  uint32_t pf_ustride = 0, pf_gtok = 0;
  uint32_t pf_gkind = 0;  // this call: 0 per-token kernel, 1 gh_pf_attn_g_*, 2 gh_pf_attn_m_k
  uint32_t pf_maxn = 0;   // this call: the longest active list of a token

  template <typename T>
  T* at(size_t off) const {
    return reinterpret_cast<T*>(arena + off);
  }
  size_t row_bytes(uint32_t cols) const {
    return (size_t)(cols / 32) * (mode == GH_QUANT_Q8 ? 36 : mode == GH_QUANT_Q4 ? 20 : 64);
  }
  // the tied head: bf16 rows in mode none, else Q8_0 (src/gpu/model_gpu.zig:160-161)
  size_t head_bytes() const {
    return (size_t)cfg.vocab_size * (cfg.hidden_size / 32) * (mode == GH_QUANT_NONE ? 64 : 36);
  }
  ~gh_model();
};

namespace {
gh_status ensure_prefill(gh_model* m, uint32_t T, uint32_t stride);
gh_status reset_gates(gh_model* m);
gh_status prefill_forward(gh_model* m, uint32_t T, bool want_logits);
}  // namespace

gh_model::~gh_model() {
  if (ctx && ctx->stream) hipStreamSynchronize(ctx->stream);
  if (graph_decode) gh_graph_destroy(graph_decode);
  if (graph_prefill) gh_graph_destroy(graph_prefill);
  if (arena) hipFree(arena);
  if (pf_arena) hipFree(pf_arena);
  if (embed_dev) hipFree(embed_dev);
  if (trace) hipFree(trace);
  if (pf_trace) hipFree(pf_trace);
  if (h_io) hipHostFree(h_io);
  if (h_token) hipHostFree(h_token);
  if (ring) gh_ring_destroy(ring);
}

namespace {

gh_status validate(const gh_context* ctx, const gh_model_config& c, gh_quant_mode mode) {
  if (mode != GH_QUANT_Q4 && mode != GH_QUANT_Q8 && mode != GH_QUANT_NONE)
    return fail(GH_ERR_UNSUPPORTED, "model: mode must be Q4, Q8 or NONE (bf16)");
  if (c.num_hidden_layers == 0 || c.num_hidden_layers > 64)
    return fail(GH_ERR_INVALID, "model: num_hidden_layers must be 1..64");
  if (c.hidden_size == 0 || c.hidden_size % 128 || c.intermediate_size == 0 ||
      c.intermediate_size % 128 || c.vocab_size == 0)
    return fail(GH_ERR_UNSUPPORTED, "model: hidden and intermediate sizes must be multiples of 128");
  if (c.num_attention_heads == 0 || c.num_key_value_heads == 0 || c.max_slots == 0)
    return fail(GH_ERR_INVALID, "model: head counts and max_slots must be positive");
  (void)ctx;
  return GH_OK;
}

// src/model/loader.zig:36-42
Layer layer_shape(const gh_model_config& c, uint32_t l) {
  Layer L{};
  L.full = c.layer_types[l] != 0;
  L.head_dim = L.full ? c.global_head_dim : c.head_dim;
  L.rot = L.full ? L.head_dim / 4 : L.head_dim;
  L.nkv = L.full ? c.num_global_key_value_heads : c.num_key_value_heads;
  L.q_dim = c.num_attention_heads * L.head_dim;
  L.kv_dim = L.nkv * L.head_dim;
  L.k_eq_v = L.full && c.attention_k_eq_v;
  L.theta = L.full ? c.rope_theta_full : c.rope_theta;
  L.scalar = 1.0f;
  return L;
}

gh_status plan(gh_model* m) {
  const gh_model_config& c = m->cfg;
  const uint32_t H = c.hidden_size, I = c.intermediate_size, V = c.vocab_size;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    size_t o = off;
    off = align_up(off + bytes, 256);
    return o;
  };
  m->layers.clear();
  m->stage_rows = std::min(c.max_slots, kStageRowsMax);
  for (uint32_t l = 0; l < c.num_hidden_layers; l++) {
    Layer L = layer_shape(c, l);
    if (L.nkv == 0 || c.num_attention_heads % L.nkv || c.num_attention_heads / L.nkv > 4)
      return fail(GH_ERR_UNSUPPORTED, "model: query heads per kv head must be 1..4");
    if (L.head_dim % 4 || L.head_dim > 512 || L.q_dim % 128 || L.rot % 2)
      return fail(GH_ERR_UNSUPPORTED, "model: head_dim must be a multiple of 4 up to 512 with "
                                      "num_heads * head_dim a multiple of 128");
    L.qkv_rows = L.q_dim + L.kv_dim * (L.k_eq_v ? 1 : 2);
    L.qkv = take((size_t)L.qkv_rows * m->row_bytes(H));
    L.o = take((size_t)H * m->row_bytes(L.q_dim));
    L.gate = take((size_t)I * m->row_bytes(H));
    L.up = take((size_t)I * m->row_bytes(H));
    L.down = take((size_t)H * m->row_bytes(I));
    L.input_norm = take(H * 4);
    L.q_norm = take(L.head_dim * 4);
    L.k_norm = take(L.head_dim * 4);
    L.post_attn = take(H * 4);
    L.pre_ffn = take(H * 4);
    L.post_ffn = take(H * 4);
    // max_slots ring rows, then stage_rows staging rows for a prefill batch
    // whose tokens overwrite slots that earlier tokens of the batch attend to
    L.k_cache = take((size_t)(c.max_slots + m->stage_rows) * L.kv_dim * 4);
    L.v_cache = take((size_t)(c.max_slots + m->stage_rows) * L.kv_dim * 4);
    m->max_q = std::max(m->max_q, L.q_dim);
    m->max_kv = std::max(m->max_kv, L.kv_dim);
    m->layers.push_back(L);
  }
  m->lm_head = take(m->head_bytes());
  m->final_norm = take(H * 4);
  m->io_bytes = align_up((size_t)H * 4, 256) + 64 + (size_t)c.max_slots * 4;
  m->io = take(m->io_bytes);
  m->x0 = m->io;
  m->step = m->io + align_up((size_t)H * 4, 256);
  m->active = m->step + 64;
  m->x1 = take(H * 4);
  m->x2 = take(H * 4);
  m->ring_clock = take((size_t)c.max_slots * 4);
  m->ring_flag = take((size_t)c.max_slots * 4);
  m->rope_tab = take(2 * 2 * 256 * 4);
  m->xprev = take((size_t)c.num_hidden_layers * H * 4);
  m->gate_flags = take((size_t)c.num_hidden_layers * 4);
  for (auto& L : m->layers) {
    m->rope_rot[L.full ? 1 : 0] = L.rot;
    m->rope_theta[L.full ? 1 : 0] = L.theta;
  }
  uint32_t max_qkv = 0;
  for (auto& L : m->layers) max_qkv = std::max(max_qkv, L.qkv_rows);
  m->qkv_out = take((size_t)max_qkv * 4);
  m->attn_out = take((size_t)m->max_q * 4);
  m->o_out = take(H * 4);
  m->act = take(I * 4);
  m->m_out = take(H * 4);
  m->logits = take((size_t)V * 4);
  m->token = take(64);
  uint32_t max_nkv = 0, max_g = 1, max_d = 0;
  for (auto& L : m->layers) {
    max_nkv = std::max(max_nkv, L.nkv);
    max_g = std::max(max_g, c.num_attention_heads / L.nkv);
    max_d = std::max(max_d, L.head_dim);
  }
  m->nsplit = gh::attention_splits(m->ctx, max_nkv, c.max_slots);
  m->attn_part = take((size_t)max_nkv * m->nsplit * max_g * (max_d + 4) * 4);
  m->amax = take(2 * 4096 * 4);  // LM-head argmax partials: 2 words per workgroup
  m->arena_bytes = off;
  return GH_OK;
}

gh_status alloc_all(gh_model* m) {
  hipError_t e = hipMalloc(&m->arena, m->arena_bytes);
  if (e != hipSuccess)
    return fail(GH_ERR_ALLOC, "model arena (" + std::to_string(m->arena_bytes >> 20) +
                                  " MiB): " + hipGetErrorString(e));
  e = hipHostMalloc(&m->h_io, m->io_bytes);
  if (e == hipSuccess) e = hipHostMalloc(&m->h_token, 64);
  if (e != hipSuccess) return fail(GH_ERR_ALLOC, std::string("pinned staging: ") + hipGetErrorString(e));
  memset(m->h_io, 0, m->io_bytes);
  memset(m->h_token, 0, 64);
  m->h_x = reinterpret_cast<float*>(m->h_io);
  m->h_step = reinterpret_cast<uint32_t*>(m->h_io + (m->step - m->io));
  m->h_active = reinterpret_cast<uint32_t*>(m->h_io + (m->active - m->io));
  // caches, activations and scratch start at zero (counters must)
  uint64_t words = m->arena_bytes / 4;
  uint32_t zero = 0;
  void* p = m->arena;
  void* args[] = {&p, &zero, &words};
  gh_status st = m->ctx->launch("gh_fill_u32_k", dim3(8192), dim3(256), 0, args);
  if (st != GH_OK) return st;
  // the inputs a replay before any forward call sees: x = 0 at clock 0,
  // slot 0, the one-slot list {0} (dense)
  m->h_step[2] = 1;
  m->h_step[3] = 2;
  e = hipMemcpyAsync(m->arena + m->step, m->h_step, 16, hipMemcpyHostToDevice, m->ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(m->ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "arena zero-fill");
  return GH_OK;
}

// Quantize [rows][cols] bf16 into dst, with the bf16 rows provided chunk by
// chunk by fill(staging, row0, nrows) (an upload or the device generator).
// Mode none keeps the bf16 rows: fill writes them in place.
template <typename Fill>
gh_status quantize_rows(gh_model* m, uint8_t* dst, uint32_t rows, uint32_t cols, gh_quant_mode q,
                        uint16_t* staging, size_t staging_elems, Fill fill) {
  if (q == GH_QUANT_NONE) return fill(reinterpret_cast<uint16_t*>(dst), 0, rows);
  const uint32_t chunk = (uint32_t)std::max<size_t>(1, staging_elems / cols);
  const size_t rb = (size_t)(cols / 32) * (q == GH_QUANT_Q8 ? 36 : 20);
  for (uint32_t r0 = 0; r0 < rows; r0 += chunk) {
    const uint32_t n = std::min(chunk, rows - r0);
    gh_status st = fill(staging, r0, n);
    if (st != GH_OK) return st;
    st = gh_quantize_matrix_dev(m->ctx, dst + (size_t)r0 * rb, staging, n, cols, q);
    if (st != GH_OK) return st;
  }
  return GH_OK;
}

gh_status upload_norm(gh_model* m, size_t off, const uint16_t* bf16, uint32_t n) {
  std::vector<float> f(n, 1.0f);  // absent weight = ones (model_gpu.zig:64-73)
  if (bf16)
    for (uint32_t i = 0; i < n; i++) {
      uint32_t u = (uint32_t)bf16[i] << 16;
      memcpy(&f[i], &u, 4);
    }
  return gh_buffer_write(m->ctx, m->arena + off, f.data(), (size_t)n * 4);
}

XPro pro_plain(const float* x) {
  XPro p{};
  p.x = x;
  p.mode = 0;
  return p;
}

// dst[0..n) = src[0..n) (u32 words) on the context stream.
gh_status copy_words(gh_model* m, void* dst, const void* src, uint64_t n) {
  void* args[] = {&dst, const_cast<void**>(&src), &n};
  const unsigned grid = (unsigned)std::min<uint64_t>((n + 255) / 256, 64);
  return m->ctx->launch("gh_copy_u32_k", dim3(grid), dim3(256), 0, args);
}

// Records one forward pass (all layers; with the LM head when logits).  The
// graph holds kernels only: the caller copies the io region in before the
// replay and the token out after it.
gh_status record_forward(gh_model* m, bool logits, float thr) {
  gh_context* ctx = m->ctx;
  const gh_model_config& c = m->cfg;
  const uint32_t H = c.hidden_size, I = c.intermediate_size;
  const char* gemv = gh::gemv_family(m->mode);
  const char* gateup = gh::gateup_family(m->mode);
  const bool head_bf16 = m->mode == GH_QUANT_NONE;
  gh_status st;
  {  // device ring: slot_idx, S and the active list from the clock (step mode 1)
    uint32_t* rc = m->at<uint32_t>(m->ring_clock);
    uint32_t* rf = m->at<uint32_t>(m->ring_flag);
    uint32_t* sp = m->at<uint32_t>(m->step);
    uint32_t* al = m->at<uint32_t>(m->active);
    uint32_t A = m->ring_a, W = std::max(1u, m->ring_w), R = m->ring_r;
    float* tab = m->at<float>(m->rope_tab);
    void* args[] = {&rc, &rf, &sp, &al, &A, &W, &R, &tab, &m->rope_rot[0], &m->rope_theta[0],
                    &m->rope_rot[1], &m->rope_theta[1]};
    if ((st = ctx->launch("gh_ring_step_k", dim3(1), dim3(1024), 0, args)) != GH_OK) return st;
  }
  if (m->trace_on && (st = copy_words(m, m->trace, m->at<float>(m->x0), H)) != GH_OK) return st;

  size_t xcur = m->x0, xoth = m->x1;
  // Gated layers (quiescence on, layers >= L / 3; src/gpu/model_dispatch.zig:
  // 45-101): their input lives in buffer A and their mid-layer residual in B.
  // gh_qgate_k before each such layer finishes the previous layer's post-FFN
  // add into A (when that layer ran), gates, and sets the layer's run flag;
  // every kernel of the layer then returns at once when the flag is 0.
  const uint32_t dense_limit = m->q_on ? c.num_hidden_layers / 3 : c.num_hidden_layers;
  const uint32_t* flags = m->at<uint32_t>(m->gate_flags);
  size_t bufA = 0, bufB = 0;
  for (uint32_t l = 0; l < c.num_hidden_layers; l++) {
    const Layer& L = m->layers[l];
    const bool gated = l >= dense_limit;
    const uint32_t* run = gated ? flags + l : nullptr;
    XPro gp{};  // mode 4: the gate in the QKV prologue
    if (gated) {
      uint32_t prev_mode;
      const Layer* P = l > 0 ? &m->layers[l - 1] : nullptr;
      if (l == dense_limit) {  // the first gated layer
        if (l == 0) {
          bufA = m->x0;
          bufB = m->x1;
          prev_mode = 0;  // the embedding, as it stands
        } else {
          bufB = xcur;  // the previous (ungated) layer's mid-layer residual
          bufA = xoth;
          prev_mode = 1;
        }
      } else {
        prev_mode = 2;
      }
      float* xmid = m->at<float>(bufB);
      float* mo = m->at<float>(m->m_out);
      const float* wpost = P && P->post_ffn != kNone ? m->at<float>(P->post_ffn) : nullptr;
      float sc = P ? P->scalar : 1.0f;
      const uint32_t* prun = l > 0 ? flags + l - 1 : nullptr;
      float* A = m->at<float>(bufA);
      float* xp = m->at<float>(m->xprev) + (size_t)l * H;
      uint32_t* ro = const_cast<uint32_t*>(flags) + l;
      if (m->qgate_kernel) {
        uint32_t Hh = H, one = 1;
        float eps = c.rms_norm_eps, th = thr;
        void* args[] = {&xmid, &mo, const_cast<float**>(&wpost), &sc, &prev_mode,
                        const_cast<uint32_t**>(&prun), &A, &xp, &th, &ro, &Hh, &eps, &one};
        if ((st = ctx->launch("gh_qgate_k", dim3(1), dim3(1024), 0, args)) != GH_OK) return st;
        if (m->trace_on && (st = copy_words(m, m->trace + (size_t)l * H, A, H)) != GH_OK)
          return st;
      } else {  // the gate runs in the QKV stream's prologue (mode 4)
        gp.x = xmid;
        gp.r = mo;
        gp.wr = wpost;
        gp.s = sc;
        gp.xa = A;
        gp.xout = A;
        gp.xprev = xp;
        gp.prun = prun;
        gp.run_out = ro;
        gp.pmode = prev_mode;
        gp.thr = thr;
        gp.mode = 4;
      }
    }
    // 1. [q|k|v] = W_qkv . norm(x)  (layer 0: RMSNorm; later: post-FFN add + norm)
    XPro p{};
    p.eps = c.rms_norm_eps;
    p.w = m->at<float>(L.input_norm);
    if (gated && gp.mode == 4) {
      p = gp;
      p.eps = c.rms_norm_eps;
      p.w = m->at<float>(L.input_norm);
    } else if (gated) {
      p.x = m->at<float>(bufA);
      p.mode = 1;
    } else if (l == 0) {
      p.x = m->at<float>(xcur);
      p.mode = 1;
    } else {
      const Layer& P = m->layers[l - 1];
      p.x = m->at<float>(xcur);
      p.r = m->at<float>(m->m_out);
      p.wr = P.post_ffn == kNone ? nullptr : m->at<float>(P.post_ffn);
      p.s = P.scalar;
      p.xout = m->at<float>(xoth);
      p.mode = 2;
      std::swap(xcur, xoth);
    }
    Q4Args qa{m->at<uint8_t>(L.qkv), m->at<float>(m->qkv_out)};
    if ((st = gh::launch_stream(ctx, gemv, &qa, p, L.qkv_rows, H, p.mode == 4 ? nullptr : run)) !=
        GH_OK)
      return st;
    if (m->trace_on && p.mode == 4 &&
        (st = copy_words(m, m->trace + (size_t)l * H, m->at<float>(bufA), H)) != GH_OK)
      return st;
    if (m->trace_on && l > 0 && !gated &&
        (st = copy_words(m, m->trace + (size_t)l * H, m->at<float>(xcur), H)) != GH_OK)
      return st;
    // 2. q/k norm + RoPE + cache write + split-K attention
    gh::AttnLaunch A{};
    AttnArgs& a = A.args;
    const float* qkv = m->at<float>(m->qkv_out);
    a.q = qkv;
    a.k_in = qkv + L.q_dim;
    a.v_in = L.k_eq_v ? qkv + L.q_dim : qkv + L.q_dim + L.kv_dim;
    a.q_norm = m->at<float>(L.q_norm);
    a.k_norm = m->at<float>(L.k_norm);
    a.k_cache = m->at<float>(L.k_cache);
    a.v_cache = m->at<float>(L.v_cache);
    a.active = m->at<uint32_t>(m->active);
    a.step = m->at<uint32_t>(m->step);
    a.flags = m->at<uint32_t>(m->step) + 3;
    a.rope_tab = m->at<float>(m->rope_tab) + (L.full ? 2 * 256 : 0);
    a.part = m->at<float>(m->attn_part);
    a.out = m->at<float>(m->attn_out);
    a.nq = c.num_attention_heads;
    a.nkv = L.nkv;
    a.D = L.head_dim;
    a.rot = L.rot;
    a.k_eq_v = L.k_eq_v ? 1 : 0;
    a.nsplit = m->nsplit;
    a.fuse = 1;
    a.theta = L.theta;
    a.eps = c.rms_norm_eps;
    a.scale = 1.0f;  // inv_sqrt_dim = 1.0 (src/model/forward.zig:80)
    a.run = run;
    if ((st = gh::launch_attention(ctx, A)) != GH_OK) return st;
    // 3. o = W_o . attn
    Q4Args oa{m->at<uint8_t>(L.o), m->at<float>(m->o_out)};
    if ((st = gh::launch_stream(ctx, gemv, &oa, pro_plain(m->at<float>(m->attn_out)), H,
                                L.q_dim, run)) != GH_OK)
      return st;
    // 4. x += post_attn_norm(o); act = geglu(W_gate, W_up . pre_ffn_norm(x))
    XPro g{};
    g.x = m->at<float>(gated ? bufA : xcur);
    g.r = m->at<float>(m->o_out);
    g.wr = L.post_attn == kNone ? nullptr : m->at<float>(L.post_attn);
    g.w = m->at<float>(L.pre_ffn);
    g.xout = m->at<float>(gated ? bufB : xoth);
    g.s = 1.0f;
    g.eps = c.rms_norm_eps;
    g.mode = 2;
    if (!gated) {
      std::swap(xcur, xoth);
      if (xoth == m->x0) xoth = m->x2;  // the caller's x stays as sent
    }
    GateUpArgs ga{m->at<uint8_t>(L.gate), m->at<uint8_t>(L.up), m->at<float>(m->act)};
    if ((st = gh::launch_stream(ctx, gateup, &ga, g, I, H, run)) != GH_OK) return st;
    // 5. m = W_down . act
    Q4Args da{m->at<uint8_t>(L.down), m->at<float>(m->m_out)};
    if ((st = gh::launch_stream(ctx, gemv, &da, pro_plain(m->at<float>(m->act)), H, I, run)) !=
        GH_OK)
      return st;
  }
  if (logits && dense_limit < c.num_hidden_layers) {
    // gated tail: the last layer's post-FFN add (when it ran) into A, then
    // token = argmax(head . final_norm(A))
    const Layer& P = m->layers.back();
    float* xmid = m->at<float>(bufB);
    float* mo = m->at<float>(m->m_out);
    const float* wpost = P.post_ffn != kNone ? m->at<float>(P.post_ffn) : nullptr;
    float sc = P.scalar;
    uint32_t prev_mode = 2, Hh = H, zero = 0;
    const uint32_t* prun = flags + c.num_hidden_layers - 1;
    float* Ab = m->at<float>(bufA);
    float* xp = m->at<float>(m->xprev);
    uint32_t* ro = m->at<uint32_t>(m->gate_flags);
    float eps = c.rms_norm_eps, th = 0.f;
    void* args[] = {&xmid, &mo, const_cast<float**>(&wpost), &sc, &prev_mode,
                    const_cast<uint32_t**>(&prun), &Ab, &xp, &th, &ro, &Hh, &eps, &zero};
    if ((st = ctx->launch("gh_qgate_k", dim3(1), dim3(1024), 0, args)) != GH_OK) return st;
    XPro p{};
    p.x = Ab;
    p.w = m->at<float>(m->final_norm);
    p.eps = c.rms_norm_eps;
    p.mode = 1;
    m->hidden_decode = bufA;
    ArgmaxArgs aa{m->at<uint8_t>(m->lm_head), m->at<float>(m->logits), m->at<uint32_t>(m->amax)};
    if ((st = gh::launch_argmax_stream(ctx, &aa, p, c.vocab_size, H, m->at<uint32_t>(m->token),
                                       head_bf16)) != GH_OK)
      return st;
    if (m->trace_on &&
        (st = copy_words(m, m->trace + (size_t)c.num_hidden_layers * H, Ab, H)) != GH_OK)
      return st;
  } else if (logits) {
    // x = (x + post_ffn_norm(m)) * layer_scalar; token = argmax(head . final_norm(x))
    const Layer& P = m->layers.back();
    XPro p{};
    p.x = m->at<float>(xcur);
    p.r = m->at<float>(m->m_out);
    p.wr = P.post_ffn == kNone ? nullptr : m->at<float>(P.post_ffn);
    p.w = m->at<float>(m->final_norm);
    p.xout = m->at<float>(xoth);
    p.s = P.scalar;
    p.eps = c.rms_norm_eps;
    p.mode = 2;
    m->hidden_decode = xoth;
    ArgmaxArgs aa{m->at<uint8_t>(m->lm_head), m->at<float>(m->logits), m->at<uint32_t>(m->amax)};
    if ((st = gh::launch_argmax_stream(ctx, &aa, p, c.vocab_size, H, m->at<uint32_t>(m->token),
                                       head_bf16)) != GH_OK)
      return st;
    if (m->trace_on &&
        (st = copy_words(m, m->trace + (size_t)c.num_hidden_layers * H, m->at<float>(xoth), H)) !=
            GH_OK)
      return st;
  }
  return GH_OK;
}

gh_status record_graphs(gh_model* m) {
  for (int pass = 0; pass < 2; pass++) {
    gh_status st = gh_graph_begin(m->ctx);
    if (st != GH_OK) return st;
    gh_status rs = record_forward(m, pass == 0, pass == 0 ? m->q_thr : 0.0f);
    void* g = nullptr;
    st = gh_graph_end(m->ctx, &g);
    if (rs != GH_OK) {
      if (g) gh_graph_destroy(g);
      return rs;
    }
    if (st != GH_OK) return st;
    (pass == 0 ? m->graph_decode : m->graph_prefill) = g;
  }
  return GH_OK;
}

gh_status finish_init(gh_model* m, gh_model** out) {
  const char* eager = getenv("GH_EAGER_DECODE");
  m->eager = eager && eager[0] == '1';
  const char* qk = getenv("GH_QGATE_KERNEL");
  m->qgate_kernel = qk && qk[0] == '1';
  m->seq_prefill_max = m->mode == GH_QUANT_Q4 ? 2u : 1u;
  if (const char* sq = getenv("GH_PF_SEQ_MAX")) m->seq_prefill_max = (uint32_t)strtoul(sq, nullptr, 10);
  gh_status st = reset_gates(m);
  if (st == GH_OK) st = record_graphs(m);
  if (st != GH_OK) {
    delete m;
    return st;
  }
  hipError_t e = hipStreamSynchronize(m->ctx->stream);
  if (e != hipSuccess) {
    delete m;
    return hip_fail(e, "model init");
  }
  *out = m;
  return GH_OK;
}

// Gate state: every layer's ran flag 1, every previous layer input 0 (the
// reference's freshly created x_prev buffers).
gh_status reset_gates(gh_model* m) {
  const gh_model_config& c = m->cfg;
  gh_status st = gh_buffer_fill_u32(m->ctx, m->arena + m->gate_flags, 1u, c.num_hidden_layers);
  if (st == GH_OK)
    st = gh_buffer_fill_u32(m->ctx, m->arena + m->xprev, 0u,
                            (size_t)c.num_hidden_layers * c.hidden_size);
  return st;
}

// Sends the host mirror's layer-0 ring state to the device arrays the ring
// kernel reads.
gh_status ring_upload(gh_model* m) {
  const uint32_t n = m->cfg.max_slots;
  std::vector<uint32_t> st(2 * (size_t)n, 0u);
  if (m->ring) gh::ring_state(m->ring, 0, st.data(), st.data() + n, n);
  gh_status s = gh_buffer_write(m->ctx, m->at<uint32_t>(m->ring_clock), st.data(), (size_t)n * 4);
  if (s == GH_OK) s = gh_buffer_write(m->ctx, m->at<uint32_t>(m->ring_flag), st.data() + n, (size_t)n * 4);
  return s;
}

gh_status rerecord(gh_model* m) {
  hipStreamSynchronize(m->ctx->stream);
  if (m->graph_decode) gh_graph_destroy(m->graph_decode);
  if (m->graph_prefill) gh_graph_destroy(m->graph_prefill);
  m->graph_decode = m->graph_prefill = nullptr;
  return record_graphs(m);
}

// One token: the first `bytes` of the io region go up (none for bytes 0),
// the graph replays, and with logits the token comes back.  The decode graph
// gates at the threshold, the prefill graph at 0 (src/gpu/model_gpu.zig:
// 182-183).
gh_status run_token(gh_model* m, bool want_logits, size_t bytes, uint32_t* out_token) {
  hipStream_t s = m->ctx->stream;
  hipError_t e = bytes ? hipMemcpyAsync(m->arena + m->io, m->h_io, bytes, hipMemcpyHostToDevice, s)
                       : hipSuccess;
  if (e != hipSuccess) return hip_fail(e, "forward: input copy");
  gh_status st = m->eager ? record_forward(m, want_logits, want_logits ? m->q_thr : 0.0f)
                          : gh_graph_launch(m->ctx, want_logits ? m->graph_decode : m->graph_prefill);
  if (st != GH_OK) return st;
  if (want_logits) {
    e = hipMemcpyAsync(m->h_token, m->at<uint32_t>(m->token), 4, hipMemcpyDeviceToHost, s);
    if (e != hipSuccess) return hip_fail(e, "forward: token copy");
  }
  e = hipStreamSynchronize(s);
  if (e != hipSuccess) return hip_fail(e, "forward");
  m->hidden_final = want_logits ? m->hidden_decode : kNone;
  if (want_logits) *out_token = m->h_token[0];
  return GH_OK;
}

}  // namespace

extern "C" {

gh_status gh_model_init(gh_context* ctx, const gh_model_config* cfg,
                        const gh_layer_weights* layers, const uint16_t* embed_tokens,
                        const uint16_t* final_norm, gh_quant_mode mode, float quiescence_thresh,
                        gh_model** out) {
  if (!ctx || !cfg || !layers || !embed_tokens || !out)
    return fail(GH_ERR_INVALID, "gh_model_init: null argument");
  *out = nullptr;
  gh_status st = validate(ctx, *cfg, mode);
  if (st != GH_OK) return st;
  gh_model* m = new gh_model();
  m->ctx = ctx;
  m->cfg = *cfg;
  m->mode = mode;
  if ((st = plan(m)) != GH_OK || (st = alloc_all(m)) != GH_OK) {
    delete m;
    return st;
  }
  const uint32_t H = cfg->hidden_size, I = cfg->intermediate_size;
  const size_t staging_elems = 32u << 20;  // 64 MiB of bf16 per chunk
  uint16_t* staging = nullptr;
  if (hipMalloc(&staging, staging_elems * 2) != hipSuccess) {
    delete m;
    return fail(GH_ERR_ALLOC, "gh_model_init: staging");
  }
  auto upload_from = [&](const uint16_t* src, uint32_t cols) {
    return [=](uint16_t* stg, uint32_t r0, uint32_t n) {
      return gh_buffer_write(ctx, stg, src + (size_t)r0 * cols, (size_t)n * cols * 2);
    };
  };
  for (uint32_t l = 0; l < cfg->num_hidden_layers && st == GH_OK; l++) {
    Layer& L = m->layers[l];
    const gh_layer_weights& w = layers[l];
    if (!w.q_proj || !w.k_proj || !w.o_proj || !w.gate_proj || !w.up_proj || !w.down_proj ||
        !w.input_layernorm || !w.q_norm || !w.pre_feedforward_layernorm) {
      st = fail(GH_ERR_INVALID, "gh_model_init: layer " + std::to_string(l) + " misses a tensor");
      break;
    }
    if (!w.v_proj && !L.k_eq_v) {  // v_proj absent: the key projection serves as value
      L.k_eq_v = true;
      L.qkv_rows = L.q_dim + L.kv_dim;
    }
    L.scalar = w.layer_scalar;
    const size_t rb = m->row_bytes(H);
    uint8_t* qkv = m->at<uint8_t>(L.qkv);
    st = quantize_rows(m, qkv, L.q_dim, H, mode, staging, staging_elems, upload_from(w.q_proj, H));
    if (st == GH_OK)
      st = quantize_rows(m, qkv + (size_t)L.q_dim * rb, L.kv_dim, H, mode, staging, staging_elems,
                         upload_from(w.k_proj, H));
    if (st == GH_OK && !L.k_eq_v)
      st = quantize_rows(m, qkv + (size_t)(L.q_dim + L.kv_dim) * rb, L.kv_dim, H, mode, staging,
                         staging_elems, upload_from(w.v_proj, H));
    if (st == GH_OK)
      st = quantize_rows(m, m->at<uint8_t>(L.o), H, L.q_dim, mode, staging, staging_elems,
                         upload_from(w.o_proj, L.q_dim));
    if (st == GH_OK)
      st = quantize_rows(m, m->at<uint8_t>(L.gate), I, H, mode, staging, staging_elems,
                         upload_from(w.gate_proj, H));
    if (st == GH_OK)
      st = quantize_rows(m, m->at<uint8_t>(L.up), I, H, mode, staging, staging_elems,
                         upload_from(w.up_proj, H));
    if (st == GH_OK)
      st = quantize_rows(m, m->at<uint8_t>(L.down), H, I, mode, staging, staging_elems,
                         upload_from(w.down_proj, I));
    if (st == GH_OK) st = upload_norm(m, L.input_norm, w.input_layernorm, H);
    if (st == GH_OK) st = upload_norm(m, L.q_norm, w.q_norm, L.head_dim);
    if (st == GH_OK) st = upload_norm(m, L.k_norm, w.k_norm, L.head_dim);
    if (st == GH_OK) st = upload_norm(m, L.pre_ffn, w.pre_feedforward_layernorm, H);
    if (w.post_attention_layernorm) {
      if (st == GH_OK) st = upload_norm(m, L.post_attn, w.post_attention_layernorm, H);
    } else {
      L.post_attn = kNone;
    }
    if (w.post_feedforward_layernorm) {
      if (st == GH_OK) st = upload_norm(m, L.post_ffn, w.post_feedforward_layernorm, H);
    } else {
      L.post_ffn = kNone;
    }
  }
  if (st == GH_OK)
    st = quantize_rows(m, m->at<uint8_t>(m->lm_head), cfg->vocab_size, H,
                       mode == GH_QUANT_NONE ? GH_QUANT_NONE : GH_QUANT_Q8, staging, staging_elems,
                       upload_from(embed_tokens, H));
  if (st == GH_OK) st = upload_norm(m, m->final_norm, final_norm, H);
  hipStreamSynchronize(ctx->stream);
  hipFree(staging);
  if (st != GH_OK) {
    delete m;
    return st;
  }
  // GpuModelContext.init records the decode graph with the threshold
  // (src/gpu/model_gpu.zig:182); 0 records it ungated
  m->q_on = quiescence_thresh != 0.0f;
  m->q_thr = quiescence_thresh;
  return finish_init(m, out);
}

gh_status gh_model_init_synthetic(gh_context* ctx, const gh_model_config* cfg, gh_quant_mode mode,
                                  uint64_t seed, gh_model** out) {
  if (!ctx || !cfg || !out) return fail(GH_ERR_INVALID, "gh_model_init_synthetic: null argument");
  *out = nullptr;
  gh_status st = validate(ctx, *cfg, mode);
  if (st != GH_OK) return st;
  gh_model* m = new gh_model();
  m->ctx = ctx;
  m->cfg = *cfg;
  m->mode = mode;
  if ((st = plan(m)) != GH_OK || (st = alloc_all(m)) != GH_OK) {
    delete m;
    return st;
  }
  const uint32_t H = cfg->hidden_size, I = cfg->intermediate_size, V = cfg->vocab_size;
  const size_t staging_elems = 32u << 20;
  uint16_t* staging = nullptr;
  if (hipMalloc(&staging, staging_elems * 2) != hipSuccess ||
      hipMalloc(&m->embed_dev, (size_t)V * H * 2) != hipSuccess) {
    if (staging) hipFree(staging);
    delete m;
    return fail(GH_ERR_ALLOC, "gh_model_init_synthetic: staging / embedding");
  }
  // tensor t of layer l draws from stream 1000 + 16 l + t
  auto gen = [&](uint64_t stream, uint32_t cols) {
    return [=](uint16_t* stg, uint32_t r0, uint32_t n) {
      return gh_synth_normal_bf16_dev(ctx, stg, (size_t)n * cols, seed, stream, 0.0, 0.02,
                                      (uint64_t)r0 * cols);
    };
  };
  auto norm = [&](size_t off, uint32_t n, uint64_t stream) {
    std::vector<uint16_t> b(n);
    gh_synth_normal_bf16(b.data(), n, seed, stream, 1.0, 0.1, 0);
    return upload_norm(m, off, b.data(), n);
  };
  for (uint32_t l = 0; l < cfg->num_hidden_layers && st == GH_OK; l++) {
    Layer& L = m->layers[l];
    const uint64_t s0 = 1000 + 16ull * l;
    const size_t rb = m->row_bytes(H);
    uint8_t* qkv = m->at<uint8_t>(L.qkv);
    st = quantize_rows(m, qkv, L.q_dim, H, mode, staging, staging_elems, gen(s0 + 0, H));
    if (st == GH_OK)
      st = quantize_rows(m, qkv + (size_t)L.q_dim * rb, L.kv_dim, H, mode, staging, staging_elems,
                         gen(s0 + 1, H));
    if (st == GH_OK && !L.k_eq_v)
      st = quantize_rows(m, qkv + (size_t)(L.q_dim + L.kv_dim) * rb, L.kv_dim, H, mode, staging,
                         staging_elems, gen(s0 + 2, H));
    if (st == GH_OK)
      st = quantize_rows(m, m->at<uint8_t>(L.o), H, L.q_dim, mode, staging, staging_elems,
                         gen(s0 + 3, L.q_dim));
    if (st == GH_OK)
      st = quantize_rows(m, m->at<uint8_t>(L.gate), I, H, mode, staging, staging_elems,
                         gen(s0 + 4, H));
    if (st == GH_OK)
      st = quantize_rows(m, m->at<uint8_t>(L.up), I, H, mode, staging, staging_elems,
                         gen(s0 + 5, H));
    if (st == GH_OK)
      st = quantize_rows(m, m->at<uint8_t>(L.down), H, I, mode, staging, staging_elems,
                         gen(s0 + 6, I));
    if (st == GH_OK) st = norm(L.input_norm, H, s0 + 7);
    if (st == GH_OK) st = norm(L.q_norm, L.head_dim, s0 + 8);
    if (st == GH_OK) st = norm(L.k_norm, L.head_dim, s0 + 9);
    if (st == GH_OK) st = norm(L.post_attn, H, s0 + 10);
    if (st == GH_OK) st = norm(L.pre_ffn, H, s0 + 11);
    if (st == GH_OK) st = norm(L.post_ffn, H, s0 + 12);
  }
  // tied embedding / LM head: stream 999
  if (st == GH_OK) st = gh_synth_normal_bf16_dev(ctx, m->embed_dev, (size_t)V * H, seed, 999, 0.0,
                                                  0.02, 0);
  if (st == GH_OK && mode == GH_QUANT_NONE) {  // the bf16 head is the embedding itself
    hipError_t e = hipMemcpyAsync(m->at<uint8_t>(m->lm_head), m->embed_dev, (size_t)V * H * 2,
                                  hipMemcpyDeviceToDevice, ctx->stream);
    if (e != hipSuccess) st = fail(GH_ERR_HIP, std::string("LM head copy: ") + hipGetErrorString(e));
  } else if (st == GH_OK) {
    const uint32_t chunk = (uint32_t)std::max<size_t>(1, staging_elems / H);
    for (uint32_t r0 = 0; r0 < V && st == GH_OK; r0 += chunk) {
      const uint32_t n = std::min(chunk, V - r0);
      st = gh_quantize_matrix_dev(ctx, m->at<uint8_t>(m->lm_head) + (size_t)r0 * (H / 32) * 36,
                                  m->embed_dev + (size_t)r0 * H, n, H, GH_QUANT_Q8);
    }
  }
  if (st == GH_OK) st = norm(m->final_norm, H, 998);
  hipStreamSynchronize(ctx->stream);
  hipFree(staging);
  if (st != GH_OK) {
    delete m;
    return st;
  }
  return finish_init(m, out);
}

void gh_model_deinit(gh_model* m) { delete m; }

namespace {
gh_status forward_token(gh_model* m, const float* x, int want_logits, uint64_t clock,
                        uint32_t slot_idx, const uint32_t* active_slots, uint32_t n_active,
                        uint32_t* out_token);
}  // namespace

gh_status gh_dispatch_forward_token(gh_model* m, const float* x, int want_logits, uint64_t clock,
                                    uint32_t slot_idx, const uint32_t* active_slots,
                                    uint32_t n_active, uint32_t* out_token) {
  return forward_token(m, x, want_logits, clock, slot_idx, active_slots, n_active, out_token);
}

}  // extern "C"

namespace {
gh_status forward_token(gh_model* m, const float* x, int want_logits, uint64_t clock,
                        uint32_t slot_idx, const uint32_t* active_slots, uint32_t n_active,
                        uint32_t* out_token) {
  if (!m || !x || !active_slots || !out_token)
    return fail(GH_ERR_INVALID, "gh_dispatch_forward_token: null argument");
  *out_token = 0;
  const gh_model_config& c = m->cfg;
  if (n_active == 0 || n_active > c.max_slots || slot_idx >= c.max_slots)
    return fail(GH_ERR_INVALID, "gh_dispatch_forward_token: active list / slot out of range");
  for (uint32_t i = 0; i < n_active; i++)
    if (active_slots[i] >= c.max_slots)
      return fail(GH_ERR_INVALID, "gh_dispatch_forward_token: active slot out of range");
  if (clock > 0xFFFFFFFFull) return fail(GH_ERR_INVALID, "gh_dispatch_forward_token: clock > 2^32");
  memcpy(m->h_x, x, (size_t)c.hidden_size * 4);
  memcpy(m->h_active, active_slots, (size_t)n_active * 4);
  m->h_step[0] = (uint32_t)clock;
  m->h_step[1] = slot_idx;
  m->h_step[2] = n_active;
  // the list comes from the host; bit 1 tells the attention when it is 0 .. S-1
  bool dense = true;
  for (uint32_t i = 0; i < n_active && dense; i++) dense = active_slots[i] == i;
  m->h_step[3] = dense ? 2u : 0u;
  if (m->ring) {  // keep the ring state in step (the ring kernel records the activation)
    if (slot_idx != gh_ring_slot_index(m->ring, clock))
      return fail(GH_ERR_INVALID, "gh_dispatch_forward_token: slot_idx is not the ring's slot "
                                  "for this clock");
    gh_ring_activate_slot(m->ring, 0, clock);
  }
  return run_token(m, want_logits != 0, (m->active - m->io) + (size_t)n_active * 4, out_token);
}
}  // namespace

extern "C" {

gh_status gh_model_ring_init(gh_model* m, uint32_t num_anchors, uint32_t window_size,
                             uint32_t num_recall) {
  if (!m) return fail(GH_ERR_INVALID, "gh_model_ring_init: null model");
  if (window_size == 0 || (uint64_t)num_anchors + window_size + num_recall > m->cfg.max_slots)
    return fail(GH_ERR_INVALID, "gh_model_ring_init: need window > 0 and anchors + window + "
                                "recall <= max_slots");
  gh_ring* r = nullptr;
  gh_status st = gh_ring_create(1, num_anchors, window_size, num_recall, &r);
  if (st != GH_OK) return st;
  if (m->ring) gh_ring_destroy(m->ring);
  m->ring = r;
  const bool reshape = m->ring_a != num_anchors || m->ring_w != window_size || m->ring_r != num_recall;
  m->ring_a = num_anchors;
  m->ring_w = window_size;
  m->ring_r = num_recall;
  if ((st = ring_upload(m)) != GH_OK) return st;
  // the ring kernel takes the tier sizes as arguments: record again
  if (reshape && (st = rerecord(m)) != GH_OK) return st;
  return GH_OK;
}

gh_status gh_model_forward_clock(gh_model* m, const float* x, int want_logits, uint64_t clock,
                                 uint32_t* out_token) {
  if (!m || !x || !out_token) return fail(GH_ERR_INVALID, "gh_model_forward_clock: null argument");
  *out_token = 0;
  if (!m->ring) return fail(GH_ERR_INVALID, "gh_model_forward_clock: gh_model_ring_init first");
  if (clock > 0xFFFFFFFFull) return fail(GH_ERR_INVALID, "gh_model_forward_clock: clock > 2^32");
  memcpy(m->h_x, x, (size_t)m->cfg.hidden_size * 4);
  m->h_step[0] = (uint32_t)clock;
  m->h_step[1] = m->h_step[2] = 0;
  m->h_step[3] = 1;  // the ring kernel activates the slot and builds the list
  gh_ring_activate_slot(m->ring, 0, clock);
  return run_token(m, want_logits != 0, (m->step - m->io) + 16, out_token);
}

gh_status gh_model_submit_prerecorded(gh_model* m, gh_graph_kind which) {
  if (!m) return fail(GH_ERR_INVALID, "gh_model_submit_prerecorded: null model");
  if (which != GH_GRAPH_DECODE && which != GH_GRAPH_PREFILL)
    return fail(GH_ERR_INVALID, "gh_model_submit_prerecorded: unknown graph");
  uint32_t tok = 0;
  return run_token(m, which == GH_GRAPH_DECODE, 0, &tok);
}

gh_status gh_model_ring_clear_recall(gh_model* m) {
  if (!m || !m->ring) return fail(GH_ERR_INVALID, "gh_model_ring_clear_recall: no device ring");
  gh_ring_clear_recall(m->ring);
  return ring_upload(m);
}

gh_status gh_model_write_recall_kv(gh_model* m, uint32_t layer, uint32_t rank, const float* k,
                                   const float* v, uint64_t clock) {
  if (!m || !k || !v) return fail(GH_ERR_INVALID, "gh_model_write_recall_kv: null argument");
  if (!m->ring) return fail(GH_ERR_INVALID, "gh_model_write_recall_kv: gh_model_ring_init first");
  if (layer >= m->layers.size() || rank >= m->ring_r || clock > 0xFFFFFFFFull)
    return fail(GH_ERR_INVALID, "gh_model_write_recall_kv: layer, rank or clock out of range");
  const Layer& L = m->layers[layer];
  const size_t slot = (size_t)m->ring_a + m->ring_w + rank;
  gh_status st = gh_buffer_write(m->ctx, m->at<float>(L.k_cache) + slot * L.kv_dim, k, L.kv_dim * 4);
  if (st == GH_OK)
    st = gh_buffer_write(m->ctx, m->at<float>(L.v_cache) + slot * L.kv_dim, v, L.kv_dim * 4);
  if (st != GH_OK) return st;
  // writeRecallKV's bookkeeping; the device path lists layer 0's ring
  // (src/model/forward.zig:42-43), so layer 0 activates the slot
  if (layer == 0) {
    gh_ring_activate_recall(m->ring, 0, rank, clock);
    return ring_upload(m);
  }
  return GH_OK;
}

gh_status gh_model_ring_prefill(gh_model* m, const float* x, uint32_t T, uint64_t first_clock,
                                int want_logits, uint32_t* out_token) {
  if (!m || !x || !out_token) return fail(GH_ERR_INVALID, "gh_model_ring_prefill: null argument");
  *out_token = 0;
  if (!m->ring) return fail(GH_ERR_INVALID, "gh_model_ring_prefill: gh_model_ring_init first");
  if (T == 0 || first_clock + T - 1 > 0xFFFFFFFFull)
    return fail(GH_ERR_INVALID, "gh_model_ring_prefill: T is zero or a clock exceeds 2^32");
  const uint32_t total = gh_ring_total_slots(m->ring);
  std::vector<uint64_t> clocks(T);
  std::vector<uint32_t> slots(T), n(T), lists((size_t)T * total);
  // the lists as the per-token calls would see them: slot activations of the
  // earlier tokens of the batch included, later ones not; a failed call
  // leaves the ring as it was
  gh_ring* r = gh::ring_clone(m->ring);
  if (!r) return fail(GH_ERR_ALLOC, "gh_model_ring_prefill: ring copy");
  for (uint32_t t = 0; t < T; t++) {
    clocks[t] = first_clock + t;
    slots[t] = gh_ring_activate_slot(r, 0, clocks[t]);
    n[t] = gh_ring_active_slots(r, 0, clocks[t], &lists[(size_t)t * total], total);
  }
  // gh_model_prefill advances m->ring as its tokens or chunks finish: keep
  // the state from before the call to put back on failure
  gh_ring* before = gh::ring_clone(m->ring);
  if (!before) {
    gh_ring_destroy(r);
    return fail(GH_ERR_ALLOC, "gh_model_ring_prefill: ring copy");
  }
  gh_status st = gh_model_prefill(m, x, T, clocks.data(), slots.data(), lists.data(), total,
                                  n.data(), want_logits, out_token);
  gh_ring_destroy(st == GH_OK ? before : r);
  gh_ring_destroy(m->ring);
  m->ring = st == GH_OK ? r : before;
  if (st != GH_OK) {
    const std::string why = gh_last_error();
    ring_upload(m);
    return fail(st, why);
  }
  return ring_upload(m);
}

gh_status gh_model_set_quiescence(gh_model* m, float threshold) {
  if (!m) return fail(GH_ERR_INVALID, "gh_model_set_quiescence: null model");
  m->q_on = threshold != 0.0f;
  m->q_thr = threshold;
  gh_status st = reset_gates(m);
  if (st != GH_OK) return st;
  return rerecord(m);
}

gh_status gh_model_set_trace(gh_model* m, int enable) {
  if (!m) return fail(GH_ERR_INVALID, "gh_model_set_trace: null model");
  if ((enable != 0) == m->trace_on) return GH_OK;
  if (enable && !m->trace) {
    const size_t bytes = (size_t)(m->cfg.num_hidden_layers + 1) * m->cfg.hidden_size * 4;
    hipError_t e = hipMalloc(&m->trace, bytes);
    if (e != hipSuccess) return fail(GH_ERR_ALLOC, std::string("trace buffer: ") + hipGetErrorString(e));
    if (hipMemset(m->trace, 0, bytes) != hipSuccess) return fail(GH_ERR_HIP, "trace buffer clear");
  }
  m->trace_on = enable != 0;
  return rerecord(m);
}

gh_status gh_model_prefill(gh_model* m, const float* x, uint32_t T, const uint64_t* clocks,
                           const uint32_t* slot_idx, const uint32_t* active,
                           uint32_t active_stride, const uint32_t* n_active, int want_logits,
                           uint32_t* out_token) {
  if (!m || !x || !clocks || !slot_idx || !active || !n_active || !out_token)
    return fail(GH_ERR_INVALID, "gh_model_prefill: null argument");
  *out_token = 0;
  const gh_model_config& c = m->cfg;
  if (T == 0) return fail(GH_ERR_INVALID, "gh_model_prefill: T is zero");
  if (c.hidden_size > 8192)
    return fail(GH_ERR_UNSUPPORTED, "gh_model_prefill: hidden size above 8192");
  uint32_t max_n = 1;
  for (uint32_t t = 0; t < T; t++) max_n = std::max(max_n, n_active[t]);
  if (active_stride < max_n) return fail(GH_ERR_INVALID, "gh_model_prefill: active_stride < n_active");
  m->pf_maxn = max_n;
  // Slot writers of this batch.  The batched kernels write every token's K/V
  // before any token attends, so they need each token to read only its own
  // and earlier tokens' slots, and no slot written twice.  A batch that
  // breaks this (a wrapped window: token t still attends to the slot token
  // t + 1 overwrites) runs token by token instead, as does a short one.
  std::vector<int64_t> writer(c.max_slots, -1);
  bool conflict = false;
  for (uint32_t t = 0; t < T; t++) {
    if (slot_idx[t] >= c.max_slots || clocks[t] > 0xFFFFFFFFull)
      return fail(GH_ERR_INVALID, "gh_model_prefill: slot or clock out of range");
    conflict = conflict || writer[slot_idx[t]] >= 0;
    writer[slot_idx[t]] = t;
  }
  for (uint32_t t = 0; t < T; t++) {
    if (n_active[t] == 0 || n_active[t] > c.max_slots)
      return fail(GH_ERR_INVALID, "gh_model_prefill: active list length out of range");
    const uint32_t* row = active + (size_t)t * active_stride;
    for (uint32_t i = 0; i < n_active[t]; i++) {
      if (row[i] >= c.max_slots) return fail(GH_ERR_INVALID, "gh_model_prefill: active slot out of range");
      conflict = conflict || writer[row[i]] > (int64_t)t;
    }
  }
  if (m->ring)
    for (uint32_t t = 0; t < T; t++)
      if (slot_idx[t] != gh_ring_slot_index(m->ring, clocks[t]))
        return fail(GH_ERR_INVALID, "gh_model_prefill: a slot is not the ring's slot for its clock");
  // Gating on: the last prompt token computes the logits, and forwardToken's
  // GPU branch sends such a token through the decode graph, which gates at
  // the threshold (compute_logits, src/model/forward.zig:41-45; recorded with
  // quiescence_thresh, src/gpu/model_gpu.zig:182).  The tokens before it go
  // through the prefill path, whose gates run at threshold 0 (model_gpu.zig:
  // 183).
  if (m->q_on && want_logits) {
    if (T > 1) {
      gh_status ps = gh_model_prefill(m, x, T - 1, clocks, slot_idx, active, active_stride,
                                      n_active, 0, out_token);
      if (ps != GH_OK) return ps;
    }
    const uint32_t t = T - 1;
    return forward_token(m, x + (size_t)t * c.hidden_size, 1, clocks[t], slot_idx[t],
                         active + (size_t)t * active_stride, n_active[t], out_token);
  }
  if (conflict && T > m->stage_rows && T > m->seq_prefill_max) {
    // staged batches hold at most stage_rows tokens: consecutive chunks
    for (uint32_t t0 = 0; t0 < T; t0 += m->stage_rows) {
      const uint32_t n = std::min(T - t0, m->stage_rows);
      gh_status cs = gh_model_prefill(m, x + (size_t)t0 * c.hidden_size, n, clocks + t0,
                                      slot_idx + t0, active + (size_t)t0 * active_stride,
                                      active_stride, n_active + t0,
                                      t0 + n == T ? want_logits : 0, out_token);
      if (cs != GH_OK) return cs;
    }
    return GH_OK;
  }
  if (T <= m->seq_prefill_max) {
    // token by token through the recorded graphs, as the reference prefills
    // (src/interactive.zig:33-37): the prefill graph, then the decode graph
    // for a last token with logits; each token activates its ring slot itself
    for (uint32_t t = 0; t < T; t++) {
      gh_status ts = forward_token(m, x + (size_t)t * c.hidden_size, t + 1 == T && want_logits,
                                   clocks[t], slot_idx[t], active + (size_t)t * active_stride,
                                   n_active[t], out_token);
      if (ts != GH_OK) return ts;
    }
    return m->ring ? ring_upload(m) : GH_OK;
  }
  gh_status st = ensure_prefill(m, T, active_stride);
  if (st != GH_OK) return st;
  hipStream_t s = m->ctx->stream;
  // A staged batch (conflict): token t writes its K/V to staging row
  // max_slots + t, and each list entry names the staging row of the slot's
  // latest writer so far in the batch, else the ring slot, which still holds
  // its value from before the batch.  After the layers, the latest writer's
  // row of each written slot moves into the slot.
  const uint32_t nslot = c.max_slots;
  std::vector<uint32_t> staged_lists, pairs;
  if (conflict) {
    staged_lists.assign((size_t)T * active_stride, 0u);
    std::vector<int64_t> last(nslot, -1);
    for (uint32_t t = 0; t < T; t++) {
      last[slot_idx[t]] = t;
      const uint32_t* row = active + (size_t)t * active_stride;
      uint32_t* out = &staged_lists[(size_t)t * active_stride];
      for (uint32_t i = 0; i < n_active[t]; i++)
        out[i] = last[row[i]] >= 0 ? nslot + (uint32_t)last[row[i]] : row[i];
    }
    for (uint32_t sl = 0; sl < nslot; sl++)
      if (last[sl] >= 0) {
        pairs.push_back(sl);
        pairs.push_back(nslot + (uint32_t)last[sl]);
      }
    active = staged_lists.data();
  }
  const uint32_t nrows = conflict ? nslot + T : nslot;  // cache rows the lists may name
  std::vector<uint32_t> meta(3 * (size_t)T);
  for (uint32_t t = 0; t < T; t++) {
    meta[t] = (uint32_t)clocks[t];
    meta[T + t] = conflict ? nslot + t : slot_idx[t];
    meta[2 * T + t] = n_active[t];
  }
  std::vector<uint32_t> act((size_t)T * m->pf_stride, 0u);
  for (uint32_t t = 0; t < T; t++)
    memcpy(&act[(size_t)t * m->pf_stride], active + (size_t)t * active_stride, (size_t)n_active[t] * 4);
  hipError_t e = hipMemcpyAsync(m->pf_x, x, (size_t)T * c.hidden_size * 4, hipMemcpyHostToDevice, s);
  if (e == hipSuccess) e = hipMemcpyAsync(m->pf_meta, meta.data(), meta.size() * 4, hipMemcpyHostToDevice, s);
  if (e == hipSuccess) e = hipMemcpyAsync(m->pf_active, act.data(), act.size() * 4, hipMemcpyHostToDevice, s);
  // Grouped attention: the matrix-core kernel when every layer has head_dim
  // 256 and one G = nq / nkv dividing 16 (16 / G tokens per group) and the
  // batch has more than 64 tokens, else the 4-token kernel when every layer
  // has G <= 2 and head_dim <= 256, else the per-token kernel.  The union of a group's lists keeps the order of first
  // appearance; a list that names one slot twice keeps the per-token kernel
  // (a union entry counts a slot once per token).
  uint32_t gkind = 0, gtok = 0;
  {
    bool all256 = true, small = true, sameG = true;
    uint32_t G0 = 0;
    for (auto& L : m->layers) {
      const uint32_t G = c.num_attention_heads / L.nkv;
      if (G0 == 0) G0 = G;
      sameG = sameG && G == G0;
      all256 = all256 && L.head_dim == 256;
      small = small && G <= 2 && L.head_dim <= 256;
    }
    if (all256 && sameG && G0 >= 1 && G0 <= 16 && 16 % G0 == 0) {
      // up to 64 tokens the per-token kernel (one workgroup per kv head and
      // token) is as fast or faster: 12B shape, 16 / 32 / 64 tokens
      // 5.66 / 6.65 / 9.95 ms against 5.83 / 6.83 / 10.05 ms; at 96 the two
      // tie and at 128 the matrix-core kernel leads (14.67 against 14.70 ms).
      // GH_PF_ATTN_MFMA=1 (read per call) takes the matrix-core kernel for
      // any batch.
      const char* fm = getenv("GH_PF_ATTN_MFMA");
      if (T > 64 || (fm && fm[0] == '1')) gkind = 2;
      gtok = 16 / G0;
    } else if (small && nrows <= (1u << 24)) {
      gkind = 1;
      gtok = kPfGroup;
    }
  }
  m->pf_gkind = 0;
  std::vector<uint32_t> uni, ucount;
  if (gkind) {
    const uint32_t groups = (T + gtok - 1) / gtok;
    const uint32_t ustride = std::min(gtok * m->pf_stride, nrows);
    uni.assign((size_t)groups * ustride * 2, 0u);
    ucount.assign(groups, 0u);
    std::vector<uint32_t> stamp(nrows, 0u), pos(nrows);
    bool ok = true;
    for (uint32_t g = 0; g < groups && ok; g++) {
      uint32_t* u = &uni[(size_t)g * ustride * 2];
      uint32_t n = 0;
      for (uint32_t i = 0; i < gtok && g * gtok + i < T && ok; i++) {
        const uint32_t t = g * gtok + i;
        const uint32_t* row = active + (size_t)t * active_stride;
        for (uint32_t k = 0; k < n_active[t]; k++) {
          const uint32_t slot = row[k];
          if (stamp[slot] != g + 1) {
            stamp[slot] = g + 1;
            pos[slot] = n;
            u[2 * n] = slot;
            u[2 * n + 1] = 1u << i;
            n++;
          } else if ((u[2 * pos[slot] + 1] >> i) & 1u) {
            ok = false;
            break;
          } else {
            u[2 * pos[slot] + 1] |= 1u << i;
          }
        }
      }
      ucount[g] = n;
    }
    if (ok) {
      m->pf_gkind = gkind;
      m->pf_gtok = gtok;
      m->pf_ustride = ustride;
      if (e == hipSuccess)
        e = hipMemcpyAsync(m->pf_union, uni.data(), uni.size() * 4, hipMemcpyHostToDevice, s);
      if (e == hipSuccess)
        e = hipMemcpyAsync(m->pf_ucount, ucount.data(), ucount.size() * 4, hipMemcpyHostToDevice, s);
    }
  }
  std::vector<uint8_t> table;
  if (conflict) {  // offsets and row words of every cache, then the pairs
    const size_t nc = 2 * m->layers.size();
    table.resize(nc * 12 + pairs.size() * 4);
    for (size_t l = 0; l < m->layers.size(); l++) {
      const uint64_t off[2] = {m->layers[l].k_cache, m->layers[l].v_cache};
      memcpy(&table[2 * l * 8], off, 16);
      const uint32_t w[2] = {m->layers[l].kv_dim, m->layers[l].kv_dim};
      memcpy(&table[nc * 8 + 2 * l * 4], w, 8);
    }
    memcpy(&table[nc * 12], pairs.data(), pairs.size() * 4);
    if (e == hipSuccess)
      e = hipMemcpyAsync(m->pf_scatter, table.data(), table.size(), hipMemcpyHostToDevice, s);
  }
  if (e != hipSuccess) return hip_fail(e, "gh_model_prefill: input copies");
  if (m->trace_on && m->pf_trace_cap < T) {  // the batch trace, [L][T][hidden]
    hipStreamSynchronize(s);
    if (m->pf_trace) hipFree(m->pf_trace);
    m->pf_trace = nullptr;
    m->pf_trace_cap = m->pf_trace_T = 0;
    e = hipMalloc(&m->pf_trace, (size_t)c.num_hidden_layers * T * c.hidden_size * 4);
    if (e != hipSuccess) return fail(GH_ERR_ALLOC, std::string("prefill trace: ") + hipGetErrorString(e));
    m->pf_trace_cap = T;
  }
  if (m->trace_on) m->pf_trace_T = T;
  if ((st = prefill_forward(m, T, want_logits != 0)) != GH_OK) return st;
  if (conflict) {
    const size_t nc = 2 * m->layers.size();
    uint8_t* base = m->arena;
    const uint64_t* off = reinterpret_cast<const uint64_t*>(m->pf_scatter);
    const uint32_t* words = m->pf_scatter + nc * 2;
    const uint32_t* prs = m->pf_scatter + nc * 3;
    void* args[] = {&base, &off, &words, &prs};
    if ((st = m->ctx->launch("gh_rows_scatter_k", dim3((unsigned)(pairs.size() / 2), (unsigned)nc),
                             dim3(256), 0, args)) != GH_OK)
      return st;
  }
  if (want_logits) {
    e = hipMemcpyAsync(m->h_token, m->at<uint32_t>(m->token), 4, hipMemcpyDeviceToHost, s);
    if (e != hipSuccess) return hip_fail(e, "gh_model_prefill: token copy");
  }
  e = hipStreamSynchronize(s);
  if (e != hipSuccess) return hip_fail(e, "gh_model_prefill");
  m->hidden_final = want_logits ? m->x1 : kNone;
  if (want_logits) *out_token = m->h_token[0];
  if (m->ring) {
    for (uint32_t t = 0; t < T; t++) gh_ring_activate_slot(m->ring, 0, clocks[t]);
    return ring_upload(m);
  }
  return GH_OK;
}

gh_status gh_model_embed(gh_model* m, uint32_t token, float* x_host) {
  if (!m || !x_host) return fail(GH_ERR_INVALID, "gh_model_embed: null argument");
  if (!m->embed_dev) return fail(GH_ERR_UNSUPPORTED, "gh_model_embed: model has no device embedding");
  const uint32_t H = m->cfg.hidden_size;
  if (token >= m->cfg.vocab_size) return fail(GH_ERR_INVALID, "gh_model_embed: token out of range");
  std::vector<uint16_t> row(H);
  gh_status st = gh_buffer_read(m->ctx, row.data(), m->embed_dev + (size_t)token * H, (size_t)H * 2);
  if (st != GH_OK) return st;
  const float scale = sqrtf((float)H);  // @sqrt(f32(H)), src/model/forward.zig:33
  for (uint32_t i = 0; i < H; i++) {
    uint32_t u = (uint32_t)row[i] << 16;
    float f;
    memcpy(&f, &u, 4);
    x_host[i] = f * scale;
  }
  return GH_OK;
}

}  // extern "C"

namespace {

// Prefill buffers for up to T tokens with active lists of up to stride slots.
gh_status ensure_prefill(gh_model* m, uint32_t T, uint32_t stride) {
  if (m->pf_arena && m->pf_cap >= T && m->pf_stride >= stride) return GH_OK;
  const gh_model_config& c = m->cfg;
  const uint32_t H = c.hidden_size, I = c.intermediate_size;
  T = std::max(T, m->pf_cap);
  stride = std::max(stride, m->pf_stride);
  uint32_t max_qkv = 0;
  for (auto& L : m->layers) max_qkv = std::max(max_qkv, L.qkv_rows);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    size_t o = off;
    off += (bytes + 255) & ~(size_t)255;
    return o;
  };
  const size_t o_x = take((size_t)T * H * 4), o_qkv = take((size_t)T * max_qkv * 4);
  const size_t o_o = take((size_t)T * H * 4), o_m = take((size_t)T * H * 4);
  const size_t o_xn = take((size_t)T * H * 4), o_attn = take((size_t)T * m->max_q * 4);
  const size_t o_act = take((size_t)T * I * 4), o_meta = take((size_t)3 * T * 4);
  const size_t o_active = take((size_t)T * stride * 4), o_rs = take((size_t)T * 4);
  // unions: at most ceil(T / g) groups of min(g * stride, max_slots) pairs, g <= 16
  const size_t o_union = take((size_t)(T + 15) * stride * 8), o_ucount = take((size_t)T * 4);
  // staged batches: per cache (K and V of each layer) its byte offset in the
  // arena and its row length in words, then (slot, staging row) pairs
  const size_t n_caches = 2 * m->layers.size();
  const size_t o_scatter = take(n_caches * 12 + (size_t)T * 8);
  if (m->pf_arena) {
    hipStreamSynchronize(m->ctx->stream);
    hipFree(m->pf_arena);
    m->pf_arena = nullptr;
    m->pf_cap = m->pf_stride = 0;
  }
  hipError_t e = hipMalloc(&m->pf_arena, off);
  if (e != hipSuccess) return fail(GH_ERR_ALLOC, std::string("prefill buffers: ") + hipGetErrorString(e));
  auto f32 = [&](size_t o) { return reinterpret_cast<float*>(m->pf_arena + o); };
  auto u32 = [&](size_t o) { return reinterpret_cast<uint32_t*>(m->pf_arena + o); };
  m->pf_x = f32(o_x);
  m->pf_qkv = f32(o_qkv);
  m->pf_o = f32(o_o);
  m->pf_m = f32(o_m);
  m->pf_xn = f32(o_xn);
  m->pf_attn = f32(o_attn);
  m->pf_act = f32(o_act);
  m->pf_meta = u32(o_meta);
  m->pf_active = u32(o_active);
  m->pf_rs = f32(o_rs);
  m->pf_union = u32(o_union);
  m->pf_ucount = u32(o_ucount);
  m->pf_scatter = u32(o_scatter);
  m->pf_cap = T;
  m->pf_stride = stride;
  return GH_OK;
}

// gh_pf_norm_k over T rows (mode 1: RMSNorm; mode 2: residual add + RMSNorm,
// the residual R given as rz unsummed K-split planes [rz][T][H]).
gh_status launch_pf_norm(gh_model* m, uint32_t T, const float* R, const float* wr,
                         const float* w, float s, uint32_t mode, uint32_t rz = 1) {
  uint32_t H = m->cfg.hidden_size;
  float eps = m->cfg.rms_norm_eps;
  float* X = m->pf_x;
  // the normed rows as the GEMM's A operand: fp16 hi/lo halves ([T][2H]) in pf_xn
  uint16_t* Xa = reinterpret_cast<uint16_t*>(m->pf_xn);
  float* rs = m->pf_rs;
  uint32_t perm = gh::pf_halves_format(m->mode);  // the GEMM's A-operand format
  void* args[] = {&X, const_cast<float**>(&R), const_cast<float**>(&wr), const_cast<float**>(&w),
                  &Xa, &rs, &H, &s, &eps, &mode, &perm, &rz};
  // 512 threads for rows of up to 4096 (GH_PF_NORM_1024 keeps the 1024-thread form)
  const bool narrow = H <= 8u * 512u && getenv("GH_PF_NORM_1024") == nullptr;
  return m->ctx->launch(narrow ? "gh_pf_norm_512_k" : "gh_pf_norm_k", dim3(T),
                        dim3(narrow ? 512 : 1024), 0, args);
}

gh_status prefill_forward(gh_model* m, uint32_t T, bool want_logits) {
  gh_context* ctx = m->ctx;
  const gh_model_config& c = m->cfg;
  const uint32_t H = c.hidden_size, I = c.intermediate_size;
  gh_status st;
  uint32_t* clocks = m->pf_meta;
  uint32_t* slots = m->pf_meta + T;
  uint32_t* nact = m->pf_meta + 2 * T;
  // the down projection's output as the next layer's norm reads it: its
  // K-split planes, summed by that norm (the last layer's is summed in place)
  const float* m_planes = m->pf_m;
  uint32_t m_nz = 1;
  for (uint32_t l = 0; l < c.num_hidden_layers; l++) {
    const Layer& L = m->layers[l];
    // 1. xn = norm(x) (layer 0: RMSNorm; later: post-FFN add + layer scalar + norm)
    if (l == 0) {
      st = launch_pf_norm(m, T, nullptr, nullptr, m->at<float>(L.input_norm), 1.0f, 1);
    } else {
      const Layer& P = m->layers[l - 1];
      st = launch_pf_norm(m, T, m_planes, P.post_ffn == kNone ? nullptr : m->at<float>(P.post_ffn),
                          m->at<float>(L.input_norm), P.scalar, 2, m_nz);
    }
    if (st != GH_OK) return st;
    // residual trace: row l = the last token's input to layer l, and every
    // token's in the batch trace
    if (m->trace_on &&
        ((st = copy_words(m, m->trace + (size_t)l * H, m->pf_x + (size_t)(T - 1) * H, H)) != GH_OK ||
         (st = copy_words(m, m->pf_trace + (size_t)l * T * H, m->pf_x, (uint64_t)T * H)) != GH_OK))
      return st;
    // with gating on, the per-token prefill graph runs every gate at
    // threshold 0 (model_gpu.zig:183): each gated layer ends holding the last
    // token's input as its previous input, and every layer has run
    if (m->q_on && l >= c.num_hidden_layers / 3 &&
        (st = copy_words(m, m->at<float>(m->xprev) + (size_t)l * H, m->pf_x + (size_t)(T - 1) * H,
                         H)) != GH_OK)
      return st;
    // 2. [q|k|v] rows of every token.  With head_dim 256 the norm + RoPE
    //    kernel below sums a K split's planes itself, so the GEMM may leave
    //    them unsummed (and take the faster split shape of a long prompt).
    const uint16_t* xh = reinterpret_cast<const uint16_t*>(m->pf_xn);
    const bool rope4 = L.head_dim == 256 && c.num_attention_heads + 2 * L.nkv <= 64;
    const float* qkv_planes = m->pf_qkv;
    uint32_t qkv_nz = 1;
    if ((st = gh::launch_prefill_gemm_split(ctx, m->mode, m->at<uint8_t>(L.qkv), nullptr, xh,
                                            m->pf_rs, m->pf_qkv, T, L.qkv_rows, H,
                                            rope4 ? &qkv_planes : nullptr,
                                            rope4 ? &qkv_nz : nullptr)) != GH_OK)
      return st;
    // 3. q/k norm + RoPE in place, K/V into the caches, then attention
    AttnArgs a{};
    a.q = m->pf_qkv;
    a.q_norm = m->at<float>(L.q_norm);
    a.k_norm = m->at<float>(L.k_norm);
    a.k_cache = m->at<float>(L.k_cache);
    a.v_cache = m->at<float>(L.v_cache);
    a.active = m->pf_active;
    a.n_active = nact;
    a.out_rows = m->pf_attn;
    a.nq = c.num_attention_heads;
    a.nkv = L.nkv;
    a.D = L.head_dim;
    a.rot = L.rot;
    a.k_eq_v = L.k_eq_v ? 1 : 0;
    a.nsplit = 1;
    a.theta = L.theta;
    a.eps = c.rms_norm_eps;
    a.scale = 1.0f;  // inv_sqrt_dim = 1.0 (src/model/forward.zig:80)
    a.q_stride = L.qkv_rows;
    a.active_stride = m->pf_stride;
    a.out_stride = L.q_dim;
    a.q_planes = qkv_planes;
    a.nplanes = qkv_nz;
    a.plane_stride = (uint64_t)T * L.qkv_rows;
    {
      void* args[] = {&a, &clocks, &slots};
      // head_dim 256: one workgroup per token (angles once per wave), or for
      // fewer tokens than twice the CUs ceil(jobs / 8) per token; else one
      // wavefront per (head, token).  At 256 tokens the split form measured
      // 20.39 -> 20.15 ms for the prompt, at 512 the same either way
      // (GH_PF_ROPE4_S=0/1 forces one form).
      const char* few_env = getenv("GH_PF_ROPE4_S");
      const bool few = few_env ? atoi(few_env) != 0 : T < 2u * (uint32_t)ctx->num_cus;
      st = !rope4 ? ctx->launch("gh_pf_qkv_rope_k", dim3(a.nq + a.nkv, T), dim3(64), 0, args)
           : few  ? ctx->launch("gh_pf_qkv_rope4_s_k", dim3(T, (a.nq + 2 * a.nkv + 7) / 8),
                                dim3(256), 0, args)
                  : ctx->launch("gh_pf_qkv_rope4_k", dim3(T), dim3(256), 0, args);
      if (st != GH_OK) return st;
    }
    {
      const uint32_t D = L.head_dim;
      void* args[] = {&a};
      if (m->pf_gkind != 0) {
        // one workgroup per (kv head, group of pf_gtok tokens) over the union list
        a.active = m->pf_union;
        a.n_active = m->pf_ucount;
        a.active_stride = 2 * m->pf_ustride;
        a.n_tokens = T;
        const char* name = m->pf_gkind == 2 ? "gh_pf_attn_m_k"
                           : D <= 64        ? "gh_pf_attn_g_d1_k"
                           : D <= 128       ? "gh_pf_attn_g_d2_k"
                                            : "gh_pf_attn_g_d4_k";
        const uint32_t groups = (T + m->pf_gtok - 1) / m->pf_gtok;
        if ((st = ctx->launch(name, dim3(a.nkv, groups), dim3(256), 0, args)) != GH_OK) return st;
      } else {
        const char* name = D <= 64 ? "gh_pf_attn_d1_k"
                           : D <= 128 ? "gh_pf_attn_d2_k"
                           : D <= 256 ? "gh_pf_attn_d4_k" : "gh_pf_attn_d8_k";
        // Long lists (a prompt after the window has wrapped) split each
        // token's list over several workgroups, merged per (head, token) by
        // gh_pf_attn_merge_k, up to about two workgroups per CU: with one
        // workgroup per (kv head, token) a 16-token batch has 128, each
        // walking ~540 slots.  Wrapped 16-token prompts: 7.24 ms unsplit,
        // 6.23 / 6.37 / 6.75 ms at 4 / 8 / 16 splits; 64 tokens (512
        // workgroups unsplit): 11.49 unsplit, 12.16 at 4 splits.
        uint32_t ns = 1;
        const uint32_t wgs = a.nkv * T, fill = (2u * (uint32_t)ctx->num_cus + wgs - 1) / wgs;
        if (m->pf_maxn > 64) ns = std::min(std::min(16u, fill), (m->pf_maxn + 63) / 64);
        if (const char* e = getenv("GH_PF_ATTN_SPLITS")) ns = std::max(1, std::min(16, atoi(e)));
        a.nsplit = ns;
        if (ns > 1) {
          const size_t need = (size_t)T * a.nkv * ns * (a.nq / a.nkv) * (D + 4) * sizeof(float);
          if ((st = ctx->ensure_zeroed(&ctx->attn_scratch, &ctx->attn_scratch_bytes, need)) != GH_OK)
            return st;
          a.part = static_cast<float*>(ctx->attn_scratch);
        }
        if ((st = ctx->launch(name, dim3(a.nkv * ns, T), dim3(256), 0, args)) != GH_OK) return st;
        if (ns > 1 && (st = ctx->launch("gh_pf_attn_merge_k", dim3(a.nq, T), dim3(256), 0, args)) != GH_OK)
          return st;
        a.nsplit = 1;
      }
    }
    // 4. o = W_o . attn (a K split stays unsummed: the norm below adds the planes)
    const float* o_planes = nullptr;
    uint32_t o_nz = 1;
    if ((st = gh::launch_prefill_gemm(ctx, m->mode, m->at<uint8_t>(L.o), nullptr, m->pf_attn,
                                      m->pf_o, T, H, L.q_dim, &o_planes, &o_nz)) != GH_OK)
      return st;
    // 5. x += post_attn_norm(o); act = geglu(W_gate, W_up . pre_ffn_norm(x))
    if ((st = launch_pf_norm(m, T, o_planes,
                             L.post_attn == kNone ? nullptr : m->at<float>(L.post_attn),
                             m->at<float>(L.pre_ffn), 1.0f, 2, o_nz)) != GH_OK)
      return st;
    if ((st = gh::launch_prefill_gemm_split(ctx, m->mode, m->at<uint8_t>(L.gate),
                                            m->at<uint8_t>(L.up), xh, m->pf_rs, m->pf_act, T,
                                            I, H)) != GH_OK)
      return st;
    // 6. m = W_down . act (unsummed planes for the next layer's norm; the last
    //    layer's m is summed into pf_m for the LM-head prologue)
    const bool last = l + 1 == c.num_hidden_layers;
    m_planes = m->pf_m;
    m_nz = 1;
    if ((st = gh::launch_prefill_gemm(ctx, m->mode, m->at<uint8_t>(L.down), nullptr, m->pf_act,
                                      m->pf_m, T, H, I, last ? nullptr : &m_planes,
                                      last ? nullptr : &m_nz)) != GH_OK)
      return st;
    // Many planes (the streamed down projection of a short prompt: 30) are
    // summed over all CUs first: the norm reads its token's planes from one
    // CU each, and at 16 tokens took 14.4 us with 30 planes against 5.2 us
    // with one.
    if (m_nz > 8) {
      if ((st = gh::launch_prefill_plane_sum(ctx, m_planes, m->pf_m, T, H, m_nz)) != GH_OK)
        return st;
      m_planes = m->pf_m;
      m_nz = 1;
    }
  }
  if (m->q_on) {  // every layer ran
    gh_status fs = gh_buffer_fill_u32(ctx, m->arena + m->gate_flags, 1u, c.num_hidden_layers);
    if (fs != GH_OK) return fs;
  }
  if (want_logits) {
    // last token: x = (x + post_ffn_norm(m)) * layer_scalar; argmax(head . final_norm(x))
    const Layer& P = m->layers.back();
    XPro p{};
    p.x = m->pf_x + (size_t)(T - 1) * H;
    p.r = m->pf_m + (size_t)(T - 1) * H;
    p.wr = P.post_ffn == kNone ? nullptr : m->at<float>(P.post_ffn);
    p.w = m->at<float>(m->final_norm);
    p.xout = m->at<float>(m->x1);
    p.s = P.scalar;
    p.eps = c.rms_norm_eps;
    p.mode = 2;
    ArgmaxArgs aa{m->at<uint8_t>(m->lm_head), m->at<float>(m->logits), m->at<uint32_t>(m->amax)};
    if ((st = gh::launch_argmax_stream(ctx, &aa, p, c.vocab_size, H, m->at<uint32_t>(m->token),
                                       m->mode == GH_QUANT_NONE)) != GH_OK)
      return st;
    if (m->trace_on && (st = copy_words(m, m->trace + (size_t)c.num_hidden_layers * H,
                                        m->at<float>(m->x1), H)) != GH_OK)
      return st;
  }
  return GH_OK;
}

// (device pointer, bytes) of a tensor; nullptr when absent.
std::pair<uint8_t*, size_t> tensor_ref(const gh_model* m, int layer, gh_tensor t) {
  const gh_model_config& c = m->cfg;
  const uint32_t H = c.hidden_size, I = c.intermediate_size, V = c.vocab_size;
  switch (t) {
    case GH_T_LM_HEAD:
      return {m->arena + m->lm_head, m->head_bytes()};
    case GH_T_FINAL_NORM:
      return {m->arena + m->final_norm, (size_t)H * 4};
    case GH_T_EMBED:
      return {reinterpret_cast<uint8_t*>(m->embed_dev), m->embed_dev ? (size_t)V * H * 2 : 0};
    case GH_T_LOGITS:
      return {m->arena + m->logits, (size_t)V * 4};
    case GH_T_HIDDEN:  // the final residual of the last call that computed logits
      if (m->hidden_final == kNone || m->hidden_final == 0) return {nullptr, 0};
      return {m->arena + m->hidden_final, (size_t)H * 4};
    case GH_T_STEP:
      return {m->arena + m->step, 16};
    case GH_T_ACTIVE:
      return {m->arena + m->active, (size_t)c.max_slots * 4};
    case GH_T_RING_CLOCKS:
      return {m->arena + m->ring_clock, (size_t)c.max_slots * 4};
    case GH_T_RING_FLAGS:
      return {m->arena + m->ring_flag, (size_t)c.max_slots * 4};
    case GH_T_GATE_FLAGS:
      return {m->arena + m->gate_flags, (size_t)c.num_hidden_layers * 4};
    case GH_T_GATE_PREV:
      return {m->arena + m->xprev, (size_t)c.num_hidden_layers * H * 4};
    default:
      break;
  }
  if (t == GH_T_TRACE) {  // row `layer` of the residual trace, 0..num_layers
    if (!m->trace || layer < 0 || layer > (int)m->layers.size()) return {nullptr, 0};
    return {reinterpret_cast<uint8_t*>(m->trace + (size_t)layer * H), (size_t)H * 4};
  }
  if (t == GH_T_PREFILL_TRACE) {  // layer `layer`'s input rows of the last traced batch
    if (!m->pf_trace || m->pf_trace_T == 0 || layer < 0 || layer >= (int)m->layers.size())
      return {nullptr, 0};
    const size_t n = (size_t)m->pf_trace_T * H;
    return {reinterpret_cast<uint8_t*>(m->pf_trace + (size_t)layer * n), n * 4};
  }
  if (layer < 0 || layer >= (int)m->layers.size()) return {nullptr, 0};
  const Layer& L = m->layers[layer];
  auto vec = [&](size_t off, size_t n) -> std::pair<uint8_t*, size_t> {
    if (off == kNone) return {nullptr, 0};
    return {m->arena + off, n * 4};
  };
  switch (t) {
    case GH_T_QKV: return {m->arena + L.qkv, (size_t)L.qkv_rows * m->row_bytes(H)};
    case GH_T_O_PROJ: return {m->arena + L.o, (size_t)H * m->row_bytes(L.q_dim)};
    case GH_T_GATE: return {m->arena + L.gate, (size_t)I * m->row_bytes(H)};
    case GH_T_UP: return {m->arena + L.up, (size_t)I * m->row_bytes(H)};
    case GH_T_DOWN: return {m->arena + L.down, (size_t)H * m->row_bytes(I)};
    case GH_T_INPUT_NORM: return vec(L.input_norm, H);
    case GH_T_Q_NORM: return vec(L.q_norm, L.head_dim);
    case GH_T_K_NORM: return vec(L.k_norm, L.head_dim);
    case GH_T_POST_ATTN_NORM: return vec(L.post_attn, H);
    case GH_T_PRE_FFN_NORM: return vec(L.pre_ffn, H);
    case GH_T_POST_FFN_NORM: return vec(L.post_ffn, H);
    case GH_T_K_CACHE: return vec(L.k_cache, (size_t)c.max_slots * L.kv_dim);
    case GH_T_V_CACHE: return vec(L.v_cache, (size_t)c.max_slots * L.kv_dim);
    default: return {nullptr, 0};
  }
}

}  // namespace

extern "C" {

size_t gh_model_tensor_bytes(const gh_model* m, int layer, gh_tensor t) {
  if (!m) return 0;
  auto r = tensor_ref(m, layer, t);
  return r.first ? r.second : 0;
}

gh_status gh_model_read_tensor(gh_model* m, int layer, gh_tensor t, void* host, size_t bytes) {
  if (!m || !host) return fail(GH_ERR_INVALID, "gh_model_read_tensor: null argument");
  auto r = tensor_ref(m, layer, t);
  if (!r.first) return fail(GH_ERR_INVALID, "gh_model_read_tensor: no such tensor");
  if (bytes > r.second) return fail(GH_ERR_INVALID, "gh_model_read_tensor: size exceeds tensor");
  return gh_buffer_read(m->ctx, host, r.first, bytes);
}

gh_status gh_model_write_tensor(gh_model* m, int layer, gh_tensor t, const void* host,
                                size_t bytes) {
  if (!m || !host) return fail(GH_ERR_INVALID, "gh_model_write_tensor: null argument");
  auto r = tensor_ref(m, layer, t);
  if (!r.first) return fail(GH_ERR_INVALID, "gh_model_write_tensor: no such tensor");
  if (bytes > r.second) return fail(GH_ERR_INVALID, "gh_model_write_tensor: size exceeds tensor");
  return gh_buffer_write(m->ctx, r.first, host, bytes);
}

}  // extern "C"
