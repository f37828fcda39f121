// engine.cpp -- kernel-level entry points, the counterpart of GpuEngine's
// record* helpers (src/gpu/kernels.zig:80-142): shape checks, launch-shape
// selection, and the launch on the context stream.
#include <stdlib.h>
#include <string.h>

#include <string>

#include "runtime.hpp"
#include "../common/stream_args.h"

using gh::fail;

namespace {

constexpr uint32_t kArgmaxMaxBlocks = 4096;
constexpr size_t kArgmaxScratchBytes = (64 + 2 * kArgmaxMaxBlocks) * 4;

struct GemvCfg {
  int tpr, gpl, wgs_per_cu, depth, nt;
};

unsigned x_lds_bytes(uint32_t K);

// Lanes per row team (TPR) and 4-block groups per lane per row (GPL) with
// TPR * GPL >= the row's group count and the least idle lanes; then a
// persistent grid of wgs_per_cu workgroups per CU (bounded by LDS).
GemvCfg pick_gemv(const gh_context* ctx, uint32_t M, uint32_t K, bool q8, bool wide_ok,
                  bool bf16) {
  const uint32_t ng = K / (bf16 ? 64 : 128);  // lane items per row: 64 bf16 or 128 quantized
  static const int kT[] = {16, 32, 64};
  int best_t = 64, best_g = 4;
  uint32_t best_waste = ~0u;
  for (int g : {1, 2, 4}) {
    for (int t : kT) {
      if ((uint32_t)(t * g) < ng) continue;
      if (t == 16 && g > 1) continue;  // shapes built: 16x1, 32x{1,2,4}, 64x{1,2,4}
      const uint32_t waste = t * g - ng;
      if (waste < best_waste || (waste == best_waste && t > best_t)) {
        best_waste = waste;
        best_t = t;
        best_g = g;
      }
    }
    if (best_waste != ~0u) break;  // prefer one group per lane per row
  }
  // Measured on MI355X (graph replay, 12B decode shapes): one item in flight
  // per lane and 3 (Q4) or 2 (Q8) workgroups per CU read fastest.
  GemvCfg c{best_t, best_g, q8 ? 2 : 3, 1, 256};
  // Long rows (the down projection, K = 15360): 1024-thread workgroups, so
  // one LDS staging of x serves 16 wavefronts; measured 11.6 vs 13.6 us.
  if (wide_ok && K >= 8192 && best_t * best_g >= 128) c = {best_t, best_g, 2, 1, 1024};
  if (bf16) c.depth = 1;  // the bf16 streams exist at depth 1 only
  // tuning "tpr,gpl,wgs_per_cu,depth[,nt]": GH_GEMV_CFG_<M>x<K> for one shape,
  // else GH_GEMV_CFG for every shape it fits
  const std::string shape_key = "GH_GEMV_CFG_" + std::to_string(M) + "x" + std::to_string(K);
  const char* shape_env = getenv(shape_key.c_str());
  if (const char* env = shape_env ? shape_env : getenv("GH_GEMV_CFG")) {
    int t = 0, g = 0, w = 0, d = 0, n = 256;
    const int got = sscanf(env, "%d,%d,%d,%d,%d", &t, &g, &w, &d, &n);
    const bool built = !bf16 || ((t == 64 || g == 1) && d == 1 &&
                                 (n == 256 || (t == 64 && (g == 2 || g == 4))));
    if (got >= 4 && built && (t == 16 || t == 32 || t == 64) && (g == 1 || g == 2 || g == 4) &&
        !(t == 16 && g > 1) && w >= 1 && w <= 32 && (uint32_t)(t * g) >= ng && d >= 1 &&
        d <= 2 && (n == 256 || (n == 1024 && wide_ok && t * g >= 128 && d == 1))) {
      c = {t, g, w, d, n};
    }
  }
  const unsigned lds_cap = (unsigned)(ctx->max_lds / std::max(1u, x_lds_bytes(K)));
  c.wgs_per_cu = std::max(1, std::min<int>(c.wgs_per_cu, (int)lds_cap));
  return c;
}

unsigned x_lds_bytes(uint32_t K) { return (K / 128) * 132 * 4 + (K / 32) * 4; }

gh_status check_gemv(const gh_context* ctx, const void* W, const float* X, const void* Y,
                     uint32_t M, uint32_t K, const char* who) {
  if (!ctx || !W || !X || !Y) return fail(GH_ERR_INVALID, std::string(who) + ": null pointer");
  if (M == 0 || K == 0) return fail(GH_ERR_INVALID, std::string(who) + ": M or K is zero");
  if (K % 128 != 0)
    return fail(GH_ERR_UNSUPPORTED, std::string(who) + ": K must be a multiple of 128");
  if (K > 32768)  // a row team covers at most 64 lanes x 4 groups of 128
    return fail(GH_ERR_UNSUPPORTED, std::string(who) + ": K above 32768");
  if ((reinterpret_cast<uintptr_t>(W) & 15) || (reinterpret_cast<uintptr_t>(X) & 15))
    return fail(GH_ERR_INVALID, std::string(who) + ": W and X must be 16-byte aligned");
  if (x_lds_bytes(K) > ctx->max_lds)
    return fail(GH_ERR_UNSUPPORTED, std::string(who) + ": K too large for the LDS staging of x");
  return GH_OK;
}

}  // namespace

namespace gh {

gh_status stream_shape(gh_context* ctx, const char* family, const char* var, uint32_t M,
                       uint32_t K, StreamShape* out) {
  // The Q4 gate+up with x as given runs the normed form's code (its prologue
  // in mode 0 reads only x, so the results are bit-identical): on MI355X the
  // 15360 x 3840 stream measured 14.87-14.92 us against 15.44-15.49 us for
  // the plain form, whose unconditional first loads let x be staged before
  // they return.  The single-round shapes (8192 x 2048, 8192 x 3840,
  // 3840 x 4096) measured 0.5-0.7 us slower the same way and keep the plain
  // form.
  if (var[0] == '\0' && strcmp(family, "gh_gateup_q4") == 0 && K <= 4u * 4u * 256u) var = "n";
  // 1024-thread variants exist for the plain GEMVs (long rows)
  const bool wide_ok = var[0] == '\0' &&
                       (strcmp(family, "gh_gemv_q4") == 0 || strcmp(family, "gh_gemv_q8") == 0 ||
                        strcmp(family, "gh_gemv_bf16") == 0);
  const bool bf16 = strstr(family, "bf16") != nullptr;
  GemvCfg c = pick_gemv(ctx, M, K, strstr(family, "q8") != nullptr, wide_ok, bf16);
  // a row team covers at most 64 lanes x 4 items (of 128 quantized or 64 bf16 weights)
  if ((uint64_t)c.tpr * c.gpl * (bf16 ? 64u : 128u) < K)
    return fail(GH_ERR_UNSUPPORTED, std::string(family) + ": rows longer than " +
                                        std::to_string(bf16 ? 16384 : 32768) + " weights");
  out->lds = x_lds_bytes(K) + 256;  // + the prologue/epilogue scratch (64 floats)
  if (out->lds > ctx->max_lds) return fail(GH_ERR_UNSUPPORTED, std::string(family) + ": K too large");
  out->name = std::string(family) + var + "_t" + std::to_string(c.tpr) + "_g" +
              std::to_string(c.gpl) + "_d" + std::to_string(c.depth) + (c.nt == 1024 ? "_w" : "");
  out->nt = (unsigned)c.nt;
  // A persistent grid larger than what the CUs hold at once would run its
  // last workgroups as a second, mostly idle wave.
  const int occ = ctx->occupancy(out->name, c.nt, out->lds);
  if (occ <= 0) return fail(GH_ERR_CODE_OBJECT, "kernel not found in the code objects: " + out->name);
  // The same number of workgroups on every CU (a multiple of the CU count)
  // measured faster than fewer workgroups with an equal row count per team.
  const uint32_t teams_per_wg = c.nt / c.tpr;
  const uint32_t cap = (uint32_t)ctx->num_cus * (uint32_t)std::min(c.wgs_per_cu, occ);
  out->grid = std::min<uint32_t>(cap, (M + teams_per_wg - 1) / teams_per_wg);
  if (const char* env = getenv("GH_GEMV_GRID")) {  // tuning: "bal" = balanced rows per team
    if (env[0] == 'b') {
      const uint32_t rows_per_team = (M + cap * teams_per_wg - 1) / (cap * teams_per_wg);
      const uint32_t rows_per_wg = rows_per_team * teams_per_wg;
      out->grid = (M + rows_per_wg - 1) / rows_per_wg;
    }
  }
  return GH_OK;
}

gh_status launch_stream(gh_context* ctx, const char* family, std::vector<void*> fmt_params,
                        const XPro& xp, uint32_t M, uint32_t K, const uint32_t* run) {
  if (xp.mode != 0 && K > 4u * 4u * 256u)  // PRO_U float4 per thread of 256
    return fail(GH_ERR_UNSUPPORTED, std::string(family) + ": normed prologue needs K <= 4096");
  if (xp.mode == 4) {  // a gated layer's first projection computes the gate itself
    if (run) return fail(GH_ERR_INVALID, std::string(family) + ": mode 4 takes no run flag");
    if (!xp.x || !xp.r || !xp.w || !xp.xa || !xp.xout || !xp.xprev || !xp.run_out ||
        (xp.pmode == 2 && !xp.prun) || xp.pmode > 2)
      return fail(GH_ERR_INVALID, std::string(family) + ": mode-4 prologue inputs");
  }
  StreamShape sh;
  gh_status st = stream_shape(ctx, family, xp.mode == 4 ? "g" : xp.mode != 0 ? "n" : "", M, K, &sh);
  if (st != GH_OK) return st;
  XPro xpc = xp;
  std::vector<void*> args = std::move(fmt_params);
  args.insert(args.end(), {&xpc, &M, &K});
  if (run) {  // the gated form takes the run flag as its last parameter
    args.push_back(&run);
    sh.name += "_q";
  }
  return ctx->launch(sh.name, dim3(sh.grid), dim3(sh.nt), sh.lds, args.data());
}

const char* gemv_family(gh_quant_mode mode) {
  return mode == GH_QUANT_Q4 ? "gh_gemv_q4" : mode == GH_QUANT_Q8 ? "gh_gemv_q8" : "gh_gemv_bf16";
}
const char* gateup_family(gh_quant_mode mode) {
  return mode == GH_QUANT_Q4 ? "gh_gateup_q4" : mode == GH_QUANT_Q8 ? "gh_gateup_q8" : "gh_gateup_bf16";
}

gh_status launch_argmax_stream(gh_context* ctx, ArgmaxArgs* a, const XPro& xp, uint32_t M,
                               uint32_t K, uint32_t* token, bool bf16) {
  const char* family = bf16 ? "gh_argmax_bf16" : "gh_argmax_q8";
  StreamShape sh;
  gh_status st = stream_shape(ctx, family, xp.mode != 0, M, K, &sh);
  if (st != GH_OK) return st;
  if (sh.grid > kArgmaxMaxBlocks) return fail(GH_ERR_UNSUPPORTED, "argmax stream: grid too large");
  if ((st = launch_stream(ctx, family, {&a->W, &a->Y, &a->partial}, xp, M, K)) != GH_OK)
    return st;
  uint32_t n = sh.grid;
  void* args[] = {&a->partial, &n, &token};
  return ctx->launch("gh_argmax_final_k", dim3(1), dim3(256), 0, args);
}

gh_status check_pro(const gh_context* ctx, const XPro& p, uint32_t K, const char* who) {
  if (p.mode > 2) return fail(GH_ERR_INVALID, std::string(who) + ": prologue mode must be 0..2");
  if (!p.x || (reinterpret_cast<uintptr_t>(p.x) & 15))
    return fail(GH_ERR_INVALID, std::string(who) + ": x null or not 16-byte aligned");
  if (p.mode >= 1 && (!p.w || (reinterpret_cast<uintptr_t>(p.w) & 15)))
    return fail(GH_ERR_INVALID, std::string(who) + ": norm weight null or misaligned");
  if (p.mode == 2 && (!p.r || !p.xout || (reinterpret_cast<uintptr_t>(p.r) & 15)))
    return fail(GH_ERR_INVALID, std::string(who) + ": residual input/output null or misaligned");
  (void)ctx;
  (void)K;
  return GH_OK;
}

}  // namespace gh

namespace {
using gh::launch_stream;

XPro plain_x(const float* X) {
  XPro p{};
  p.x = X;
  p.mode = 0;
  return p;
}

XPro from_abi(const gh_xprologue* q) {
  XPro p{};
  p.x = q->x;
  p.r = q->r;
  p.wr = q->r_norm;
  p.w = q->norm;
  p.xout = q->x_out;
  p.s = q->scalar;
  p.eps = q->eps;
  p.mode = q->mode;
  return p;
}

}  // namespace

extern "C" {

gh_status gh_gemv_q4(gh_context* ctx, const void* W, const float* X, float* Y, uint32_t M,
                     uint32_t K) {
  gh_status st = check_gemv(ctx, W, X, Y, M, K, "gh_gemv_q4");
  if (st != GH_OK) return st;
  Q4Args a{static_cast<const uint8_t*>(W), Y};
  return launch_stream(ctx, "gh_gemv_q4", &a, plain_x(X), M, K);
}

gh_status gh_gemv_q8(gh_context* ctx, const void* W, const float* X, float* Y, uint32_t M,
                     uint32_t K) {
  gh_status st = check_gemv(ctx, W, X, Y, M, K, "gh_gemv_q8");
  if (st != GH_OK) return st;
  Q4Args a{static_cast<const uint8_t*>(W), Y};
  return launch_stream(ctx, "gh_gemv_q8", &a, plain_x(X), M, K);
}

gh_status gh_gemv_bf16(gh_context* ctx, const void* W, const float* X, float* Y, uint32_t M,
                       uint32_t K) {
  gh_status st = check_gemv(ctx, W, X, Y, M, K, "gh_gemv_bf16");
  if (st != GH_OK) return st;
  Q4Args a{static_cast<const uint8_t*>(W), Y};
  return launch_stream(ctx, "gh_gemv_bf16", &a, plain_x(X), M, K);
}

gh_status gh_gate_up_geglu_q4(gh_context* ctx, const void* Wg, const void* Wu, const float* X,
                              float* Y, uint32_t M, uint32_t K) {
  gh_status st = check_gemv(ctx, Wg, X, Y, M, K, "gh_gate_up_geglu_q4");
  if (st != GH_OK) return st;
  if (!Wu || (reinterpret_cast<uintptr_t>(Wu) & 15))
    return fail(GH_ERR_INVALID, "gh_gate_up_geglu_q4: Wu null or misaligned");
  GateUpArgs a{static_cast<const uint8_t*>(Wg), static_cast<const uint8_t*>(Wu), Y};
  return launch_stream(ctx, "gh_gateup_q4", &a, plain_x(X), M, K);
}

gh_status gh_norm_gemv(gh_context* ctx, gh_quant_mode mode, const void* W, float* Y, uint32_t M,
                       uint32_t K, const gh_xprologue* pro) {
  if (!pro) return fail(GH_ERR_INVALID, "gh_norm_gemv: prologue is null");
  if (mode != GH_QUANT_Q4 && mode != GH_QUANT_Q8 && mode != GH_QUANT_NONE)
    return fail(GH_ERR_UNSUPPORTED, "gh_norm_gemv: mode must be Q4, Q8 or NONE (bf16)");
  gh_status st = check_gemv(ctx, W, pro->x, Y, M, K, "gh_norm_gemv");
  if (st != GH_OK) return st;
  XPro p = from_abi(pro);
  if ((st = gh::check_pro(ctx, p, K, "gh_norm_gemv")) != GH_OK) return st;
  Q4Args a{static_cast<const uint8_t*>(W), Y};
  return launch_stream(ctx, gh::gemv_family(mode), &a, p, M, K);
}

gh_status gh_norm_gate_up_geglu(gh_context* ctx, gh_quant_mode mode, const void* Wg,
                                const void* Wu, float* Y, uint32_t M, uint32_t K,
                                const gh_xprologue* pro) {
  if (!pro) return fail(GH_ERR_INVALID, "gh_norm_gate_up_geglu: prologue is null");
  if (mode != GH_QUANT_Q4 && mode != GH_QUANT_Q8 && mode != GH_QUANT_NONE)
    return fail(GH_ERR_UNSUPPORTED, "gh_norm_gate_up_geglu: mode must be Q4, Q8 or NONE (bf16)");
  gh_status st = check_gemv(ctx, Wg, pro->x, Y, M, K, "gh_norm_gate_up_geglu");
  if (st != GH_OK) return st;
  if (!Wu || (reinterpret_cast<uintptr_t>(Wu) & 15))
    return fail(GH_ERR_INVALID, "gh_norm_gate_up_geglu: Wu null or misaligned");
  XPro p = from_abi(pro);
  if ((st = gh::check_pro(ctx, p, K, "gh_norm_gate_up_geglu")) != GH_OK) return st;
  GateUpArgs a{static_cast<const uint8_t*>(Wg), static_cast<const uint8_t*>(Wu), Y};
  return launch_stream(ctx, gh::gateup_family(mode), &a, p, M, K);
}

namespace {
gh_status norm_gemv_argmax(gh_context* ctx, const void* W, float* logits, uint32_t* token,
                           uint32_t M, uint32_t K, const gh_xprologue* pro, bool bf16,
                           const char* who) {
  if (!pro || !token) return fail(GH_ERR_INVALID, std::string(who) + ": null argument");
  gh_status st = check_gemv(ctx, W, pro->x, token, M, K, who);
  if (st != GH_OK) return st;
  XPro p = from_abi(pro);
  if ((st = gh::check_pro(ctx, p, K, who)) != GH_OK) return st;
  st = ctx->ensure_zeroed(&ctx->argmax_scratch, &ctx->argmax_scratch_bytes, kArgmaxScratchBytes);
  if (st != GH_OK) return st;
  uint32_t* base = static_cast<uint32_t*>(ctx->argmax_scratch);
  ArgmaxArgs a{static_cast<const uint8_t*>(W), logits, base + 64};
  return gh::launch_argmax_stream(ctx, &a, p, M, K, token, bf16);
}
}  // namespace

gh_status gh_norm_gemv_argmax_q8(gh_context* ctx, const void* W, float* logits,
                                 uint32_t* token, uint32_t M, uint32_t K,
                                 const gh_xprologue* pro) {
  return norm_gemv_argmax(ctx, W, logits, token, M, K, pro, false, "gh_norm_gemv_argmax_q8");
}

gh_status gh_norm_gemv_argmax_bf16(gh_context* ctx, const void* W, float* logits,
                                   uint32_t* token, uint32_t M, uint32_t K,
                                   const gh_xprologue* pro) {
  return norm_gemv_argmax(ctx, W, logits, token, M, K, pro, true, "gh_norm_gemv_argmax_bf16");
}

gh_status gh_rmsnorm(gh_context* ctx, const float* X, const float* W, float* Y, uint32_t dim,
                     float eps) {
  if (!ctx || !X || !W || !Y || dim == 0) return fail(GH_ERR_INVALID, "gh_rmsnorm: bad argument");
  void* args[] = {const_cast<float**>(&X), const_cast<float**>(&W), &Y, &dim, &eps};
  return ctx->launch("gh_rmsnorm_k", dim3(1), dim3(1024), 0, args);
}

gh_status gh_add_rmsnorm(gh_context* ctx, float* X, const float* R, const float* W, float* Y,
                         uint32_t dim, float eps, float scalar) {
  if (!ctx || !X || !R || !W || !Y || dim == 0)
    return fail(GH_ERR_INVALID, "gh_add_rmsnorm: bad argument");
  void* args[] = {&X, const_cast<float**>(&R), const_cast<float**>(&W), &Y, &dim, &eps, &scalar};
  return ctx->launch("gh_add_rmsnorm_k", dim3(1), dim3(1024), 0, args);
}

gh_status gh_qkv_rope(gh_context* ctx, const float* Q_in, const float* K_in, const float* V_in,
                      const float* Q_norm, const float* K_norm, float* Q_out, float* K_cache,
                      float* V_cache, const uint32_t* step_params, uint32_t num_q,
                      uint32_t num_kv, uint32_t head_dim, uint32_t rotary_dim, uint32_t k_eq_v,
                      float theta, float eps) {
  if (!ctx || !Q_in || !K_in || (!V_in && !k_eq_v) || !Q_norm || !K_norm || !Q_out || !K_cache ||
      !V_cache || !step_params)
    return fail(GH_ERR_INVALID, "gh_qkv_rope: null pointer");
  if (num_q == 0 || num_kv == 0 || head_dim == 0 || rotary_dim > head_dim || rotary_dim % 2)
    return fail(GH_ERR_INVALID, "gh_qkv_rope: bad head shape");
  if (!V_in) V_in = K_in;
  void* args[] = {const_cast<float**>(&Q_in), const_cast<float**>(&K_in),
                  const_cast<float**>(&V_in), const_cast<float**>(&Q_norm),
                  const_cast<float**>(&K_norm), &Q_out, &K_cache, &V_cache,
                  const_cast<uint32_t**>(&step_params), &num_q, &num_kv, &head_dim,
                  &rotary_dim, &k_eq_v, &theta, &eps};
  return ctx->launch("gh_qkv_rope_k", dim3(num_q + num_kv), dim3(64), 0, args);
}

}  // extern "C"

namespace gh {

// Attention launch shared by the standalone entry point and the model.
gh_status launch_attention(gh_context* ctx, const AttnLaunch& L) {
  const uint32_t G = L.args.nq / L.args.nkv;
  const uint32_t D = L.args.D;
  if (L.args.nkv == 0 || L.args.nq % L.args.nkv != 0 || G > 4)
    return fail(GH_ERR_UNSUPPORTED, "attention: query heads per kv head must be 1..4");
  if (L.args.nsplit == 0 || L.args.nsplit > 256)
    return fail(GH_ERR_UNSUPPORTED, "attention: 1..256 splits");
  const int dpl = D <= 64 ? 1 : (D <= 128 ? 2 : (D <= 256 ? 4 : 8));
  if (D > 512 || D % 4 != 0 || D % dpl != 0)
    return fail(GH_ERR_UNSUPPORTED, "attention: head_dim must be a multiple of 4 up to 512");
  void* args[] = {const_cast<AttnArgs*>(&L.args)};
  // a.run non-null: the gated forms (nothing when the layer's flag is 0)
  const bool gated = L.args.run != nullptr;
  const std::string name = std::string("gh_attn_d") + std::to_string(dpl) + (gated ? "_q_k" : "_k");
  gh_status st = ctx->launch(name, dim3(L.args.nkv * L.args.nsplit), dim3(256), 0, args);
  if (st != GH_OK) return st;
  return ctx->launch(gated ? "gh_attn_merge_q_k" : "gh_attn_merge_k", dim3(L.args.nq), dim3(256),
                     0, args);
}

namespace {
// The weight-streaming GEMM of a short batch (T <= 16, gh_pf_sgemm_* /
// gh_pf_sgateup_*): workgroups of 4 waves over 4 RGW row groups of 16 and a
// K slice of KR quant blocks.  LDS holds the slice's T activation rows (128 KR
// + 16 bytes each) and each wave's weight set rows (16 rows of SB blocks + 16
// bytes per matrix: SB = 16 for Q4/Q8, 8 for bf16).  Slices of 16 blocks and
// about one round of resident workgroups (RGW row groups per wave so that
// the grid is near the CUs' workgroup slots) measured fastest at the 12B
// shapes (16 tokens, Q4: QKV 8192 x 3840 at RGW 2, o 3840 x 4096 at 1,
// gate+up 2 x 15360 x 3840 and down 3840 x 15360 at 4); wider slices (24, 32)
// and 2-4x the workgroups were slower.  GH_PF_STREAM="kr,rgw" forces both
// (kr a multiple of 4, at most 32).  af: A is the f32 rows (Ax) and the
// kernel splits each slice itself (gh_pf_*_f_k; rs unused).
// LDS of one workgroup of the streamed GEMM: T staged token rows of a
// kr-block slice, then the set rows of each of its waves (4 waves for up to
// 16 tokens, 8 for 17-48), plus 256 bytes for its static per-token slice
// scales.
uint32_t stream_lds(gh_quant_mode mode, bool pair, uint32_t T, uint32_t kr) {
  const uint32_t block_bytes = mode == GH_QUANT_Q8 ? 36u : mode == GH_QUANT_NONE ? 64u : 20u;
  const uint32_t set_blocks = mode == GH_QUANT_NONE ? 8u : 16u;
  const uint32_t wave_bytes = 16u * (set_blocks * block_bytes + 16u);
  const uint32_t nw = T <= 16 ? 4u : 8u;
  return T * (128u * kr + 16u) + nw * (pair ? 2u : 1u) * wave_bytes + 256u;
}

// The streamed GEMM's slice width in quant blocks: 16 (or all of K); for
// more than 32 tokens, else 12 or 8 if the staged rows fit in LDS then (and
// the slices stay at 64 or fewer); 0 when none does.  Narrower slices multiply
// the planes: the bf16 gate/up pair of 40 tokens in 4-block slices (30
// planes) took the prompt from 9.9 to 14.7 ms.
uint32_t stream_kr(const gh_context* ctx, gh_quant_mode mode, bool pair, uint32_t T, uint32_t nb) {
  const uint32_t narrowest = T <= 32 ? std::min(16u, nb) : std::min(8u, nb);
  for (uint32_t kr = std::min(16u, nb); kr >= narrowest; kr -= 4)
    if (stream_lds(mode, pair, T, kr) <= ctx->max_lds && (nb + kr - 1) / kr <= 64) return kr;
  return 0;
}

gh_status launch_prefill_stream(gh_context* ctx, gh_quant_mode mode, const void* W0,
                                const void* W1, const void* Ax, const float* rs, float* C,
                                uint32_t T, uint32_t N, uint32_t K, const float** planes,
                                uint32_t* nplanes, bool af) {
  const bool pair = W1 != nullptr;
  const uint32_t nmat = pair ? 2u : 1u;
  const uint32_t nb = K / 32, cus = (uint32_t)ctx->num_cus, rgs = (N + 15) / 16;
  // waves per workgroup; 16-token groups per wave
  const uint32_t nw = T <= 16 ? 4u : 8u, tg = T <= 16 ? 1u : T <= 32 ? 2u : 3u;
  auto lds_of = [&](uint32_t kr) { return stream_lds(mode, pair, T, kr); };
  uint32_t KR = stream_kr(ctx, mode, pair, T, nb);
  if (KR == 0) return fail(GH_ERR_UNSUPPORTED, "prefill GEMM: stream slice exceeds LDS");
  const std::string kname = std::string(pair ? "gh_pf_sgateup_" : "gh_pf_sgemm_") +
                            (mode == GH_QUANT_Q8 ? "q8" : mode == GH_QUANT_NONE ? "bf16" : "q4") +
                            (af ? "_f" : "") + (tg == 3 ? "_t3_k" : tg == 2 ? "_t2_k" : "_k");
  // RGW: the grid sized for the workgroups LDS lets a CU hold, at most two.
  // Sizing it for the 3-4 a CU could hold with a one-matrix set buffer
  // (fewer row groups per wave, so shorter streams) measured slower: gate+up
  // 46.3 against 36.0 us, QKV 20.4 against 16.1 (16 tokens, f32 input, plane
  // sums included); and that buffer itself, at the same grid, 37.0 against
  // 35.1 us for the gate+up.
  const uint32_t per_cu = std::max(1u, std::min(2u, (uint32_t)(ctx->max_lds / lds_of(KR))));
  const uint32_t slots = per_cu * cus, nz16 = (nb + KR - 1) / KR;
  uint32_t RGW = (uint32_t)(((uint64_t)rgs * nz16 + (nw / 2) * slots) / (nw * (uint64_t)slots));
  RGW = std::max(1u, std::min(8u, RGW));
  if (const char* env = getenv("GH_PF_STREAM")) {
    unsigned kr = 0, rgw = 0;
    if (sscanf(env, "%u,%u", &kr, &rgw) == 2 && kr >= 4 && kr % 4 == 0 && kr <= 32 &&
        lds_of(std::min(kr, nb)) <= ctx->max_lds && rgw >= 1 && rgw <= 8) {
      KR = std::min(kr, nb);
      RGW = rgw;
    }
  }
  const uint32_t nz = (nb + KR - 1) / KR;
  if (nz > 64) return fail(GH_ERR_UNSUPPORTED, "prefill GEMM: more than 64 K slices");
  const unsigned lds = lds_of(KR);
  if (lds > ctx->max_lds) return fail(GH_ERR_UNSUPPORTED, "prefill GEMM: stream slice exceeds LDS");
  float* out = C;
  if (nz > 1) {
    const size_t need = (size_t)nz * nmat * T * N * sizeof(float);
    gh_status st = ctx->ensure_zeroed(&ctx->gemm_scratch, &ctx->gemm_scratch_bytes, need);
    if (st != GH_OK) return st;
    out = static_cast<float*>(ctx->gemm_scratch);
  }
  const void* W1a = pair ? W1 : W0;
  void* args[] = {const_cast<void**>(&Ax), const_cast<float**>(&rs), const_cast<void**>(&W0),
                  const_cast<void**>(&W1a), &out, &T, &N, &K, &KR, &RGW};
  const dim3 grid((rgs + nw * RGW - 1) / (nw * RGW), 1, nz);
  // dynamic LDS: all of it but the static slice scales' share
  gh_status st = ctx->launch(kname, grid, dim3(64 * nw), lds - 256u, args);
  if (planes) {
    *planes = nz > 1 ? out : C;
    *nplanes = nz;
  }
  if (st != GH_OK || nz == 1 || planes) return st;
  const uint64_t tn = (uint64_t)T * N;
  const unsigned rgrid = (unsigned)std::min<uint64_t>((tn + 255) / 256, 4ull * cus);
  uint32_t nzz = nz;
  void* rargs[] = {&out, &C, &T, &N, &nzz, const_cast<uint32_t*>(&nmat)};
  return ctx->launch("gh_pf_splitk_k", dim3(rgrid), dim3(256), 0, rargs);
}

// Short batches stream the weights (16-byte pieces of 4-block runs: K a
// multiple of 128, rows 16-byte aligned): up to 16 tokens, and up to 48 (bf16
// rows: 40) when the 8-wave workgroup's LDS fits (GH_PF_STREAM_MAX lowers the
// limit).  Measured on the 12B shape against the tile GEMMs, prompts of
// 33 / 40 / 48 tokens: Q4 9.3 / 9.4 / 9.5 -> 7.2 / 7.9 / 8.0 ms, Q8 (33, 48)
// 10.2 / 10.5 -> 8.4 / 9.4, bf16 9.5 / 9.6 / 9.9 -> 8.8 / 9.0 / 10.0.
bool stream_ok(const gh_context* ctx, gh_quant_mode mode, uint32_t T, uint32_t K, const void* W0,
               const void* W1) {
  uint32_t tmax = mode == GH_QUANT_NONE ? 40u : 48u;
  if (const char* env = getenv("GH_PF_STREAM_MAX")) tmax = std::min(tmax, (uint32_t)atoi(env));
  return T <= tmax && K % 128 == 0 &&
         !((reinterpret_cast<uintptr_t>(W0) | reinterpret_cast<uintptr_t>(W1 ? W1 : W0)) & 15) &&
         stream_kr(ctx, mode, W1 != nullptr, T, K / 32) != 0 &&
         getenv("GH_PF_NO_STREAM") == nullptr;
}
}  // namespace

gh_status launch_prefill_gemm_split(gh_context* ctx, gh_quant_mode mode, const void* W0,
                                    const void* W1, const void* Ax, const float* rs, float* C,
                                    uint32_t T, uint32_t N, uint32_t K, const float** planes,
                                    uint32_t* nplanes) {
  if (mode != GH_QUANT_Q4 && mode != GH_QUANT_Q8 && mode != GH_QUANT_NONE)
    return fail(GH_ERR_UNSUPPORTED, "prefill GEMM: mode must be Q4, Q8 or NONE (bf16)");
  if (!W0 || !Ax || !rs || !C || T == 0 || N == 0 || K == 0)
    return fail(GH_ERR_INVALID, "prefill GEMM: null pointer or zero size");
  if (K % 32 != 0) return fail(GH_ERR_UNSUPPORTED, "prefill GEMM: K must be a multiple of 32");
  if (K > 16384) return fail(GH_ERR_UNSUPPORTED, "prefill GEMM: K above 16384");
  // bf16 rows are read 16 bytes at a time, quantized blocks 4 bytes at a time
  const uintptr_t walign = mode == GH_QUANT_NONE ? 15 : 3;
  if ((reinterpret_cast<uintptr_t>(Ax) & 15) || (reinterpret_cast<uintptr_t>(W0) & walign) ||
      (W1 && (reinterpret_cast<uintptr_t>(W1) & walign)))
    return fail(GH_ERR_INVALID, "prefill GEMM: A halves must be 16-byte aligned, W 4-byte "
                                "(16-byte for bf16 rows)");
  const bool pair = W1 != nullptr;
  if (pair && planes) return fail(GH_ERR_INVALID, "prefill GEMM: unsummed planes of a gate/up pair");
  if (stream_ok(ctx, mode, T, K, W0, W1))
    return launch_prefill_stream(ctx, mode, W0, W1, Ax, rs, C, T, N, K, planes, nplanes, false);
  // A product without planes of 256k + 1..127 tokens (a 288-token gate+up:
  // 720 tiles, the last 240 three-quarters padding) runs as two products: the
  // multiple of 256 on the tiles, the rest as its own product (the
  // weight-streaming GEMM up to 48 tokens, tiles above).  Prompts of 272 /
  // 288 / 300 / 320 / 352 tokens: 26.8 / 26.8 / 26.9 / 27.3 / 27.6 -> 23.3 /
  // 23.9 / 24.6 / 25.1 / 26.6 ms (GH_PF_REST_MAX=n: at most n tokens).
  const uint32_t rest = T % 256;
  const uint32_t rest_max = getenv("GH_PF_REST_MAX") ? (uint32_t)atoi(getenv("GH_PF_REST_MAX")) : 127u;
  if (!planes && T > 256 && rest > 0 && rest <= rest_max &&
      getenv("GH_PF_NO_REST_SPLIT") == nullptr) {
    const uint32_t main = T - rest;
    gh_status st = launch_prefill_gemm_split(ctx, mode, W0, W1, Ax, rs, C, main, N, K, nullptr,
                                             nullptr);
    if (st != GH_OK) return st;
    const uint16_t* Ar = static_cast<const uint16_t*>(Ax) + (size_t)main * 2 * K;  // fp16 halves
    return launch_prefill_gemm_split(ctx, mode, W0, W1, Ar, rs + main, C + (size_t)main * N, rest,
                                     N, K, nullptr, nullptr);
  }
  const uint32_t cus = (uint32_t)ctx->num_cus;
  // the large tile when it still gives every CU a workgroup, or (plain
  // products of more than 64 tokens) when splitting K lifts it to that
  const uint32_t bn_big = pair ? 64 : 128;
  const uint32_t tiles_big = ((N + bn_big - 1) / bn_big) * ((T + 127) / 128);
  // A caller that takes unsummed planes also gets the split for a product
  // whose large tiles give each CU only one workgroup (the QKV projection of
  // 512 tokens: 256 tiles of 128x128, split in 2, measured 85 us against
  // 112 us as 512 tiles of 128x64).
  // From 65 tokens (one 128-row tile holds the batch): at 80 / 96 / 112 tokens
  // the QKV projection's 64x64 tiles came to exactly the CU count or more and
  // ran unsplit (86.6 us at 96 tokens against 32.4 us split at 128), and the
  // prompt took 16.4-16.8 ms against 14.2-14.6 ms this way.
  // With the 8-wave tiles this holds down to a handful of tiles: the o and
  // down projections of 65-256 tokens (30-60 tiles, split up to 17 ways)
  // measured 80 / 96 / 128 / 192-token prompts 12.30 / 12.56 / 13.08 / 19.19
  // -> 11.17 / 11.43 / 11.95 / 17.07 ms against 64x64 tiles
  // (GH_PF_BIG_SPLIT_MIN=n restores a minimum of n / 4 tiles).
  const uint32_t bs_min = getenv("GH_PF_BIG_SPLIT_MIN") ? (uint32_t)atoi(getenv("GH_PF_BIG_SPLIT_MIN")) : 1u;
  const bool big_split = !pair && T > 64 && 4 * tiles_big >= bs_min &&
                         (tiles_big < cus || (planes && tiles_big < 2 * cus)) &&
                         getenv("GH_PF_NO_BIG_SPLIT") == nullptr;
  // A Q4 gate/up pair whose 128x64 tiles give half the CUs or more but not
  // all (65-128 tokens at the 12B shape: 240 tiles) takes them with K split
  // (480 workgroups) rather than 480 unsplit 64x64 tiles: 65-128-token
  // prompts 13.0-13.5 against 14.0-14.6 ms.
  const bool pair_split = pair && mode == GH_QUANT_Q4 && T > 64 && tiles_big < cus &&
                          2 * tiles_big >= cus;
  const bool big = tiles_big >= cus || big_split || pair_split;
  // a plain product whose 128x128 tiles give each CU only one workgroup (the
  // QKV projection of 512 tokens: 256 tiles) takes 128x64 tiles, two per CU
  const uint32_t tiles_n64 = ((N + 63) / 64) * ((T + 127) / 128);
  const bool narrow = !pair && big && !big_split && tiles_big < 2 * cus && tiles_n64 >= 2 * cus &&
                      getenv("GH_PF_NO_N64") == nullptr;
  const uint32_t bm = big ? 128 : 64, bn = big ? (narrow ? 64 : bn_big) : 64;
  std::string name = std::string(pair ? "gh_pf_gateup_" : "gh_pf_gemm_") +
                     (mode == GH_QUANT_Q8 ? "q8" : mode == GH_QUANT_NONE ? "bf16" : "q4") +
                     (big ? "_m128_n" : "_m64_n") +
                     std::to_string(bn) + "_k1";

  dim3 grid((N + bn - 1) / bn, (T + bm - 1) / bm);
  // Split K when the tiles alone leave CUs idle: about two workgroups per CU,
  // at least 8 K steps per split (GH_PF_SPLIT=n forces n, 1 disables).
  const uint32_t tiles = grid.x * grid.y, nsteps = K / 32;
  uint32_t nz = 1;
  if (!big && tiles < cus) nz = std::min<uint32_t>((2 * cus + tiles - 1) / tiles, std::max(1u, nsteps / 8));
  // large tiles: as many splits as keep every workgroup resident (two per CU)
  if (big_split || pair_split) nz = std::min<uint32_t>(std::max(1u, 2 * cus / tiles), std::max(1u, nsteps / 8));
  if (const char* env = getenv("GH_PF_SPLIT")) {
    const int v = atoi(env);
    if (v >= 1 && (!big || big_split)) nz = std::min<uint32_t>((uint32_t)v, nsteps);
  }
  nz = std::min<uint32_t>(nz, 64u);
  float* out = C;
  const uint32_t nmat = pair ? 2u : 1u;
  if (nz > 1) {
    const size_t need = (size_t)nz * nmat * T * N * sizeof(float);
    gh_status st = ctx->ensure_zeroed(&ctx->gemm_scratch, &ctx->gemm_scratch_bytes, need);
    if (st != GH_OK) return st;
    out = static_cast<float*>(ctx->gemm_scratch);
    name += "_s";
    grid.z = nz;
  }
  // 128-row tiles in 8-wave workgroups (four waves per SIMD instead of two,
  // the same two tiles per CU), except a gate/up pair with more than three
  // unsplit tiles per CU (the 512-token gate+up: 317 -> 319 us Q4, 332 -> 337
  // Q8, 304 -> 307 bf16; 288-384-token prompts 1.3-1.9% faster with it, 448
  // 0.3% slower).  Measured at the 12B shapes, bit-identical: 512
  // tokens QKV 116.9 -> 113.3 us, o 64.5 -> 60.5, down 169.2 -> 163.6 (Q4;
  // Q8 and bf16 alike), 96-300-token products 7-17% faster; prompts of 128 /
  // 256 / 512 tokens 13.15 / 19.96 / 31.87 -> 12.99 / 19.89 / 31.68 ms.
  // GH_PF_W8=0/1 forces one form.
  bool w8 = big && !(pair && nz == 1 && tiles > 3 * cus);
  if (const char* env = getenv("GH_PF_W8")) w8 = big && atoi(env) != 0;
  if (w8) name += "_w8";
  gh_status st;
  if (pair) {
    void* args[] = {const_cast<void**>(&Ax), const_cast<float**>(&rs), const_cast<void**>(&W0),
                    const_cast<void**>(&W1), &out, &T, &N, &K};
    st = ctx->launch(name, grid, dim3(w8 ? 512 : 256), 0, args);
  } else {
    void* args[] = {const_cast<void**>(&Ax), const_cast<float**>(&rs), const_cast<void**>(&W0),
                    &out, &T, &N, &K};
    st = ctx->launch(name, grid, dim3(w8 ? 512 : 256), 0, args);
  }
  if (planes) {
    *planes = nz > 1 ? out : C;
    *nplanes = nz;
  }
  if (st != GH_OK || nz == 1 || planes) return st;
  const uint64_t tn = (uint64_t)T * N;
  const unsigned rgrid = (unsigned)std::min<uint64_t>((tn + 255) / 256, 4ull * cus);
  void* rargs[] = {&out, &C, &T, &N, &nz, const_cast<uint32_t*>(&nmat)};
  return ctx->launch("gh_pf_splitk_k", dim3(rgrid), dim3(256), 0, rargs);
}

gh_status launch_prefill_plane_sum(gh_context* ctx, const float* planes, float* C, uint32_t T,
                                   uint32_t N, uint32_t nplanes) {
  if (!planes || !C || T == 0 || N == 0 || nplanes == 0)
    return fail(GH_ERR_INVALID, "prefill plane sum: null pointer or zero size");
  const uint64_t tn = (uint64_t)T * N;
  const unsigned rgrid = (unsigned)std::min<uint64_t>((tn + 255) / 256, 4ull * ctx->num_cus);
  uint32_t one = 1;
  void* rargs[] = {const_cast<float**>(&planes), &C, &T, &N, &nplanes, &one};
  return ctx->launch("gh_pf_splitk_k", dim3(rgrid), dim3(256), 0, rargs);
}

// f32 A: split into fp16 hi/lo halves with a power-of-two scale per row
// (gh_pf_halves_k, once per row rather than in every tile that reads it),
// then the GEMM.
gh_status launch_prefill_gemm(gh_context* ctx, gh_quant_mode mode, const void* W0, const void* W1,
                              const float* A, float* C, uint32_t T, uint32_t N, uint32_t K,
                              const float** planes, uint32_t* nplanes) {
  if (!A || T == 0 || K == 0 || K % 32 != 0) return fail(GH_ERR_INVALID, "prefill GEMM: bad A");
  if (K > 16384) return fail(GH_ERR_UNSUPPORTED, "prefill GEMM: K above 16384");
  if (reinterpret_cast<uintptr_t>(A) & 15) return fail(GH_ERR_INVALID, "prefill GEMM: A must be 16-byte aligned");
  // the weight checks of the GEMM itself, before the halves are made
  if (mode != GH_QUANT_Q4 && mode != GH_QUANT_Q8 && mode != GH_QUANT_NONE)
    return fail(GH_ERR_UNSUPPORTED, "prefill GEMM: mode must be Q4, Q8 or NONE (bf16)");
  const uintptr_t walign = mode == GH_QUANT_NONE ? 15 : 3;
  if (!W0 || (reinterpret_cast<uintptr_t>(W0) & walign) ||
      (W1 && (reinterpret_cast<uintptr_t>(W1) & walign)))
    return fail(GH_ERR_INVALID, "prefill GEMM: W null or misaligned (4 bytes; 16 for bf16 rows)");
  if (W1 && planes) return fail(GH_ERR_INVALID, "prefill GEMM: unsummed planes of a gate/up pair");
  // a short batch's streamed GEMM splits the f32 rows as it stages them
  if (stream_ok(ctx, mode, T, K, W0, W1))
    return launch_prefill_stream(ctx, mode, W0, W1, A, nullptr, C, T, N, K, planes, nplanes, true);
  const size_t ax_bytes = (size_t)T * K * 4;  // 2 K halves per row
  gh_status st = ctx->ensure_zeroed(&ctx->half_scratch, &ctx->half_scratch_bytes,
                                    ax_bytes + (size_t)T * sizeof(float));
  if (st != GH_OK) return st;
  char* hb = static_cast<char*>(ctx->half_scratch);
  void* Ax = hb;
  float* rs = reinterpret_cast<float*>(hb + ax_bytes);
  uint32_t fmt = gh::pf_halves_format(mode);
  void* args[] = {const_cast<float**>(&A), &Ax, &rs, &K, &fmt};
  if ((st = ctx->launch("gh_pf_halves_k", dim3(T), dim3(1024), 0, args)) != GH_OK) return st;
  return launch_prefill_gemm_split(ctx, mode, W0, W1, Ax, rs, C, T, N, K, planes, nplanes);
}

gh_status fused_attn_args(gh_context* ctx, const float* Q_in, const float* K_in,
                          const float* V_in, const float* Q_norm, const float* K_norm,
                          float* K_cache, float* V_cache, const uint32_t* active_slots,
                          const uint32_t* step_params, float* out, uint32_t num_q,
                          uint32_t num_kv, uint32_t head_dim, uint32_t rotary_dim,
                          uint32_t k_eq_v, float theta, float eps, uint32_t max_slots,
                          const float* rope_table, const char* who, AttnLaunch* L,
                          size_t* part_bytes) {
  if (!ctx || !Q_in || !K_in || (!V_in && !k_eq_v) || !Q_norm || !K_norm || !K_cache ||
      !V_cache || !active_slots || !step_params || !out)
    return fail(GH_ERR_INVALID, std::string(who) + ": null pointer");
  if (num_kv == 0 || num_q % num_kv || rotary_dim > head_dim || rotary_dim % 2 || max_slots == 0)
    return fail(GH_ERR_INVALID, std::string(who) + ": bad head shape");
  *L = AttnLaunch{};
  AttnArgs& a = L->args;
  a.q = Q_in;
  a.k_in = K_in;
  a.v_in = V_in ? V_in : K_in;
  a.q_norm = Q_norm;
  a.k_norm = K_norm;
  a.k_cache = K_cache;
  a.v_cache = V_cache;
  a.active = active_slots;
  a.step = step_params;
  a.out = out;
  a.nq = num_q;
  a.nkv = num_kv;
  a.D = head_dim;
  a.rot = rotary_dim;
  a.k_eq_v = k_eq_v ? 1 : 0;
  a.fuse = 1;
  a.theta = theta;
  a.eps = eps;
  a.scale = 1.0f;  // inv_sqrt_dim = 1.0 (src/model/forward.zig:80)
  a.flags = step_params + 3;  // bit 1: the list is 0 .. S-1
  a.rope_tab = rope_table;
  a.nsplit = attention_splits(ctx, num_kv, max_slots);
  *part_bytes = (size_t)num_kv * a.nsplit * (num_q / num_kv) * (head_dim + 4) * 4;
  return GH_OK;
}

uint32_t attention_splits(const gh_context* ctx, uint32_t nkv, uint32_t max_slots) {
  // The grid's splits per kv head: enough for a full cache at about
  // ATT_SLOTS_PER_SPLIT slots each (8 per wave), at most ~one workgroup per
  // CU.  The kernels run only attn_live_splits(grid, S) of them, so the count
  // at a given S does not depend on the capacity (20 at S = 544 for any
  // capacity of 560 slots or more).  GH_ATTN_SPLITS sets the grid's count.
  uint32_t ns = std::max<uint32_t>(1u, (max_slots + ATT_SLOTS_PER_SPLIT - 1) / ATT_SLOTS_PER_SPLIT);
  ns = std::min<uint32_t>(ns, std::max<uint32_t>(1u, (uint32_t)ctx->num_cus / std::max(1u, nkv)));
  if (const char* env = getenv("GH_ATTN_SPLITS")) {
    int v = atoi(env);
    if (v >= 1 && v <= 256) ns = (uint32_t)v;
  }
  return std::max<uint32_t>(1u, std::min<uint32_t>(ns, 256u));
}

}  // namespace gh

extern "C" {

gh_status gh_decode_attn(gh_context* ctx, const float* Q, const float* K_cache,
                         const float* V_cache, const uint32_t* active_slots, float* out,
                         const uint32_t* step_params, uint32_t head_dim, uint32_t kv_dim,
                         uint32_t gqa_ratio, float inv_sqrt_dim, uint32_t num_q_heads) {
  if (!ctx || !Q || !K_cache || !V_cache || !active_slots || !out || !step_params)
    return fail(GH_ERR_INVALID, "gh_decode_attn: null pointer");
  if (gqa_ratio == 0 || num_q_heads % gqa_ratio || head_dim == 0 ||
      kv_dim != (num_q_heads / gqa_ratio) * head_dim)
    return fail(GH_ERR_INVALID, "gh_decode_attn: kv_dim must equal (num_q / gqa) * head_dim");
  gh::AttnLaunch L{};
  AttnArgs& a = L.args;
  a.q = Q;
  // unused without the fused prologue, but every row pointer the kernel
  // loads through must be valid memory: the query rows stand in
  a.k_in = a.v_in = a.q_norm = a.k_norm = Q;
  a.k_cache = const_cast<float*>(K_cache);
  a.v_cache = const_cast<float*>(V_cache);
  a.active = active_slots;
  a.step = step_params;
  a.out = out;
  a.nq = num_q_heads;
  a.nkv = num_q_heads / gqa_ratio;
  a.D = head_dim;
  a.rot = 0;
  a.fuse = 0;
  a.scale = inv_sqrt_dim;
  a.flags = step_params + 3;  // bit 1: the list is 0 .. S-1
  a.nsplit = gh::attention_splits(ctx, a.nkv, 1024);
  const size_t part_bytes = (size_t)a.nkv * a.nsplit * gqa_ratio * (head_dim + 4) * 4;
  gh_status st = ctx->ensure_zeroed(&ctx->attn_scratch, &ctx->attn_scratch_bytes, part_bytes);
  if (st != GH_OK) return st;
  a.part = static_cast<float*>(ctx->attn_scratch);
  return gh::launch_attention(ctx, L);
}

gh_status gh_qkv_rope_attn(gh_context* ctx, const float* Q_in, const float* K_in,
                           const float* V_in, const float* Q_norm, const float* K_norm,
                           float* K_cache, float* V_cache, const uint32_t* active_slots,
                           const uint32_t* step_params, float* out, uint32_t num_q,
                           uint32_t num_kv, uint32_t head_dim, uint32_t rotary_dim,
                           uint32_t k_eq_v, float theta, float eps, uint32_t max_slots,
                           const float* rope_table) {
  gh::AttnLaunch L{};
  size_t part_bytes = 0;
  gh_status st = gh::fused_attn_args(ctx, Q_in, K_in, V_in, Q_norm, K_norm, K_cache, V_cache,
                                     active_slots, step_params, out, num_q, num_kv, head_dim,
                                     rotary_dim, k_eq_v, theta, eps, max_slots, rope_table,
                                     "gh_qkv_rope_attn", &L, &part_bytes);
  if (st != GH_OK) return st;
  st = ctx->ensure_zeroed(&ctx->attn_scratch, &ctx->attn_scratch_bytes, part_bytes);
  if (st != GH_OK) return st;
  L.args.part = static_cast<float*>(ctx->attn_scratch);
  return gh::launch_attention(ctx, L);
}

gh_status gh_rope_table(gh_context* ctx, const uint32_t* step_params, uint32_t rotary_dim,
                        float theta, float* table) {
  if (!ctx || !step_params || !table) return fail(GH_ERR_INVALID, "gh_rope_table: null pointer");
  if (rotary_dim == 0 || rotary_dim % 2 || rotary_dim > 512)
    return fail(GH_ERR_INVALID, "gh_rope_table: rotary_dim must be even, 2..512");
  void* args[] = {const_cast<uint32_t**>(&step_params), &rotary_dim, &theta, &table};
  return ctx->launch("gh_rope_table_k", dim3(1), dim3(256), 0, args);
}

gh_status gh_prefill_gemm(gh_context* ctx, gh_quant_mode mode, const void* W, const float* A,
                          float* C, uint32_t T, uint32_t N, uint32_t K) {
  if (!ctx) return fail(GH_ERR_INVALID, "gh_prefill_gemm: ctx is null");
  if (!W) return fail(GH_ERR_INVALID, "gh_prefill_gemm: W is null");
  return gh::launch_prefill_gemm(ctx, mode, W, nullptr, A, C, T, N, K);
}

gh_status gh_prefill_gate_up_geglu(gh_context* ctx, gh_quant_mode mode, const void* Wg,
                                   const void* Wu, const float* A, float* act, uint32_t T,
                                   uint32_t N, uint32_t K) {
  if (!ctx) return fail(GH_ERR_INVALID, "gh_prefill_gate_up_geglu: ctx is null");
  if (!Wg || !Wu) return fail(GH_ERR_INVALID, "gh_prefill_gate_up_geglu: null weights");
  return gh::launch_prefill_gemm(ctx, mode, Wg, Wu, A, act, T, N, K);
}

gh_status gh_argmax(gh_context* ctx, const float* logits, uint32_t* out_token, uint32_t vocab) {
  if (!ctx || !logits || !out_token || vocab == 0)
    return fail(GH_ERR_INVALID, "gh_argmax: bad argument");
  const uint32_t grid = std::min<uint32_t>(256u, (vocab + 1023) / 1024);
  gh_status st = ctx->ensure_zeroed(&ctx->argmax_scratch, &ctx->argmax_scratch_bytes,
                                    kArgmaxScratchBytes);
  if (st != GH_OK) return st;
  uint32_t* partial = static_cast<uint32_t*>(ctx->argmax_scratch) + 64;
  void* args[] = {const_cast<float**>(&logits), &vocab, &partial};
  gh_status st2 = ctx->launch("gh_argmax_k", dim3(grid), dim3(256), 0, args);
  if (st2 != GH_OK) return st2;
  uint32_t n = grid;
  void* fargs[] = {&partial, &n, &out_token};
  return ctx->launch("gh_argmax_final_k", dim3(1), dim3(256), 0, fargs);
}

}  // extern "C"
