// engine.cpp -- kernel-level entry points, the counterpart of GpuEngine's
// record* helpers (src/gpu/kernels.zig:80-142): shape checks, launch-shape
// selection, and the launch on the context stream.
#include <stdlib.h>

#include <string>

#include "runtime.hpp"

using gh::fail;

namespace {

struct GemvCfg {
  int tpr, gpl, wgs_per_cu, depth;
};

unsigned x_lds_bytes(uint32_t K);

// Lanes per row team (TPR) and 4-block groups per lane per row (GPL) with
// TPR * GPL >= the row's group count and the least idle lanes; then a
// persistent grid of wgs_per_cu workgroups per CU (bounded by LDS).
GemvCfg pick_gemv(const gh_context* ctx, uint32_t M, uint32_t K) {
  const uint32_t ng = K / 128;
  static const int kT[] = {8, 16, 32, 64};
  int best_t = 64, best_g = 4;
  uint32_t best_waste = ~0u;
  for (int g : {1, 2, 4}) {
    for (int t : kT) {
      if ((uint32_t)(t * g) < ng) continue;
      if (t == 8 && g == 4) continue;
      const uint32_t waste = t * g - ng;
      if (waste < best_waste || (waste == best_waste && t > best_t)) {
        best_waste = waste;
        best_t = t;
        best_g = g;
      }
    }
    if (best_waste != ~0u) break;  // prefer one group per lane per row
  }
  GemvCfg c{best_t, best_g, 4, 3};
  if (const char* env = getenv("GH_GEMV_CFG")) {  // tuning override "tpr,gpl,wgs_per_cu,depth"
    int t = 0, g = 0, w = 0, d = 0;
    if (sscanf(env, "%d,%d,%d,%d", &t, &g, &w, &d) == 4 && (t == 8 || t == 16 || t == 32 || t == 64) &&
        (g == 1 || g == 2 || g == 4) && !(t == 8 && g == 4) && w >= 1 && w <= 32 &&
        (uint32_t)(t * g) >= ng && d >= 2 && d <= 4) {
      c = {t, g, w, d};
    }
  }
  const unsigned lds_cap = (unsigned)(ctx->max_lds / std::max(1u, x_lds_bytes(K)));
  c.wgs_per_cu = std::max(1, std::min<int>(c.wgs_per_cu, (int)lds_cap));
  (void)M;
  return c;
}

unsigned x_lds_bytes(uint32_t K) { return (K / 128) * 132 * 4 + (K / 32) * 4; }

gh_status check_gemv(const gh_context* ctx, const void* W, const float* X, const float* Y,
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

gh_status launch_gemv(gh_context* ctx, const char* family, void** args, uint32_t M, uint32_t K) {
  GemvCfg c = pick_gemv(ctx, M, K);
  const uint32_t teams_per_wg = 256 / c.tpr;
  const uint32_t max_grid = (M + teams_per_wg - 1) / teams_per_wg;
  const unsigned grid = std::min<uint32_t>(max_grid, (uint32_t)ctx->num_cus * c.wgs_per_cu);
  std::string name = std::string(family) + "_t" + std::to_string(c.tpr) + "_g" +
                     std::to_string(c.gpl) + "_d" + std::to_string(c.depth);
  return ctx->launch(name, dim3(grid), dim3(256), x_lds_bytes(K), args);
}

}  // namespace

extern "C" {

gh_status gh_gemv_q4(gh_context* ctx, const void* W, const float* X, float* Y, uint32_t M,
                     uint32_t K) {
  gh_status st = check_gemv(ctx, W, X, Y, M, K, "gh_gemv_q4");
  if (st != GH_OK) return st;
  void* args[] = {const_cast<void**>(&W), const_cast<float**>(&X), &Y, &M, &K};
  return launch_gemv(ctx, "gh_gemv_q4", args, M, K);
}

gh_status gh_gemv_q8(gh_context* ctx, const void* W, const float* X, float* Y, uint32_t M,
                     uint32_t K) {
  gh_status st = check_gemv(ctx, W, X, Y, M, K, "gh_gemv_q8");
  if (st != GH_OK) return st;
  void* args[] = {const_cast<void**>(&W), const_cast<float**>(&X), &Y, &M, &K};
  return launch_gemv(ctx, "gh_gemv_q8", args, M, K);
}

gh_status gh_gate_up_geglu_q4(gh_context* ctx, const void* Wg, const void* Wu, const float* X,
                              float* Y, uint32_t M, uint32_t K) {
  gh_status st = check_gemv(ctx, Wg, X, Y, M, K, "gh_gate_up_geglu_q4");
  if (st != GH_OK) return st;
  if (!Wu || (reinterpret_cast<uintptr_t>(Wu) & 15))
    return fail(GH_ERR_INVALID, "gh_gate_up_geglu_q4: Wu null or misaligned");
  void* args[] = {const_cast<void**>(&Wg), const_cast<void**>(&Wu), const_cast<float**>(&X), &Y,
                  &M, &K};
  return launch_gemv(ctx, "gh_gateup_q4", args, M, K);
}

}  // extern "C"
