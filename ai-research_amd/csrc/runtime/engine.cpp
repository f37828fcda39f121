// engine.cpp -- kernel-level entry points, the counterpart of GpuEngine's
// record* helpers (src/gpu/kernels.zig:80-142): shape checks, launch-shape
// selection, and the launch on the context stream.
#include <stdlib.h>

#include <string>

#include "runtime.hpp"

using gh::fail;

namespace {

struct GemvCfg {
  int tpr, rpt;
};

// Lanes per row team: the smallest power of two (8..64) covering the row's
// 4-block groups, so one pass over the groups needs no second iteration
// unless a row has more than 64 groups.  Rows per lane: 2 when that still
// leaves >= 2 workgroups per CU, else 1.
GemvCfg pick_gemv(const gh_context* ctx, uint32_t M, uint32_t K) {
  const uint32_t ng = K / 128;
  int tpr = 8;
  while (tpr < 64 && (uint32_t)tpr < ng) tpr <<= 1;
  const uint32_t teams = 256 / tpr;
  int rpt = (M / (teams * 2) >= (uint32_t)ctx->num_cus * 2) ? 2 : 1;
  if (const char* env = getenv("GH_GEMV_CFG")) {  // tuning override "tpr,rpt"
    int t = 0, r = 0;
    if (sscanf(env, "%d,%d", &t, &r) == 2 && (t == 8 || t == 16 || t == 32 || t == 64) &&
        (r == 1 || r == 2 || r == 4)) {
      tpr = t;
      rpt = r;
    }
  }
  return {tpr, rpt};
}

unsigned x_lds_bytes(uint32_t K) { return (K / 128) * 132 * 4 + (K / 32) * 4; }

gh_status check_gemv(const gh_context* ctx, const void* W, const float* X, const float* Y,
                     uint32_t M, uint32_t K, const char* who) {
  if (!ctx || !W || !X || !Y) return fail(GH_ERR_INVALID, std::string(who) + ": null pointer");
  if (M == 0 || K == 0) return fail(GH_ERR_INVALID, std::string(who) + ": M or K is zero");
  if (K % 128 != 0)
    return fail(GH_ERR_UNSUPPORTED, std::string(who) + ": K must be a multiple of 128");
  if ((reinterpret_cast<uintptr_t>(W) & 15) || (reinterpret_cast<uintptr_t>(X) & 15))
    return fail(GH_ERR_INVALID, std::string(who) + ": W and X must be 16-byte aligned");
  if (x_lds_bytes(K) > ctx->max_lds)
    return fail(GH_ERR_UNSUPPORTED, std::string(who) + ": K too large for the LDS staging of x");
  return GH_OK;
}

gh_status launch_gemv(gh_context* ctx, const char* family, void** args, uint32_t M, uint32_t K) {
  GemvCfg c = pick_gemv(ctx, M, K);
  const uint32_t rows_per_wg = (256 / c.tpr) * c.rpt;
  const unsigned grid = (M + rows_per_wg - 1) / rows_per_wg;
  std::string name = std::string(family) + "_t" + std::to_string(c.tpr) + "_r" + std::to_string(c.rpt);
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
