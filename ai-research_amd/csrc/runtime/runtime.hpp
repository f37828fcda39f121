// runtime.hpp -- internal C++ side of the C ABI (not installed).
#pragma once
#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "gemma_hip.h"

struct gh_context {
  int device = 0;
  hipStream_t stream = nullptr;
  char name[256] = {0};
  int num_cus = 0;
  size_t max_lds = 0;
  std::vector<hipModule_t> modules;
  // Scratch of the standalone split-K attention (split partials) and argmax
  // (partials plus a last-block counter that every launch leaves at zero)
  // entry points, zero-filled when (re)allocated.
  void* attn_scratch = nullptr;
  size_t attn_scratch_bytes = 0;
  void* argmax_scratch = nullptr;
  size_t argmax_scratch_bytes = 0;
  void* gemm_scratch = nullptr;  // split-K partial planes of the prefill GEMM
  size_t gemm_scratch_bytes = 0;
  void* half_scratch = nullptr;  // the prefill GEMM's A operand: fp16 hi/lo halves, row scales
  size_t half_scratch_bytes = 0;
  gh_status ensure_zeroed(void** buf, size_t* have, size_t need);
  std::unordered_map<std::string, hipFunction_t> fns;
  std::mutex mu;

  gh_status load(const char* dir);
  hipFunction_t fn(const std::string& name);
  gh_status launch(const std::string& name, dim3 grid, dim3 block, unsigned lds, void** args);
  // Workgroups of `block` threads one CU holds at once (registers and LDS);
  // 0 when the kernel is missing.
  int occupancy(const std::string& name, int block, unsigned lds);
  std::unordered_map<std::string, int> occ;
  ~gh_context();
};

#include "../common/attn_args.h"
#include "../common/stream_args.h"

namespace gh {
using Context = gh_context;
struct AttnLaunch {
  AttnArgs args;
};
gh_status launch_attention(gh_context* ctx, const AttnLaunch& L);
// Row-stream GEMV launch (gemv.hip); family = gh_gemv_q4, gh_gemv_q8,
// gh_gateup_q4, gh_gateup_q8 or gh_argmax_q8.  The kernels take the
// argument block's members as separate parameters, in member order.
// run non-null: the gated form (a layer of the gated decode graph), which
// does nothing when *run == 0.
gh_status launch_stream(gh_context* ctx, const char* family, std::vector<void*> fmt_params,
                        const XPro& xp, uint32_t M, uint32_t K, const uint32_t* run = nullptr);
inline gh_status launch_stream(gh_context* ctx, const char* family, Q4Args* a, const XPro& xp,
                               uint32_t M, uint32_t K, const uint32_t* run = nullptr) {
  return launch_stream(ctx, family, {&a->W, &a->Y}, xp, M, K, run);
}
inline gh_status launch_stream(gh_context* ctx, const char* family, GateUpArgs* a,
                               const XPro& xp, uint32_t M, uint32_t K,
                               const uint32_t* run = nullptr) {
  return launch_stream(ctx, family, {&a->Wg, &a->Wu, &a->Y}, xp, M, K, run);
}
// The fused LM-head stream (family gh_argmax_q8, or gh_argmax_bf16 for the
// bf16 head) followed by the reduction of its block partials to the token.
gh_status launch_argmax_stream(gh_context* ctx, ArgmaxArgs* a, const XPro& xp, uint32_t M,
                               uint32_t K, uint32_t* token, bool bf16 = false);
// Stream family names of a weight mode (Q4_0, Q8_0 or bf16 rows).
const char* gemv_family(gh_quant_mode mode);
const char* gateup_family(gh_quant_mode mode);
// Kernel name and persistent grid of one row-stream launch.
struct StreamShape {
  std::string name;
  unsigned grid = 0, lds = 0, nt = 256;
};
// var: "" x as given, "n" normed prologue (modes 1, 2), "g" a gated layer's
// input and gate (mode 4)
gh_status stream_shape(gh_context* ctx, const char* family, const char* var, uint32_t M,
                       uint32_t K, StreamShape* out);
inline gh_status stream_shape(gh_context* ctx, const char* family, bool normed, uint32_t M,
                              uint32_t K, StreamShape* out) {
  return stream_shape(ctx, family, normed ? "n" : "", M, K, out);
}
uint32_t attention_splits(const gh_context* ctx, uint32_t nkv, uint32_t max_slots);
// Argument checks and the launch block of the fused q/k norm + RoPE + cache
// write + split-K attention (gh_qkv_rope_attn and its allocation-free
// variant); the caller supplies the split partials (*part_bytes bytes).
gh_status fused_attn_args(gh_context* ctx, const float* Q_in, const float* K_in,
                          const float* V_in, const float* Q_norm, const float* K_norm,
                          float* K_cache, float* V_cache, const uint32_t* active_slots,
                          const uint32_t* step_params, float* out, uint32_t num_q,
                          uint32_t num_kv, uint32_t head_dim, uint32_t rotary_dim,
                          uint32_t k_eq_v, float theta, float eps, uint32_t max_slots,
                          const float* rope_table, const char* who, AttnLaunch* L,
                          size_t* part_bytes);
// Prefill MFMA GEMM (prefill.hip): C [T][N] = A [T][K] . deq(W0)^T, or with
// W1, C = gelu_tanh(A . deq(W0)^T) * (A . deq(W1)^T); A and C f32.
// A single product (W1 null) may leave a K split unsummed: with planes
// given, *planes/*nplanes receive the partial planes ([nplanes][T][N] f32, in
// the context's GEMM scratch, valid until the next split GEMM) and C is not
// written; an unsplit product writes C and returns (C, 1).
gh_status launch_prefill_gemm(gh_context* ctx, gh_quant_mode mode, const void* W0, const void* W1,
                              const float* A, float* C, uint32_t T, uint32_t N, uint32_t K,
                              const float** planes = nullptr, uint32_t* nplanes = nullptr);
// The same with A given as its fp16 hi/lo halves Ax ([T][2K], the hi and lo
// halves of each 32-element block side by side) and row scales rs
// (A = rs[t] (hi + lo)), as gh_pf_norm_k / gh_pf_halves_k write them.
gh_status launch_prefill_gemm_split(gh_context* ctx, gh_quant_mode mode, const void* W0,
                                    const void* W1, const void* Ax, const float* rs, float* C,
                                    uint32_t T, uint32_t N, uint32_t K,
                                    const float** planes = nullptr, uint32_t* nplanes = nullptr);
// C [T][N] = the sum of nplanes K-split planes ([nplanes][T][N]) in plane
// order (gh_pf_splitk_k, spread over the CUs).
gh_status launch_prefill_plane_sum(gh_context* ctx, const float* planes, float* C, uint32_t T,
                                   uint32_t N, uint32_t nplanes);
// The A-operand halves a prefill GEMM of this weight mode reads (gh_pf_norm_k
// and gh_pf_halves_k): 1 = fp16 in the Q4 unpacking's K order (Q4_0),
// 0 = fp16 in K order (Q8_0), 2 = bf16 in K order (bf16 rows).
inline uint32_t pf_halves_format(gh_quant_mode mode) {
  return mode == GH_QUANT_Q4 ? 1u : mode == GH_QUANT_NONE ? 2u : 0u;
}
// Resolves the allocation-free entry point's device scratch for `device`
// (noalloc.hip); called by gh_context_init with that device current.
gh_status noalloc_setup(int device);
// Internal helpers of the host ring (ring.cpp).
gh_ring* ring_clone(const gh_ring* r);
void ring_state(const gh_ring* r, uint32_t layer, uint32_t* clocks, uint32_t* flags, uint32_t n);
gh_status fail(gh_status st, const std::string& msg);
gh_status hip_fail(hipError_t e, const char* what);
}  // namespace gh
