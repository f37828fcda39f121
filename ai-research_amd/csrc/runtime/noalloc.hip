// noalloc.hip -- the allocation-free entry point: gh_qkv_rope_attn with its
// split partials in a fixed device array instead of context scratch that the
// first call allocates.  For callers that cannot allocate (code under HIP
// graph capture, serving loops that forbid hipMalloc).
//
// The array is a file-scope __device__ variable of this library's own gfx950
// code object; each device holds its own copy until the process ends.  In
// host code its name is only a stand-in: the device address comes from
// hipGetSymbolAddress, once per device with that device current (at
// gh_context_init), and only that address is passed to the kernels.
//
// Every call on one device shares that device's array and leaves the last
// call's partials in it: calls that overlap on one device (two streams, two
// threads) race.  Nothing needs clearing between calls, because every split
// writes its whole partial record before the merge kernel reads it.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "runtime.hpp"

namespace {
constexpr size_t kScratchFloats = 262144;  // 1 MiB of split partials
constexpr int kMaxDevices = 64;
float* g_scratch[kMaxDevices] = {};  // per-device address of `scratch`
std::string g_setup_error;           // why a device has no address
std::mutex g_scratch_mu;
}  // namespace

static __device__ __align__(256) float scratch[kScratchFloats];

namespace gh {

// A failure is kept in g_setup_error only, for the entry point to report: the
// caller (gh_context_init) succeeds regardless, so the thread's last-error
// message is left as it was.
gh_status noalloc_setup(int device) {
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (device < 0 || device >= kMaxDevices) {
    g_setup_error = "device ordinal above 63";
    return GH_ERR_UNSUPPORTED;
  }
  if (g_scratch[device]) return GH_OK;
  void* p = nullptr;
  hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p) {
    g_setup_error = std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e);
    return GH_ERR_HIP;
  }
  g_scratch[device] = static_cast<float*>(p);
  return GH_OK;
}

}  // namespace gh

extern "C" gh_status gh_qkv_rope_attn_noalloc(
    gh_context* ctx, const float* Q_in, const float* K_in, const float* V_in,
    const float* Q_norm, const float* K_norm, float* K_cache, float* V_cache,
    const uint32_t* active_slots, const uint32_t* step_params, float* out, uint32_t num_q,
    uint32_t num_kv, uint32_t head_dim, uint32_t rotary_dim, uint32_t k_eq_v, float theta,
    float eps, uint32_t max_slots, const float* rope_table) {
  gh::AttnLaunch L{};
  size_t part_bytes = 0;
  gh_status st = gh::fused_attn_args(ctx, Q_in, K_in, V_in, Q_norm, K_norm, K_cache, V_cache,
                                     active_slots, step_params, out, num_q, num_kv, head_dim,
                                     rotary_dim, k_eq_v, theta, eps, max_slots, rope_table,
                                     "gh_qkv_rope_attn_noalloc", &L, &part_bytes);
  if (st != GH_OK) return st;
  if (part_bytes > kScratchFloats * sizeof(float))
    return gh::fail(GH_ERR_UNSUPPORTED,
                    "gh_qkv_rope_attn_noalloc: the split partials need " +
                        std::to_string(part_bytes) + " bytes, above the fixed 1 MiB scratch "
                        "(num_kv * splits * (num_q / num_kv) * (head_dim + 4) * 4)");
  float* part = nullptr;
  std::string why;
  {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (ctx->device >= 0 && ctx->device < kMaxDevices) part = g_scratch[ctx->device];
    why = g_setup_error;
  }
  if (!part)
    return gh::fail(GH_ERR_HIP, "gh_qkv_rope_attn_noalloc: the context's device has no scratch "
                                "address (set up by gh_context_init): " + why);
  L.args.part = part;
  return gh::launch_attention(ctx, L);
}
