// attn_args.h -- kernel argument block of the split-K decode attention,
// shared by the gfx950 kernel and the host launcher (passed by value).
#pragma once
#include <stdint.h>

// Decode attention splits: the grid holds nsplit splits per kv head (sized
// from the cache capacity), and the ones that run are about one per this
// many active slots, at most nsplit (attn_live_splits); the others exit at
// once.  At S = 544 (the steady context of a 32 + 512 ring) that is 20
// splits of 28 slots.
#define ATT_SLOTS_PER_SPLIT 28u

static inline
#ifdef __HIPCC__
    __host__ __device__
#endif
    uint32_t
    attn_live_splits(uint32_t nsplit, uint32_t S) {
  const uint32_t want = (S + ATT_SLOTS_PER_SPLIT - 1) / ATT_SLOTS_PER_SPLIT;
  return want < 1u ? 1u : (want < nsplit ? want : nsplit);
}

struct AttnArgs {
  const float* q;          // [nq][D]: raw projections when fuse, else normalised + roped
  const float* k_in;       // fuse: raw k [nkv][D]
  const float* v_in;       // fuse: raw v [nkv][D]
  const float* q_norm;     // fuse: [D]
  const float* k_norm;     // fuse: [D]
  float* k_cache;          // [slots][nkv * D]
  float* v_cache;
  const uint32_t* active;  // [S] slot numbers (src/ring_buffer.zig getActiveSlots)
  const uint32_t* step;    // {clock, slot_idx, S, 0}
  float* part;             // [nkv][nsplit][G][D + 4] split partials (o, m, l, pad);
                           // decode: splits >= attn_live_splits(nsplit, S) unused
  float* out;              // [nq][D], written by the merge kernel
  uint32_t nq, nkv, D, rot, k_eq_v, nsplit, fuse;
  float theta, eps, scale;
  // batched prefill (gh_pf_* kernels): token t of the batch reads its q at
  // q + t * q_stride, its active list at active + t * active_stride (length
  // n_active[t]), and writes its output at out_rows + t * out_stride.
  const uint32_t* n_active;
  float* out_rows;
  uint32_t q_stride, active_stride, out_stride;
  // grouped prefill (gh_pf_attn_g_*): tokens in the batch; active/n_active
  // then hold one union list per group of consecutive tokens
  uint32_t n_tokens;
  // decode: *flags bit 1 (value 2) set means the active list is 0 .. S-1, so
  // slot i is i and the list need not be read (null: read the list)
  const uint32_t* flags;
  // decode, fused: cos[ROPE_TAB_HALF] then sin[ROPE_TAB_HALF] of this
  // token's angles for this layer's (rot, theta) (null: computed in-kernel)
  const float* rope_tab;
  // layer gating: when non-null and *run == 0 the launch does nothing
  const uint32_t* run;
  // batched prefill, gh_pf_qkv_rope4_k: the [q|k|v] rows as nplanes unsummed
  // K-split planes of the QKV GEMM (plane p of token t at
  // q_planes + p * plane_stride + t * q_stride), summed in plane order while
  // loading; the roped q rows go to q.  nplanes 0: the rows are q itself.
  const float* q_planes;
  uint32_t nplanes;
  uint64_t plane_stride;
};
