// attn.hip -- per-head Q/K RMSNorm + partial RoPE + ring-cache write, and
// split-K GQA decode attention over the active ring slots, for gfx950.
//
// Semantics (scale 1.0, no 1/sqrt(d); split-half RoPE on the first rot dims):
//   shaders/qkv_rope.wgsl:25-180, src/model/forward.zig:125-143,
//   src/kernels.zig:46-61,132-150            (norm + RoPE + cache write)
//   shaders/decode_attn.wgsl:19-108, src/model/forward.zig:77-104
//                                             (softmax(q . K[s]) . V[s])
// Layout: K/V caches [slot][kv_heads * D] f32 per layer (ring_buffer.zig
// slots), active slot list u32[S], step params u32 {clock, slot_idx, S, 0}
// read on the device like the reference's Step_params buffer.
//
// Attention design: one workgroup per (kv head, split of the active list),
// then a small merge kernel.  The G = nq / nkv query heads of a kv head share
// every K/V load (GQA bytes are read once).  A wavefront owns all D dims of a
// slot (one 16-byte load per lane per K or V row for D = 256) and walks its
// slots in tiles: a tile's loads go out together, its scores are reduced
// together (DPP inside rows of 16 lanes), and the online softmax is updated
// once per tile.  Waves merge through LDS; each split writes (o, m, l); the
// merge kernel combines the splits in split order, so the result does not
// depend on scheduling.
//
// Batched prefill: gh_pf_qkv_rope_k (norm + RoPE + cache write for T tokens),
// then one of three attention kernels, chosen by the host: gh_pf_attn_m_k
// (matrix cores, head_dim 256: 16 query columns of consecutive tokens per
// workgroup over the union of their active lists), gh_pf_attn_g_d*_k (4
// tokens per workgroup on the vector ALUs), gh_pf_attn_d*_k (one token per
// workgroup, attn_split over its own list, or over one of a.nsplit shares of
// a long list, combined by gh_pf_attn_merge_k).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../common/rope.h"

#define ATT_NT 256
#define ATT_WAVES (ATT_NT / 64)
#define MAX_D 512
#define MAX_G 4
#define MAX_SPLIT 256

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// RMS of one head (in: global, D floats) computed by one wavefront; returns
// 1 / sqrt(mean(x^2) + eps) as src/kernels.zig:50 does.
__device__ __forceinline__ float head_inv_rms(const float* __restrict__ in, uint32_t D, float eps,
                                              uint32_t lane) {
  float ss = 0.f;
  for (uint32_t d = lane; d < D; d += 64) ss += in[d] * in[d];
  ss = wave_sum(ss);
  return 1.0f / sqrtf(ss / (float)D + eps);
}

// out = RoPE_partial(in * inv * w) (w == nullptr: unit weight), one wavefront.
// Pairs (i, i + rot/2) for i < rot/2 rotate by clock * theta^(-2i/rot);
// dims >= rot are only normalised.  out may alias in (each pair is read and
// written by the same lane).
__device__ __forceinline__ void norm_rope_head(const float* in, const float* __restrict__ w,
                                               float* out, uint32_t D, uint32_t rot, float theta,
                                               float inv, uint32_t clock, uint32_t lane) {
  const uint32_t half = rot / 2;
  for (uint32_t i = lane; i < half; i += 64) {
    const float w0 = w ? w[i] : 1.0f, w1 = w ? w[i + half] : 1.0f;
    const float v0 = in[i] * inv * w0;
    const float v1 = in[i + half] * inv * w1;
    const float freq = 1.0f / powf(theta, (2.0f * (float)i) / (float)rot);
    const float ang = (float)clock * freq;
    const float c = cosf(ang), s = sinf(ang);
    out[i] = v0 * c - v1 * s;
    out[i + half] = v0 * s + v1 * c;
  }
  for (uint32_t d = rot + lane; d < D; d += 64) out[d] = in[d] * inv * (w ? w[d] : 1.0f);
}

// ---------------------------------------------------------------------------
// qkv_rope (shaders/qkv_rope.wgsl): one wavefront per head; heads [0, nq) are
// query heads (normalised + roped into q_out, which may be q_in), heads
// [nq, nq + nkv) write K/V of the current token into the caches at
// step[1] * kv_dim.
// ---------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(64) void gh_qkv_rope_k(
    const float* q_in, const float* __restrict__ k_in, const float* __restrict__ v_in,
    const float* __restrict__ q_norm, const float* __restrict__ k_norm, float* q_out,
    float* __restrict__ k_cache, float* __restrict__ v_cache, const uint32_t* __restrict__ step,
    uint32_t nq, uint32_t nkv, uint32_t D, uint32_t rot, uint32_t k_eq_v, float theta, float eps) {
  const uint32_t h = blockIdx.x, lane = threadIdx.x;
  const uint32_t clock = step[0], slot = step[1];
  if (h < nq) {
    const float* in = q_in + (size_t)h * D;
    const float inv = head_inv_rms(in, D, eps, lane);
    norm_rope_head(in, q_norm, q_out + (size_t)h * D, D, rot, theta, inv, clock, lane);
    return;
  }
  const uint32_t kh = h - nq;
  if (kh >= nkv) return;
  const size_t kv_dim = (size_t)nkv * D;
  const float* kin = k_in + (size_t)kh * D;
  const float* vin = (k_eq_v ? k_in : v_in) + (size_t)kh * D;
  float* kc = k_cache + (size_t)slot * kv_dim + (size_t)kh * D;
  float* vc = v_cache + (size_t)slot * kv_dim + (size_t)kh * D;
  const float kinv = head_inv_rms(kin, D, eps, lane);
  norm_rope_head(kin, k_norm, kc, D, rot, theta, kinv, clock, lane);
  const float vinv = head_inv_rms(vin, D, eps, lane);
  for (uint32_t d = lane; d < D; d += 64) vc[d] = vin[d] * vinv;
}

// ---------------------------------------------------------------------------
// split-K decode attention
// ---------------------------------------------------------------------------
#include "../common/attn_args.h"

// Full-wavefront sum with every lane receiving the same, bit-identical total:
// DPP butterflies inside each row of 16 lanes (xor 1, xor 2, half-row
// mirror, row mirror), then two cross-row exchanges.  Each step adds a value
// to its partner's in a commutative pair, so all lanes end with one value.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float wave_allsum(float v) {
  v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp<0x141>(v);  // row_half_mirror
  v += dpp<0x140>(v);  // row_mirror
  v += __shfl_xor(v, 16, 64);
  v += __shfl_xor(v, 32, 64);
  return v;
}

template <int DPL>
__device__ __forceinline__ void load_row(const float* p, float* r) {
  if constexpr (DPL == 1) {
    r[0] = p[0];
  } else if constexpr (DPL == 2) {
    const float2 t = *reinterpret_cast<const float2*>(p);
    r[0] = t.x; r[1] = t.y;
  } else {
#pragma unroll
    for (int j = 0; j < DPL; j += 4) {
      const float4 t = *reinterpret_cast<const float4*>(p + j);
      r[j] = t.x; r[j + 1] = t.y; r[j + 2] = t.z; r[j + 3] = t.w;
    }
  }
}

// Stage one head (D floats) normalised -- in * (mean(in^2) + eps)^-1/2 * w,
// w == nullptr meaning ones -- into LDS, one wavefront, one global read.
template <int DPL>
__device__ __forceinline__ void norm_head_to_lds(const float* __restrict__ in,
                                                 const float* __restrict__ w, float* out,
                                                 uint32_t D, float eps, uint32_t lane) {
  float v[DPL];
  const uint32_t d0 = lane * DPL;
  const bool dl = d0 < D;
  if (dl) load_row<DPL>(in + d0, v);
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < DPL; j++) ss += dl ? v[j] * v[j] : 0.f;
  const float inv = 1.0f / sqrtf(wave_allsum(ss) / (float)D + eps);
  if (dl) {
#pragma unroll
    for (int j = 0; j < DPL; j++) out[d0 + j] = v[j] * inv * (w ? w[d0 + j] : 1.0f);
  }
}

// RoPE angles of the pairs a lane rotates: i = lane + 64 k < rot/2, freq =
// theta^(-2i/rot).  Computed before the head loads return (they depend on
// nothing loaded) so the transcendental work hides under the load latency.
#define ROPE_K (MAX_D / 128)
__device__ __forceinline__ void rope_angles(uint32_t rot, float theta, uint32_t clock,
                                            uint32_t lane, float* c, float* s) {
#pragma unroll
  for (int k = 0; k < ROPE_K; k++) {
    const uint32_t i = lane + 64 * k;
    c[k] = 1.f;
    s[k] = 0.f;
    if (i < rot / 2) gh_rope_angle(i, rot, theta, clock, &c[k], &s[k]);
  }
}

// The same angles read from a per-token table (cos then sin, ROPE_TAB_HALF
// each) that the step kernel wrote with gh_rope_angle.
__device__ __forceinline__ void rope_angles_tab(const float* __restrict__ tab, uint32_t rot,
                                                uint32_t lane, float* c, float* s) {
#pragma unroll
  for (int k = 0; k < ROPE_K; k++) {
    // lanes past rot / 2 load a valid entry they never use (rope_lds reads
    // the angles of pairs i < rot / 2 only): no branch, no select, so the
    // loads stay in flight until the rotation needs them
    const uint32_t ic = min(lane + 64u * k, (uint32_t)ROPE_TAB_HALF - 1u);
    c[k] = tab[ic];
    s[k] = tab[ROPE_TAB_HALF + ic];
  }
  (void)rot;
}

// Partial RoPE in place on an LDS head, one wavefront: pairs (i, i + rot/2)
// for i < rot/2 rotate by the angles of rope_angles.
__device__ __forceinline__ void rope_lds(float* h, uint32_t rot, const float* c, const float* s,
                                         uint32_t lane) {
  const uint32_t half = rot / 2;
#pragma unroll
  for (int k = 0; k < ROPE_K; k++) {
    const uint32_t i = lane + 64 * k;
    if (i < half) {
      const float v0 = h[i], v1 = h[i + half];
      h[i] = v0 * c[k] - v1 * s[k];
      h[i + half] = v0 * s[k] + v1 * c[k];
    }
  }
}

#define ATT_CHUNK ATT_NT  // active-list indices staged in LDS per round (one per thread)

// One workgroup per (kv head, split of the active list).  Each wavefront
// owns all D dims of a slot (DPL per lane) and walks the split's slots in
// tiles of T: the 2T row loads of a tile are issued together, the T x G
// scores are reduced together, and the online softmax (running max m,
// running sum l, rescaled output o per query head) is updated once per tile.
// The waves' states merge through LDS and the split writes its partial
// (o[D], m, l); gh_attn_merge_k combines the splits.  No inter-workgroup
// synchronisation inside the kernel: a device-scope fence per workgroup
// costs more than the whole attention at these sizes.
template <int DPL, int T, bool PF>
__device__ __forceinline__ void attn_split(const AttnArgs& a) {
  __shared__ float qs[MAX_G][MAX_D];
  __shared__ float knew[MAX_D], vnew[MAX_D];
  __shared__ uint32_t sidx[ATT_CHUNK];
  __shared__ float wm[ATT_WAVES][MAX_G], wl[ATT_WAVES][MAX_G];
  __shared__ float wo[ATT_WAVES][MAX_G][MAX_D];

  const uint32_t D = a.D, G = a.nq / a.nkv;
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const size_t kv_dim = (size_t)a.nkv * D;
  // decode: one split of one token; prefill: one split of token blockIdx.y's
  // list (nsplit 1: all of it, and the workgroup writes the output rows)
  const uint32_t nsplit = a.nsplit;
  const uint32_t kvh = blockIdx.x / nsplit;
  const uint32_t split = blockIdx.x % nsplit;
  const uint32_t tok = PF ? blockIdx.y : 0u;
  const uint32_t clock = PF ? 0u : a.step[0], cur_slot = PF ? 0u : a.step[1];
  const uint32_t S = PF ? a.n_active[tok] : a.step[2];
  const uint32_t* active = PF ? a.active + (size_t)tok * a.active_stride : a.active;
  const float* qsrc = PF ? a.q + (size_t)tok * a.q_stride : a.q;
  const bool fuse = !PF && a.fuse;

  // this split's share of the active list, staged in rounds of ATT_CHUNK
  // indices; the first round's load goes out before the prologue's
  const uint32_t per = (S + nsplit - 1) / nsplit;
  const uint32_t s0 = min(S, split * per), s1 = min(S, s0 + per);
  const uint32_t n0 = min(s1 - s0, (uint32_t)ATT_CHUNK);
  const uint32_t idx0 = tid < n0 ? active[s0 + tid] : 0u;  // ATT_CHUNK == ATT_NT

  // 1. query heads of this kv group (and, fused, this token's K/V) into LDS
  if (fuse) {
    float rc[ROPE_K], rs[ROPE_K];
    rope_angles(a.rot, a.theta, clock, lane, rc, rs);
    for (uint32_t g = wave; g < G + 2; g += ATT_WAVES) {
      if (g < G)
        norm_head_to_lds<DPL>(a.q + (size_t)(kvh * G + g) * D, a.q_norm, qs[g], D, a.eps, lane);
      else if (g == G)
        norm_head_to_lds<DPL>(a.k_in + (size_t)kvh * D, a.k_norm, knew, D, a.eps, lane);
      else
        norm_head_to_lds<DPL>((a.k_eq_v ? a.k_in : a.v_in) + (size_t)kvh * D, nullptr, vnew, D,
                              a.eps, lane);
    }
    if (tid < n0) sidx[tid] = idx0;
    __syncthreads();
    for (uint32_t g = wave; g < G + 1; g += ATT_WAVES) rope_lds(g < G ? qs[g] : knew, a.rot, rc, rs, lane);
  } else {
    for (uint32_t i = tid; i < G * D; i += ATT_NT) qs[i / D][i % D] = qsrc[(size_t)kvh * G * D + i];
    if (tid < n0) sidx[tid] = idx0;
  }
  __syncthreads();
  if (fuse && split == 0) {  // ring_buffer.writeKV for this layer
    float* kc = a.k_cache + (size_t)cur_slot * kv_dim + (size_t)kvh * D;
    float* vc = a.v_cache + (size_t)cur_slot * kv_dim + (size_t)kvh * D;
    for (uint32_t d = tid; d < D; d += ATT_NT) {
      kc[d] = knew[d];
      vc[d] = vnew[d];
    }
  }

  // 2. online softmax over the split's slots
  const uint32_t d0 = lane * DPL;
  const bool dl = d0 < D;
  float q[MAX_G][DPL], o[MAX_G][DPL], m[MAX_G], l[MAX_G];
#pragma unroll
  for (int g = 0; g < MAX_G; g++) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int j = 0; j < DPL; j++) {
      q[g][j] = (g < (int)G && dl) ? qs[g][d0 + j] : 0.f;
      o[g][j] = 0.f;
    }
  }
  const float* kbase = a.k_cache + (size_t)kvh * D + d0;
  const float* vbase = a.v_cache + (size_t)kvh * D + d0;

  for (uint32_t r0 = s0; r0 < s1; r0 += ATT_CHUNK) {
    const uint32_t n = min(s1 - r0, (uint32_t)ATT_CHUNK);
    if (r0 != s0) {     // the first round was staged with the prologue
      __syncthreads();  // previous round's indices are no longer read
      for (uint32_t t = tid; t < n; t += ATT_NT) sidx[t] = active[r0 + t];
      __syncthreads();
    }
    for (uint32_t base = wave * T; base < n; base += ATT_WAVES * T) {
      float kr[T][DPL], vr[T][DPL];
#pragma unroll
      for (int j = 0; j < T; j++) {
        const uint32_t slot = sidx[min(base + j, n - 1)];
        if (fuse && slot == cur_slot) {  // this token's K/V: from LDS, not the cache
#pragma unroll
          for (int e = 0; e < DPL; e++) {
            kr[j][e] = dl ? knew[d0 + e] : 0.f;
            vr[j][e] = dl ? vnew[d0 + e] : 0.f;
          }
        } else if (dl) {
          load_row<DPL>(kbase + (size_t)slot * kv_dim, kr[j]);
          load_row<DPL>(vbase + (size_t)slot * kv_dim, vr[j]);
        } else {
#pragma unroll
          for (int e = 0; e < DPL; e++) kr[j][e] = vr[j][e] = 0.f;
        }
      }
#pragma unroll
      for (int g = 0; g < MAX_G; g++) {
        if (g >= (int)G) break;
        float s[T];
#pragma unroll
        for (int j = 0; j < T; j++) {
          float p = 0.f;
#pragma unroll
          for (int e = 0; e < DPL; e++) p += q[g][e] * kr[j][e];
          s[j] = p;
        }
#pragma unroll
        for (int j = 0; j < T; j++) s[j] = wave_allsum(s[j]) * a.scale;
        float mt = m[g];
#pragma unroll
        for (int j = 0; j < T; j++)
          if (base + j < n) mt = fmaxf(mt, s[j]);
        const float corr = __expf(m[g] - mt);  // m = -inf, mt finite: 0
        l[g] *= corr;
#pragma unroll
        for (int e = 0; e < DPL; e++) o[g][e] *= corr;
#pragma unroll
        for (int j = 0; j < T; j++) {
          const float p = base + j < n ? __expf(s[j] - mt) : 0.f;
          l[g] += p;
#pragma unroll
          for (int e = 0; e < DPL; e++) o[g][e] += p * vr[j][e];
        }
        m[g] = mt;
      }
    }
  }

  // 3. merge the waves of this workgroup (wave order), write the split partial
#pragma unroll
  for (int g = 0; g < MAX_G; g++) {
    if (g >= (int)G) break;
    if (lane == 0) {
      wm[wave][g] = m[g];
      wl[wave][g] = l[g];
    }
    if (dl) {
#pragma unroll
      for (int e = 0; e < DPL; e++) wo[wave][g][d0 + e] = o[g][e];
    }
  }
  __syncthreads();
  const uint32_t PS = D + 4;  // partial record: o[D], m, l (+2 pad: float4 rows)
  // partials: [token][kv head][split][g] records (decode: token 0)
  float* part = PF && nsplit == 1 ? nullptr
                                  : a.part + (((size_t)tok * a.nkv + kvh) * nsplit + split) * G * PS;
  for (uint32_t i = tid; i < G * D; i += ATT_NT) {
    const uint32_t g = i / D, d = i % D;
    float M = -INFINITY;
    for (int w = 0; w < ATT_WAVES; w++) M = fmaxf(M, wm[w][g]);
    float L = 0.f, O = 0.f;
    for (int w = 0; w < ATT_WAVES; w++) {
      const float c = wm[w][g] == -INFINITY ? 0.f : __expf(wm[w][g] - M);
      L += wl[w][g] * c;
      O += wo[w][g][d] * c;
    }
    if (PF && nsplit == 1) {  // the whole list: the final output row of this token
      a.out_rows[(size_t)tok * a.out_stride + (size_t)(kvh * G + g) * D + d] = L > 0.f ? O / L : 0.f;
    } else {
      part[g * PS + d] = O;
      if (d == 0) {
        part[g * PS + D] = M;
        part[g * PS + D + 1] = L;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Decode attention, one workgroup per (kv head, split of the active list).
// The same work as attn_split's decode form, ordered for latency: a kernel
// this small is a chain of memory round trips, so every load that does not
// depend on another goes out first.
//  - Each wave reads its own tile's slot numbers (lanes 0..T-1, broadcast
//    with readlane) instead of staging the split's list in LDS behind a
//    barrier; when the step flags say the list is 0 .. S-1 it reads nothing.
//  - Fused: each wave loads its prologue head rows (q heads, this token's k
//    and v, their norm weights, the RoPE table) and then its first tile's
//    K/V rows, and only then normalises; the K/V latency hides the prologue.
//    Loads complete in order, so the prologue's waits do not wait for K/V.
//  - RoPE angles come from the per-token table when one is given.
// This token's own slot is served from LDS (its cache row is written by
// split 0 in the same launch).  Waves merge through LDS and each split
// writes (o, m, l) for gh_attn_merge_k, as attn_split does.
// ---------------------------------------------------------------------------
// A zero the compiler cannot see through, so a value derived from it counts
// as per-lane: a slot number loaded with it stays in a vector register
// instead of being moved to a scalar one (and waited for) right after its
// load.
__device__ __forceinline__ uint32_t opaque_zero() {
  uint32_t z;
  asm volatile("v_mov_b32 %0, 0" : "=v"(z));
  return z;
}

struct DecodeSmem {
  float qs[MAX_G][MAX_D];
  float knew[MAX_D], vnew[MAX_D];
  float wm[ATT_WAVES][MAX_G], wl[ATT_WAVES][MAX_G];
  float wo[ATT_WAVES][MAX_G][MAX_D];
};

// DENSE: the list is 0 .. S-1 (step flags bit 1) and is not read.  The two
// forms are separate straight-line bodies, so no load sits under a branch.
// GATED: a gated layer's form; it loads the run flag at entry and tests it
// just before its first global write, so the flag's latency hides under the
// prologue and first-tile loads (all of which stay in bounds either way).
template <int DPL, int T, bool DENSE, bool GATED>
__device__ __forceinline__ void attn_decode(const AttnArgs& a, DecodeSmem& sm) {
  auto& qs = sm.qs;
  auto& knew = sm.knew;
  auto& vnew = sm.vnew;
  auto& wm = sm.wm;
  auto& wl = sm.wl;
  auto& wo = sm.wo;

  const uint32_t D = a.D, G = a.nq / a.nkv;
  const uint32_t tid = threadIdx.x, lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const size_t kv_dim = (size_t)a.nkv * D;
  const uint32_t nsplit = a.nsplit;
  const uint32_t kvh = blockIdx.x / nsplit, split = blockIdx.x % nsplit;
  const uint32_t clock = a.step[0], cur_slot = a.step[1], S = a.step[2];
  const bool fuse = a.fuse != 0;
  const uint32_t go = GATED ? *a.run : 1u;
  // the splits that run: about ATT_SLOTS_PER_SPLIT active slots each
  const uint32_t live = attn_live_splits(nsplit, S);
  if (split >= live) return;  // uniform over the workgroup
  const uint32_t per = (S + live - 1) / live;
  const uint32_t s0 = min(S, split * per), s1 = min(S, s0 + per);
  const uint32_t n = s1 - s0;
  const uint32_t d0 = lane * DPL;
  const bool dl = d0 < D;
  const uint32_t dc = dl ? d0 : 0u;  // loads stay in bounds; lanes past D are ignored
  const float* kbase = a.k_cache + (size_t)kvh * D + dc;
  const float* vbase = a.v_cache + (size_t)kvh * D + dc;
  const uint32_t last = S > 0u ? S - 1u : 0u;  // the last list position (S = 0: none read)

  // Slot numbers of a tile starting at list position s0 + base, clamped to the
  // split (the extra entries are masked in the softmax): scalar loads, so
  // waiting for them never waits for a vector load.
  // With S = 0 no list entry exists: position 0 of the step record stands in.
  const uint32_t* lp = S > 0u ? a.active : a.step;
  auto tile_slots = [&](uint32_t base, uint32_t* sl) {
    const uint32_t z = DENSE ? 0u : opaque_zero();
#pragma unroll
    for (int j = 0; j < T; j++) {
      const uint32_t pos = min(s0 + min(base + (uint32_t)j, n > 0u ? n - 1u : 0u), last);
      if constexpr (DENSE)
        sl[j] = pos;
      else
        sl[j] = lp[pos + z];  // with S = 0 the slot read is never used
    }
  };

  // 1. this wave's first tile's slot numbers (the earliest loads)
  const uint32_t base0 = wave * T;
  uint32_t slot0[T];
  tile_slots(base0, slot0);
  // the scheduler keeps the phases in this order: slot numbers, prologue
  // loads, K/V loads; the first wait (for the slot numbers) then leaves the
  // prologue loads in flight
  __builtin_amdgcn_sched_barrier(0);

  // 2. prologue loads: up to two head rows per wave (G query heads, then
  //    this token's k and v), their norm weights, the RoPE angles.  Every
  //    pointer is valid in every mode (the host passes real rows), so the
  //    loads need no branch.
  float hv[2][DPL], hw[2][DPL], rc[ROPE_K], rs[ROPE_K];
  const uint32_t nheads = fuse ? G + 2 : G;
  if (fuse && a.rope_tab) rope_angles_tab(a.rope_tab, a.rot, lane, rc, rs);
#pragma unroll
  for (int h = 0; h < 2; h++) {
    const uint32_t g = min(wave + (uint32_t)h * ATT_WAVES, nheads - 1);
    const float* src = g < G ? a.q + (size_t)(kvh * G + g) * D
                       : g == G ? a.k_in + (size_t)kvh * D
                                : (a.k_eq_v ? a.k_in : a.v_in) + (size_t)kvh * D;
    load_row<DPL>(src + dc, hv[h]);
    load_row<DPL>((g == G ? a.k_norm : a.q_norm) + dc, hw[h]);
  }
  __builtin_amdgcn_sched_barrier(0);

  // 3. the first tile's K/V rows (this token's own slot is replaced from LDS
  //    after the prologue)
  float kr[T][DPL], vr[T][DPL];
#pragma unroll
  for (int j = 0; j < T; j++) {
    load_row<DPL>(kbase + (size_t)slot0[j] * kv_dim, kr[j]);
    load_row<DPL>(vbase + (size_t)slot0[j] * kv_dim, vr[j]);
  }
  __builtin_amdgcn_sched_barrier(0);

  // 4. prologue compute: normalise (fused) or copy the heads into LDS
  if (fuse && !a.rope_tab) rope_angles(a.rot, a.theta, clock, lane, rc, rs);
#pragma unroll
  for (int h = 0; h < 2; h++) {
    const uint32_t g = wave + (uint32_t)h * ATT_WAVES;
    if (g < nheads) {
      float inv = 1.f;
      if (fuse) {
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < DPL; j++) ss += dl ? hv[h][j] * hv[h][j] : 0.f;
        inv = 1.0f / sqrtf(wave_allsum(ss) / (float)D + a.eps);
      }
      const bool weighted = fuse && g <= G;  // v is normalised to unit RMS only
      float* out = g < G ? qs[g] : g == G ? knew : vnew;
      if (dl) {
#pragma unroll
        for (int j = 0; j < DPL; j++)
          out[d0 + j] = fuse ? hv[h][j] * inv * (weighted ? hw[h][j] : 1.0f) : hv[h][j];
      }
    }
  }
  __syncthreads();
  if (fuse)
    for (uint32_t g = wave; g < G + 1; g += ATT_WAVES) rope_lds(g < G ? qs[g] : knew, a.rot, rc, rs, lane);
  __syncthreads();
  if (GATED && go == 0u) return;  // a gated-off layer: uniform, nothing written yet
  if (fuse && split == 0) {  // ring_buffer.writeKV for this layer
    float* kc = a.k_cache + (size_t)cur_slot * kv_dim + (size_t)kvh * D;
    float* vc = a.v_cache + (size_t)cur_slot * kv_dim + (size_t)kvh * D;
    for (uint32_t d = tid; d < D; d += ATT_NT) {
      kc[d] = knew[d];
      vc[d] = vnew[d];
    }
  }

  // 5. online softmax over the wave's tiles
  float q[MAX_G][DPL], o[MAX_G][DPL], m[MAX_G], l[MAX_G];
#pragma unroll
  for (int g = 0; g < MAX_G; g++) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int j = 0; j < DPL; j++) {
      q[g][j] = (g < (int)G && dl) ? qs[g][d0 + j] : 0.f;
      o[g][j] = 0.f;
    }
  }
  for (uint32_t base = base0; base < n; base += ATT_WAVES * T) {
    if (base != base0) {  // later tiles: slot numbers, then the rows
      tile_slots(base, slot0);
#pragma unroll
      for (int j = 0; j < T; j++) {
        load_row<DPL>(kbase + (size_t)slot0[j] * kv_dim, kr[j]);
        load_row<DPL>(vbase + (size_t)slot0[j] * kv_dim, vr[j]);
      }
    }
#pragma unroll
    for (int j = 0; j < T; j++) {
      if (fuse && slot0[j] == cur_slot) {  // this token's K/V: from LDS, not the cache
#pragma unroll
        for (int e = 0; e < DPL; e++) {
          kr[j][e] = dl ? knew[d0 + e] : 0.f;
          vr[j][e] = dl ? vnew[d0 + e] : 0.f;
        }
      }
    }
#pragma unroll
    for (int g = 0; g < MAX_G; g++) {
      if (g >= (int)G) break;
      float sc[T];
#pragma unroll
      for (int j = 0; j < T; j++) {
        float p = 0.f;
#pragma unroll
        for (int e = 0; e < DPL; e++) p += q[g][e] * kr[j][e];
        sc[j] = p;
      }
#pragma unroll
      for (int j = 0; j < T; j++) sc[j] = wave_allsum(sc[j]) * a.scale;
      float mt = m[g];
#pragma unroll
      for (int j = 0; j < T; j++)
        if (base + j < n) mt = fmaxf(mt, sc[j]);
      const float corr = __expf(m[g] - mt);  // m = -inf, mt finite: 0
      l[g] *= corr;
#pragma unroll
      for (int e = 0; e < DPL; e++) o[g][e] *= corr;
#pragma unroll
      for (int j = 0; j < T; j++) {
        const float p = base + j < n ? __expf(sc[j] - mt) : 0.f;
        l[g] += p;
#pragma unroll
        for (int e = 0; e < DPL; e++) o[g][e] += p * vr[j][e];
      }
      m[g] = mt;
    }
  }

  // 6. merge the waves (wave order), write the split partial (o, m, l)
#pragma unroll
  for (int g = 0; g < MAX_G; g++) {
    if (g >= (int)G) break;
    if (lane == 0) {
      wm[wave][g] = m[g];
      wl[wave][g] = l[g];
    }
    if (dl) {
#pragma unroll
      for (int e = 0; e < DPL; e++) wo[wave][g][d0 + e] = o[g][e];
    }
  }
  __syncthreads();
  const uint32_t PS = D + 4;
  float* part = a.part + ((size_t)kvh * nsplit + split) * G * PS;
  for (uint32_t i = tid; i < G * D; i += ATT_NT) {
    const uint32_t g = i / D, d = i % D;
    float M = -INFINITY;
    for (int w = 0; w < ATT_WAVES; w++) M = fmaxf(M, wm[w][g]);
    float L = 0.f, O = 0.f;
    for (int w = 0; w < ATT_WAVES; w++) {
      const float c = wm[w][g] == -INFINITY ? 0.f : __expf(wm[w][g] - M);
      L += wl[w][g] * c;
      O += wo[w][g][d] * c;
    }
    part[g * PS + d] = O;
    if (d == 0) {
      part[g * PS + D] = M;
      part[g * PS + D + 1] = L;
    }
  }
}

template <int DPL, int T, bool GATED = false>
__device__ __forceinline__ void attn_decode_k(const AttnArgs& a) {
  __shared__ DecodeSmem sm;
  if (a.flags != nullptr && (*a.flags & 2u) != 0u)
    attn_decode<DPL, T, true, GATED>(a, sm);
  else
    attn_decode<DPL, T, false, GATED>(a, sm);
}

extern "C" __global__ __launch_bounds__(ATT_NT) void gh_attn_d1_k(AttnArgs a) { attn_decode_k<1, 8>(a); }
extern "C" __global__ __launch_bounds__(ATT_NT) void gh_attn_d2_k(AttnArgs a) { attn_decode_k<2, 8>(a); }
extern "C" __global__ __launch_bounds__(ATT_NT) void gh_attn_d4_k(AttnArgs a) { attn_decode_k<4, 8>(a); }
extern "C" __global__ __launch_bounds__(ATT_NT) void gh_attn_d8_k(AttnArgs a) { attn_decode_k<8, 4>(a); }
// gated layers (quiescence on): nothing when the layer's run flag is 0
#define GH_ATTN_GATED(DPL, T)                                                                   \
  extern "C" __global__ __launch_bounds__(ATT_NT) void gh_attn_d##DPL##_q_k(AttnArgs a) {       \
    attn_decode_k<DPL, T, true>(a);                                                             \
  }
GH_ATTN_GATED(1, 8) GH_ATTN_GATED(2, 8) GH_ATTN_GATED(4, 8) GH_ATTN_GATED(8, 4)

// Batched prefill: grid (kv heads x a.nsplit, tokens); each workgroup runs
// token blockIdx.y's whole active list (a.nsplit 1), or one share of it whose
// partials gh_pf_attn_merge_k combines (q already normalised and roped by
// gh_pf_qkv_rope_k, this batch's K/V already in the caches).
extern "C" __global__ __launch_bounds__(ATT_NT) void gh_pf_attn_d1_k(AttnArgs a) { attn_split<1, 8, true>(a); }
extern "C" __global__ __launch_bounds__(ATT_NT) void gh_pf_attn_d2_k(AttnArgs a) { attn_split<2, 8, true>(a); }
extern "C" __global__ __launch_bounds__(ATT_NT) void gh_pf_attn_d4_k(AttnArgs a) { attn_split<4, 8, true>(a); }
extern "C" __global__ __launch_bounds__(ATT_NT) void gh_pf_attn_d8_k(AttnArgs a) { attn_split<8, 4, true>(a); }

// v + (v of lane l ^ 16) and v + (v of lane l ^ 32), with the gfx950 lane
// swaps (no LDS round trip); both partners compute the same sum.
__device__ __forceinline__ float swap16_add(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float swap32_add(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float wave_allsum_swap(float v) {
  v += dpp<0xB1>(v);
  v += dpp<0x4E>(v);
  v += dpp<0x141>(v);
  v += dpp<0x140>(v);
  return swap32_add(swap16_add(v));
}

// Batched prefill over groups of PF_GT consecutive tokens: grid (kv heads,
// token groups), group ngroups-1-blockIdx.y first (the longest lists of a
// causal batch start first).  A workgroup walks the union of its tokens'
// active lists once (entries: slot | token mask << 24, built on the host),
// so each K/V row it loads serves all PF_GT tokens x G query heads; a token
// skips the slots its mask bit does not cover.  Requires G <= 2 and D <= 256;
// the online softmax, wave merge and output follow attn_split.  The list
// holds (slot, token mask) pairs; the staging packs each into one word.
#define PF_GT 4
#define PF_QN (PF_GT * 2)  // query vectors per workgroup: tokens x heads (G <= 2)
#define PF_MAXD 256
template <int DPL, int TT>
__device__ __forceinline__ void attn_pf_group(const AttnArgs& a) {
  __shared__ float qs[PF_QN][PF_MAXD];
  __shared__ uint32_t sidx[ATT_CHUNK];
  __shared__ float wm[ATT_WAVES][PF_QN], wl[ATT_WAVES][PF_QN];
  __shared__ float wo[ATT_WAVES][PF_QN][PF_MAXD];

  const uint32_t D = a.D, G = a.nq / a.nkv, gsh = G == 2 ? 1u : 0u;
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const size_t kv_dim = (size_t)a.nkv * D;
  const uint32_t kvh = blockIdx.x, grp = gridDim.y - 1 - blockIdx.y;
  const uint32_t t0 = grp * PF_GT, nt = min((uint32_t)PF_GT, a.n_tokens - t0);
  const uint32_t qn_used = nt * G;
  const uint32_t S = a.n_active[grp];
  const uint32_t* list = a.active + (size_t)grp * a.active_stride;
  const uint32_t n0 = min(S, (uint32_t)ATT_CHUNK);
  const uint32_t idx0 = tid < n0 ? list[2 * tid] | list[2 * tid + 1] << 24 : 0u;

  // 1. the group's query vectors (token i, head g at qs[i * G + g]) into LDS
  for (uint32_t i = tid; i < qn_used * D; i += ATT_NT) {
    const uint32_t qn = i / D, d = i % D;
    const uint32_t t = t0 + (qn >> gsh), g = qn & (G - 1);
    qs[qn][d] = a.q[(size_t)t * a.q_stride + (size_t)(kvh * G + g) * D + d];
  }
  if (tid < n0) sidx[tid] = idx0;
  __syncthreads();

  // 2. online softmax over the union list, per query vector
  const uint32_t d0 = lane * DPL;
  const bool dl = d0 < D;
  float q[PF_QN][DPL], o[PF_QN][DPL], m[PF_QN], l[PF_QN];
#pragma unroll
  for (int qn = 0; qn < PF_QN; qn++) {
    m[qn] = -INFINITY;
    l[qn] = 0.f;
#pragma unroll
    for (int j = 0; j < DPL; j++) {
      q[qn][j] = ((uint32_t)qn < qn_used && dl) ? qs[qn][d0 + j] : 0.f;
      o[qn][j] = 0.f;
    }
  }
  const float* kbase = a.k_cache + (size_t)kvh * D + d0;
  const float* vbase = a.v_cache + (size_t)kvh * D + d0;

  for (uint32_t r0 = 0; r0 < S; r0 += ATT_CHUNK) {
    const uint32_t n = min(S - r0, (uint32_t)ATT_CHUNK);
    if (r0 != 0) {
      __syncthreads();
      for (uint32_t t = tid; t < n; t += ATT_NT)
        sidx[t] = list[2 * (r0 + t)] | list[2 * (r0 + t) + 1] << 24;
      __syncthreads();
    }
    for (uint32_t base = wave * TT; base < n; base += ATT_WAVES * TT) {
      float kr[TT][DPL], vr[TT][DPL];
      uint32_t msk[TT], any = 0;
#pragma unroll
      for (int j = 0; j < TT; j++) {
        const uint32_t e = sidx[min(base + j, n - 1)];
        const uint32_t slot = e & 0xFFFFFFu;
        msk[j] = base + j < n ? e >> 24 : 0u;
        any |= msk[j];
        if (dl) {
          load_row<DPL>(kbase + (size_t)slot * kv_dim, kr[j]);
          load_row<DPL>(vbase + (size_t)slot * kv_dim, vr[j]);
        } else {
#pragma unroll
          for (int e2 = 0; e2 < DPL; e2++) kr[j][e2] = vr[j][e2] = 0.f;
        }
      }
#pragma unroll
      for (int qn = 0; qn < PF_QN; qn++) {
        const uint32_t bit = (uint32_t)qn >> gsh;
        if ((uint32_t)qn >= qn_used || !((any >> bit) & 1u)) continue;  // wave-uniform
        float s[TT];
#pragma unroll
        for (int j = 0; j < TT; j++) {
          float p = 0.f;
#pragma unroll
          for (int e2 = 0; e2 < DPL; e2++) p += q[qn][e2] * kr[j][e2];
          s[j] = p;
        }
#pragma unroll
        for (int j = 0; j < TT; j++) s[j] = wave_allsum_swap(s[j]) * a.scale;
        float mt = m[qn];
#pragma unroll
        for (int j = 0; j < TT; j++)
          if ((msk[j] >> bit) & 1u) mt = fmaxf(mt, s[j]);
        const float corr = __expf(m[qn] - mt);  // m = -inf, mt finite: 0
        l[qn] *= corr;
#pragma unroll
        for (int e2 = 0; e2 < DPL; e2++) o[qn][e2] *= corr;
#pragma unroll
        for (int j = 0; j < TT; j++) {
          const float p = (msk[j] >> bit) & 1u ? __expf(s[j] - mt) : 0.f;
          l[qn] += p;
#pragma unroll
          for (int e2 = 0; e2 < DPL; e2++) o[qn][e2] += p * vr[j][e2];
        }
        m[qn] = mt;
      }
    }
  }

  // 3. merge the waves (wave order) and write each token's output rows
#pragma unroll
  for (int qn = 0; qn < PF_QN; qn++) {
    if ((uint32_t)qn >= qn_used) break;
    if (lane == 0) {
      wm[wave][qn] = m[qn];
      wl[wave][qn] = l[qn];
    }
    if (dl) {
#pragma unroll
      for (int e2 = 0; e2 < DPL; e2++) wo[wave][qn][d0 + e2] = o[qn][e2];
    }
  }
  __syncthreads();
  for (uint32_t i = tid; i < qn_used * D; i += ATT_NT) {
    const uint32_t qn = i / D, d = i % D;
    const uint32_t t = t0 + (qn >> gsh), g = qn & (G - 1);
    float M = -INFINITY;
    for (int w = 0; w < ATT_WAVES; w++) M = fmaxf(M, wm[w][qn]);
    float L = 0.f, O = 0.f;
    for (int w = 0; w < ATT_WAVES; w++) {
      const float c = wm[w][qn] == -INFINITY ? 0.f : __expf(wm[w][qn] - M);
      L += wl[w][qn] * c;
      O += wo[w][qn][d] * c;
    }
    a.out_rows[(size_t)t * a.out_stride + (size_t)(kvh * G + g) * D + d] = L > 0.f ? O / L : 0.f;
  }
}

extern "C" __global__ __launch_bounds__(ATT_NT) void gh_pf_attn_g_d1_k(AttnArgs a) { attn_pf_group<1, 8>(a); }
extern "C" __global__ __launch_bounds__(ATT_NT) void gh_pf_attn_g_d2_k(AttnArgs a) { attn_pf_group<2, 8>(a); }
extern "C" __global__ __launch_bounds__(ATT_NT) void gh_pf_attn_g_d4_k(AttnArgs a) { attn_pf_group<4, 8>(a); }

// Batched q/k norm + RoPE + cache write (qkv_rope.wgsl for T tokens): grid
// (nq + nkv heads, tokens), one wavefront each.  Token t's q/k/v rows start
// at a.q + t * q_stride (q, then k, then v unless k_eq_v); its position and
// ring slot are clocks[t] and slots[t].
extern "C" __global__ __launch_bounds__(64) void gh_pf_qkv_rope_k(AttnArgs a,
                                                                 const uint32_t* clocks,
                                                                 const uint32_t* slots) {
  const uint32_t h = blockIdx.x, t = blockIdx.y, lane = threadIdx.x, D = a.D;
  const uint32_t clock = clocks[t], slot = slots[t];
  float* row = const_cast<float*>(a.q) + (size_t)t * a.q_stride;
  const size_t q_dim = (size_t)a.nq * D, kv_dim = (size_t)a.nkv * D;
  if (h < a.nq) {
    float* q = row + (size_t)h * D;
    const float inv = head_inv_rms(q, D, a.eps, lane);
    norm_rope_head(q, a.q_norm, q, D, a.rot, a.theta, inv, clock, lane);
    return;
  }
  const uint32_t kh = h - a.nq;
  if (kh >= a.nkv) return;
  const float* kin = row + q_dim + (size_t)kh * D;
  const float* vin = (a.k_eq_v ? row + q_dim : row + q_dim + kv_dim) + (size_t)kh * D;
  float* kc = a.k_cache + (size_t)slot * kv_dim + (size_t)kh * D;
  float* vc = a.v_cache + (size_t)slot * kv_dim + (size_t)kh * D;
  const float kinv = head_inv_rms(kin, D, a.eps, lane);
  norm_rope_head(kin, a.k_norm, kc, D, a.rot, a.theta, kinv, clock, lane);
  const float vinv = head_inv_rms(vin, D, a.eps, lane);
  for (uint32_t d = lane; d < D; d += 64) vc[d] = vin[d] * vinv;
}

// The same for head_dim 256, one workgroup per token (grid (tokens), 256
// threads, gridDim.y of them per token): a token's head rows are jobs --
// query heads [0, nq), key heads [nq, nq + nkv), value heads after them --
// and wave w of workgroup (t, y) takes jobs w + 4 (y + G i), i = 0, 1, ...
// (G = gridDim.y, at most JOBS per wave).  Every job's row (4 floats per
// lane) loads before any is used, the RoPE angles are computed once per wave
// rather than once per head, and each head is normalised in registers,
// rotated through the wave's LDS row (rope_lds), and stored: q to a.q, k and
// v into the caches at slots[t].  With a.nplanes >= 1 the rows are the QKV
// GEMM's unsummed K-split planes, added in plane order as they load, PLANES
// planes in flight at a time.
// Two forms: one workgroup per token (JOBS 16, G = 1: a long prompt's tokens
// fill the CUs), and for a few tokens ceil((nq + 2 nkv) / 8) workgroups per
// token with 8 planes in flight (JOBS 2): at 16 tokens and 8 planes the
// first form took 12.6 us per layer and the second 6.0, at 512 tokens and 2
// planes 12.8 against 15.9 us.
template <int JOBS, int PLANES>
__device__ __forceinline__ void pf_qkv_rope4(const AttnArgs& a, const uint32_t* clocks,
                                             const uint32_t* slots) {
  __shared__ float hb[ATT_WAVES][256];
  const uint32_t t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t clock = clocks[t], slot = slots[t];
  float* row = const_cast<float*>(a.q) + (size_t)t * a.q_stride;
  const float* srow = a.nplanes ? a.q_planes + (size_t)t * a.q_stride : row;
  const uint32_t nq = a.nq, nkv = a.nkv, njobs = nq + 2 * nkv;
  const uint32_t jstride = ATT_WAVES * gridDim.y, j0 = wave + ATT_WAVES * blockIdx.y;
  const uint32_t per = (njobs + jstride - 1) / jstride;  // the same for every wave
  const size_t q_dim = (size_t)nq * 256, kv_dim = (size_t)nkv * 256;
  auto src = [&](uint32_t j) -> size_t {  // offset of job j's row in a token row
    if (j < nq) return (size_t)j * 256;
    if (j < nq + nkv) return q_dim + (size_t)(j - nq) * 256;
    return (a.k_eq_v ? q_dim : q_dim + kv_dim) + (size_t)(j - nq - nkv) * 256;
  };
  const uint32_t d0 = lane * 4;
  float4 v[JOBS];
#pragma unroll
  for (int i = 0; i < JOBS; i++) {
    const uint32_t j = min(j0 + jstride * (uint32_t)i, njobs - 1);
    v[i] = *reinterpret_cast<const float4*>(srow + src(j) + d0);
  }
  for (uint32_t p = 1; p < a.nplanes; p += PLANES) {  // uniform
    float4 w[PLANES][JOBS];
#pragma unroll
    for (int u = 0; u < PLANES; u++) {
      const float* prow = srow + (size_t)min(p + u, a.nplanes - 1) * a.plane_stride;
#pragma unroll
      for (int i = 0; i < JOBS; i++) {
        const uint32_t j = min(j0 + jstride * (uint32_t)i, njobs - 1);
        w[u][i] = *reinterpret_cast<const float4*>(prow + src(j) + d0);
      }
    }
#pragma unroll
    for (int u = 0; u < PLANES; u++)
      if (p + u < a.nplanes) {  // uniform
#pragma unroll
        for (int i = 0; i < JOBS; i++)
          v[i] = make_float4(v[i].x + w[u][i].x, v[i].y + w[u][i].y, v[i].z + w[u][i].z,
                             v[i].w + w[u][i].w);
      }
  }
  const float4 one = make_float4(1.f, 1.f, 1.f, 1.f);  // a missing norm weight
  const float4 wq = a.q_norm ? *reinterpret_cast<const float4*>(a.q_norm + d0) : one;
  const float4 wk = a.k_norm ? *reinterpret_cast<const float4*>(a.k_norm + d0) : one;
  float rc[ROPE_K], rsn[ROPE_K];
  rope_angles(a.rot, a.theta, clock, lane, rc, rsn);
  float* h = hb[wave];
#pragma unroll
  for (int i = 0; i < JOBS; i++) {
    if ((uint32_t)i < per) {  // per is the same for the whole workgroup
      const uint32_t j = j0 + jstride * (uint32_t)i;
      const bool isq = j < nq, isk = !isq && j < nq + nkv;
      const float4 x = v[i];
      const float ss = wave_allsum(x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w);
      const float inv = 1.0f / sqrtf(ss / 256.0f + a.eps);
      const float4 w = isq ? wq : isk ? wk : one;
      *reinterpret_cast<float4*>(h + d0) =
          make_float4(x.x * inv * w.x, x.y * inv * w.y, x.z * inv * w.z, x.w * inv * w.w);
      __syncthreads();
      if (isq || isk) rope_lds(h, a.rot, rc, rsn, lane);
      __syncthreads();
      const float4 y = *reinterpret_cast<const float4*>(h + d0);
      if (j < njobs) {
        float* dst = isq ? row + (size_t)j * 256
                     : isk ? a.k_cache + (size_t)slot * kv_dim + (size_t)(j - nq) * 256
                           : a.v_cache + (size_t)slot * kv_dim + (size_t)(j - nq - nkv) * 256;
        *reinterpret_cast<float4*>(dst + d0) = y;
      }
    }
  }
}
extern "C" __global__ __launch_bounds__(ATT_NT) void gh_pf_qkv_rope4_k(AttnArgs a,
                                                                      const uint32_t* clocks,
                                                                      const uint32_t* slots) {
  pf_qkv_rope4<16, 1>(a, clocks, slots);
}
extern "C" __global__ __launch_bounds__(ATT_NT) void gh_pf_qkv_rope4_s_k(AttnArgs a,
                                                                        const uint32_t* clocks,
                                                                        const uint32_t* slots) {
  pf_qkv_rope4<2, 8>(a, clocks, slots);
}

// Combine the split partials of one query head:
// out = sum_s exp(m_s - M) o_s / sum_s exp(m_s - M) l_s.  One workgroup of
// 256 threads per query head; wave w takes splits w, w + 4, ...  Every load
// of the common case (D <= 256, up to 32 splits) -- the thread's (m, l) and
// its partial-row slices -- is issued before any is used, with clamped
// indices, so the kernel costs one L2 round trip; only the weights wait for
// the block-wide max.  The four waves' sums combine in wave order through LDS.
#define MERGE_U 8
// GATED: as in attn_decode, the run flag is loaded at entry and tested just
// before the output row is written.
// PF: the batched prefill's split partials, one workgroup per (query head,
// token blockIdx.y); all a.nsplit splits ran; the output row goes to out_rows.
template <bool GATED, bool PF = false>
__device__ __forceinline__ void attn_merge(const AttnArgs& a) {
  __shared__ float c[MAX_SPLIT];
  __shared__ float red[ATT_WAVES];
  __shared__ float4 acc[ATT_WAVES][MAX_D / 4];
  const uint32_t D = a.D, G = a.nq / a.nkv, h = blockIdx.x, tid = threadIdx.x;
  const uint32_t lane = tid & 63, wave = tid >> 6;
  const uint32_t go = GATED ? *a.run : 1u;
  const uint32_t kvh = h / G, g = h % G, PS = D + 4;
  const uint32_t tok = PF ? blockIdx.y : 0u;
  // the splits that ran
  const uint32_t ns = PF ? a.nsplit : attn_live_splits(a.nsplit, a.step[2]);
  const float* allp =
      a.part + ((size_t)tok * a.nkv + kvh) * a.nsplit * G * PS + (size_t)g * PS;
  const size_t stride = (size_t)G * PS;  // one split to the next
  const uint32_t D4 = D / 4;
  auto row = [&](uint32_t sp, uint32_t col) {  // clamped: out-of-range reads get weight 0
    sp = sp < ns ? sp : ns - 1;
    col = col < D4 ? col : D4 - 1;
    return *reinterpret_cast<const float4*>(allp + sp * stride + col * 4);
  };
  // thread t owns split t's (m, l) (ns <= 256); the first column pass's rows
  const uint32_t tc = tid < ns ? tid : ns - 1;
  const float2 mlv = *reinterpret_cast<const float2*>(allp + tc * stride + D);
  float4 t0[MERGE_U];
#pragma unroll
  for (int u = 0; u < MERGE_U; u++) t0[u] = row(wave + u * ATT_WAVES, lane);
  const float ms = tid < ns ? mlv.x : -INFINITY;
  const float ls = tid < ns ? mlv.y : 0.f;
  float M = ms;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
  if (lane == 0) red[wave] = M;
  __syncthreads();
  M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float cs = ms == -INFINITY ? 0.f : __expf(ms - M);
  if (tid < ns) c[tid] = cs;
  float L = wave_allsum(cs * ls);
  __syncthreads();  // red[] reads done, c[] written
  if (lane == 0) red[wave] = L;
  __syncthreads();
  L = (red[0] + red[1]) + (red[2] + red[3]);
  const float inv = L > 0.f ? 1.0f / L : 0.f;
  // weighted column sums: lane -> float4 column, wave -> splits w, w+4, ...
  if (D4 <= 64 && ns <= ATT_WAVES * MERGE_U) {
    // one pass (D <= 256, up to 32 splits): the rows loaded first are all
    // there is, summed straight-line in the order of the general loop below
    // (0.25 us faster per launch than running that loop once)
    float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int u = 0; u < MERGE_U; u++) {
      const uint32_t sp = wave + u * ATT_WAVES;
      const float w = sp < ns ? c[sp] : 0.f;
      O.x += t0[u].x * w;
      O.y += t0[u].y * w;
      O.z += t0[u].z * w;
      O.w += t0[u].w * w;
    }
    if (lane < D4) acc[wave][lane] = O;
  } else
  for (uint32_t col = lane; col < D4; col += 64) {
    float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
    for (uint32_t sp0 = wave; sp0 < ns; sp0 += ATT_WAVES * MERGE_U) {
      float4 t[MERGE_U];
      const bool first = col == lane && sp0 == wave;
#pragma unroll
      for (int u = 0; u < MERGE_U; u++) t[u] = first ? t0[u] : row(sp0 + u * ATT_WAVES, col);
#pragma unroll
      for (int u = 0; u < MERGE_U; u++) {
        const uint32_t sp = sp0 + u * ATT_WAVES;
        const float w = sp < ns ? c[sp] : 0.f;
        O.x += t[u].x * w;
        O.y += t[u].y * w;
        O.z += t[u].z * w;
        O.w += t[u].w * w;
      }
    }
    acc[wave][col] = O;
  }
  __syncthreads();
  if (GATED && go == 0u) return;  // a gated-off layer
  for (uint32_t col = tid; col < D4; col += ATT_NT) {
    const float4 a0 = acc[0][col], a1 = acc[1][col], a2 = acc[2][col], a3 = acc[3][col];
    float4 r;
    r.x = ((a0.x + a1.x) + (a2.x + a3.x)) * inv;
    r.y = ((a0.y + a1.y) + (a2.y + a3.y)) * inv;
    r.z = ((a0.z + a1.z) + (a2.z + a3.z)) * inv;
    r.w = ((a0.w + a1.w) + (a2.w + a3.w)) * inv;
    float* orow = PF ? a.out_rows + (size_t)tok * a.out_stride : a.out;
    *reinterpret_cast<float4*>(orow + (size_t)h * D + col * 4) = r;
  }
}

extern "C" __global__ __launch_bounds__(ATT_NT) void gh_attn_merge_k(AttnArgs a) { attn_merge<false>(a); }
extern "C" __global__ __launch_bounds__(ATT_NT) void gh_attn_merge_q_k(AttnArgs a) { attn_merge<true>(a); }
extern "C" __global__ __launch_bounds__(ATT_NT) void gh_pf_attn_merge_k(AttnArgs a) {
  attn_merge<false, true>(a);
}

// ---------------------------------------------------------------------------
// Matrix-core batched prefill attention, head_dim 256, fp32 throughout.
//
// Grid (kv heads, token groups), long and short groups paired.  A group
// is 16 / G consecutive tokens, so its query vectors form 16 columns (column
// c: token c / G, head c % G); the host's union list holds (slot, token mask)
// pairs.  The four waves take the union's 16-slot tiles in turn, and per tile
//   S^T (16 slots x 16 columns) = K . Q^T      64 x v_mfma_f32_16x16x4_f32
//   O^T (256 dims x 16 columns) += V^T . P^T   64 x v_mfma_f32_16x16x4_f32
// with the online softmax in between.  Operand mapping (lane l, column
// l % 16, lane group l / 16):
//   K . Q^T: the k index of step (j, c) is dim (l/16)*64 + 4j + c, so a lane
//     loads 64 contiguous floats of its K row (slot l % 16 of the tile) and
//     reads the same dims of column l % 16's query from LDS.  The result
//     lands as S[column l % 16][slot 4*(l/16) + r], r = 0..3 --
//   which is the B operand of V^T . P^T when the k index of step r is slot
//     4*(l/16) + r: the probabilities feed the second product without a
//     shuffle.  Its A operand row i of output tile t is dim 16 i + t, so a
//     lane loads 16 contiguous floats (dims 16*(l%16) ..) of each of its 4
//     V rows; the result O[column l%16][16*(4*(l/16) + r) + t] sits in o[t][r].
// The row max and row sum of the softmax reduce over r in the lane and over
// the 4 lane groups with lane swaps, so every lane of a column holds the same
// (m, l).  The waves merge through LDS in wave order and write each token's
// output rows.  Products and sums are fp32; only the summation order differs
// from the per-token kernel.
// ---------------------------------------------------------------------------
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 mfma_f32_4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ float swap16_max(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float swap32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

#define PFM_D 256
struct PfmEntries {
  uint32_t kslot;     // K row: slot of tile entry l % 16
  uint32_t vslot[4];  // V rows / scores: tile entries 4*(l/16) + r
  uint32_t vmask[4];  // their token masks (0 past the end of the list)
};
__device__ __forceinline__ void pfm_entries(const uint32_t* list, uint32_t S, uint32_t tile,
                                            uint32_t col, uint32_t quad, PfmEntries& e) {
  const uint32_t e0 = tile * 16;
  e.kslot = list[2 * min(e0 + col, S - 1)];
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const uint32_t i = e0 + 4 * quad + r, ic = min(i, S - 1);
    e.vslot[r] = list[2 * ic];
    e.vmask[r] = i < S ? list[2 * ic + 1] : 0u;
  }
}

extern "C" __global__ __launch_bounds__(ATT_NT, 2) void gh_pf_attn_m_k(AttnArgs a) {
  // 64 KB: the query operand (16 steps x 64 lanes of float4) during the
  // loop, then the waves' o registers ([wave][64 regs][64 lanes]) for the merge
  __shared__ float4 smem4[ATT_WAVES * 64 * 64 / 4];
  __shared__ float wm[ATT_WAVES][16], wl[ATT_WAVES][16];
  float4* qs4 = smem4;
  float* wo = reinterpret_cast<float*>(smem4);

  const uint32_t G = a.nq / a.nkv;
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t col = lane & 15, quad = lane >> 4;
  const size_t kv_dim = (size_t)a.nkv * PFM_D;
  // group order: the first half of blockIdx.y runs the longest groups in
  // descending order, the second half the shortest in ascending order, so the
  // workgroups y and y + half that share a CU sum to about the same work
  const uint32_t gy = gridDim.y, half = (gy + 1) / 2, y = blockIdx.y;
  const uint32_t kvh = blockIdx.x, grp = y < half ? gy - 1 - y : y - half;
  const uint32_t t0 = grp * (16 / G);
  const uint32_t S = a.n_active[grp];
  const uint32_t* list = a.active + (size_t)grp * a.active_stride;
  const uint32_t ntiles = (S + 15) / 16;

  // 1. query columns into LDS in operand order: qs4[j * 64 + l] = dims
  //    (l/16)*64 + 4j .. +4 of column l % 16 (zeros past the last token)
  for (uint32_t i = tid; i < 16 * 64; i += ATT_NT) {
    const uint32_t j = i >> 6, ln = i & 63, c = ln & 15;
    const uint32_t t = t0 + c / G, g = c % G;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (t < a.n_tokens)
      v = *reinterpret_cast<const float4*>(a.q + (size_t)t * a.q_stride +
                                           (size_t)(kvh * G + g) * PFM_D + (ln >> 4) * 64 + 4 * j);
    qs4[i] = v;
  }
  // entries of this wave's first two tiles (indices clamped into the list, so
  // every load below is unconditional and in bounds, and masks past the end
  // are zero)
  PfmEntries cur, nxt;
  pfm_entries(list, S, wave, col, quad, cur);
  pfm_entries(list, S, wave + ATT_WAVES, col, quad, nxt);
  __syncthreads();

  // 2. the wave's tiles: scores, online softmax, weighted V
  const uint32_t bit = col / G;  // this column's token within the group
  f32x4 o[16];
#pragma unroll
  for (int t = 0; t < 16; t++) o[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;
  const float* kb = a.k_cache + (size_t)kvh * PFM_D + quad * 64;
  const float* vb = a.v_cache + (size_t)kvh * PFM_D + col * 16;
  // The first half of tile i + 4's K rows loads while tile i's V . P
  // products run, the second half at the top of its iteration, and its V
  // rows once the first half's score products have freed their registers.
  // This keeps a wave within 256 registers (two waves per SIMD).
  float4 kr[16], vr[4][4];
  {
    const float4* kp = reinterpret_cast<const float4*>(kb + (size_t)cur.kslot * kv_dim);
#pragma unroll
    for (int j = 0; j < 8; j++) kr[j] = kp[j];
  }
  for (uint32_t tile = wave; tile < ntiles; tile += ATT_WAVES) {
    {
      const float4* kp = reinterpret_cast<const float4*>(kb + (size_t)cur.kslot * kv_dim);
#pragma unroll
      for (int j = 8; j < 16; j++) kr[j] = kp[j];
    }

    // four independent accumulation chains (one per float4 component)
    f32x4 s0 = f32x4{0.f, 0.f, 0.f, 0.f}, s1 = s0, s2 = s0, s3 = s0;
#pragma unroll
    for (int j = 0; j < 16; j++) {
      if (j == 8) {  // the first half's K registers are free: V rows load now
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const float4* vp = reinterpret_cast<const float4*>(vb + (size_t)cur.vslot[r] * kv_dim);
#pragma unroll
          for (int i = 0; i < 4; i++) vr[r][i] = vp[i];
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      const float4 q4 = qs4[j * 64 + lane];
      s0 = mfma_f32_4(kr[j].x, q4.x, s0);
      s1 = mfma_f32_4(kr[j].y, q4.y, s1);
      s2 = mfma_f32_4(kr[j].z, q4.z, s2);
      s3 = mfma_f32_4(kr[j].w, q4.w, s3);
    }
    const f32x4 s = (s0 + s1) + (s2 + s3);
    __builtin_amdgcn_sched_barrier(0);  // K registers are free from here on
    {
      const float4* kp = reinterpret_cast<const float4*>(kb + (size_t)nxt.kslot * kv_dim);
#pragma unroll
      for (int j = 0; j < 8; j++) kr[j] = kp[j];
    }
    uint32_t vmask[4];
#pragma unroll
    for (int r = 0; r < 4; r++) vmask[r] = cur.vmask[r];
    cur = nxt;
    pfm_entries(list, S, tile + 2 * ATT_WAVES, col, quad, nxt);
    float sv[4], mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      sv[r] = s[r] * a.scale;
      if ((vmask[r] >> bit) & 1u) mx = fmaxf(mx, sv[r]);
    }
    mx = swap32_max(swap16_max(mx));
    const float mt = fmaxf(m, mx);
    const float corr = mt == -INFINITY ? 1.f : __expf(m - mt);  // m = -inf, mt finite: 0
    float p[4], ps = 0.f;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      p[r] = (vmask[r] >> bit) & 1u ? __expf(sv[r] - mt) : 0.f;
      ps += p[r];
    }
    ps = swap32_add(swap16_add(ps));
    l = l * corr + ps;
    m = mt;
#pragma unroll
    for (int t = 0; t < 16; t++) o[t] *= corr;
#pragma unroll
    for (int r = 0; r < 4; r++) {
#pragma unroll
      for (int t = 0; t < 16; t++) {  // consecutive products into different tiles
        const float4 v4 = vr[r][t >> 2];
        const float v = (t & 3) == 0 ? v4.x : (t & 3) == 1 ? v4.y : (t & 3) == 2 ? v4.z : v4.w;
        o[t] = mfma_f32_4(v, p[r], o[t]);
      }
    }
  }

  // 3. merge the four waves (wave order) and write the output rows
  __syncthreads();  // every wave is done with the query operand (aliased below)
#pragma unroll
  for (int t = 0; t < 16; t++) {
#pragma unroll
    for (int r = 0; r < 4; r++) wo[(wave * 64 + t * 4 + r) * 64 + lane] = o[t][r];
  }
  if (quad == 0) {
    wm[wave][col] = m;
    wl[wave][col] = l;
  }
  __syncthreads();
  const uint32_t c = tid >> 4, i = tid & 15;  // output column, dims 16 i .. 16 i + 15
  const uint32_t t = t0 + c / G, g = c % G;
  if (t < a.n_tokens) {
    float M = -INFINITY;
    for (int w = 0; w < ATT_WAVES; w++) M = fmaxf(M, wm[w][c]);
    float cw[ATT_WAVES], L = 0.f;
    for (int w = 0; w < ATT_WAVES; w++) {
      cw[w] = wm[w][c] == -INFINITY ? 0.f : __expf(wm[w][c] - M);
      L += wl[w][c] * cw[w];
    }
    const uint32_t ln = (i >> 2) * 16 + c, r = i & 3;
    float res[16];
#pragma unroll
    for (int d = 0; d < 16; d++) {
      float O = 0.f;
      for (int w = 0; w < ATT_WAVES; w++) O += wo[(w * 64 + d * 4 + r) * 64 + ln] * cw[w];
      res[d] = L > 0.f ? O / L : 0.f;
    }
    float4* dst = reinterpret_cast<float4*>(a.out_rows + (size_t)t * a.out_stride +
                                            (size_t)(kvh * G + g) * PFM_D + i * 16);
#pragma unroll
    for (int j = 0; j < 4; j++) dst[j] = make_float4(res[4 * j], res[4 * j + 1], res[4 * j + 2], res[4 * j + 3]);
  }
}
