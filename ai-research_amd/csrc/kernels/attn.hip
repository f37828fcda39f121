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
// Attention design: one workgroup per (kv head, split of the active list).
// The G = nq / nkv query heads of a kv head share every K/V load (GQA bytes
// are read once).  A wavefront owns 64 lanes x DPL = D dims of a slot (one
// 16-byte load per lane per K or V row for D = 256); its waves take slots
// round-robin with two slots in flight, keep an online softmax (running max,
// running sum, rescaled output) per query head, and merge through LDS.  Each
// split writes (m, l, o) partials; the last split of a kv head to finish
// (device-scope counter, self-resetting) merges them in split order, so the
// result does not depend on scheduling.
#include <hip/hip_runtime.h>
#include <stdint.h>

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

template <int DPL>
__device__ __forceinline__ void load_row(const float* p, float* r) {
  if constexpr (DPL == 4) {
    const float4 t = *reinterpret_cast<const float4*>(p);
    r[0] = t.x; r[1] = t.y; r[2] = t.z; r[3] = t.w;
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

template <int DPL>
__device__ __forceinline__ void attn_body(const AttnArgs& a) {
  __shared__ float qs[MAX_G][MAX_D];
  __shared__ float knew[MAX_D], vnew[MAX_D];
  __shared__ float wm[ATT_WAVES][MAX_G], wl[ATT_WAVES][MAX_G];
  __shared__ float wo[ATT_WAVES][MAX_G][MAX_D];
  __shared__ uint32_t last_flag;

  const uint32_t D = a.D, G = a.nq / a.nkv;
  const uint32_t kvh = blockIdx.x / a.nsplit, split = blockIdx.x % a.nsplit;
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t clock = a.step[0], cur_slot = a.step[1], S = a.step[2];
  const size_t kv_dim = (size_t)a.nkv * D;

  // 1. query heads of this kv group (and, fused, this token's K/V) into LDS
  if (a.fuse) {
    for (uint32_t g = wave; g < G + 2; g += ATT_WAVES) {
      if (g < G) {
        const float* in = a.q + (size_t)(kvh * G + g) * D;
        const float inv = head_inv_rms(in, D, a.eps, lane);
        norm_rope_head(in, a.q_norm, qs[g], D, a.rot, a.theta, inv, clock, lane);
      } else if (g == G) {
        const float* in = a.k_in + (size_t)kvh * D;
        const float inv = head_inv_rms(in, D, a.eps, lane);
        norm_rope_head(in, a.k_norm, knew, D, a.rot, a.theta, inv, clock, lane);
      } else {
        const float* in = (a.k_eq_v ? a.k_in : a.v_in) + (size_t)kvh * D;
        const float inv = head_inv_rms(in, D, a.eps, lane);
        for (uint32_t d = lane; d < D; d += 64) vnew[d] = in[d] * inv;
      }
    }
  } else {
    for (uint32_t i = tid; i < G * D; i += ATT_NT) qs[i / D][i % D] = a.q[(size_t)kvh * G * D + i];
  }
  __syncthreads();
  if (a.fuse && split == 0) {  // ring_buffer.writeKV for this layer
    float* kc = a.k_cache + (size_t)cur_slot * kv_dim + (size_t)kvh * D;
    float* vc = a.v_cache + (size_t)cur_slot * kv_dim + (size_t)kvh * D;
    for (uint32_t d = tid; d < D; d += ATT_NT) {
      kc[d] = knew[d];
      vc[d] = vnew[d];
    }
  }

  // 2. this split's share of the active list
  const uint32_t chunk = (S + a.nsplit - 1) / a.nsplit;
  const uint32_t s0 = split * chunk;
  const uint32_t s1 = min(S, s0 + chunk);
  const uint32_t d0 = lane * DPL;  // this lane's dims
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

  auto fetch = [&](uint32_t si, float* kr, float* vr) {
    const uint32_t slot = a.active[si];
    if (a.fuse && slot == cur_slot) {  // this token's K/V: from LDS, not the cache
#pragma unroll
      for (int j = 0; j < DPL; j++) {
        kr[j] = dl ? knew[d0 + j] : 0.f;
        vr[j] = dl ? vnew[d0 + j] : 0.f;
      }
    } else if (dl) {
      load_row<DPL>(kbase + (size_t)slot * kv_dim, kr);
      load_row<DPL>(vbase + (size_t)slot * kv_dim, vr);
    } else {
#pragma unroll
      for (int j = 0; j < DPL; j++) kr[j] = vr[j] = 0.f;
    }
  };
  auto consume = [&](const float* kr, const float* vr) {
#pragma unroll
    for (int g = 0; g < MAX_G; g++) {
      if (g >= (int)G) break;
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < DPL; j++) s += q[g][j] * kr[j];
      s = wave_sum(s) * a.scale;
      const float mn = fmaxf(m[g], s);
      const float corr = __expf(m[g] - mn);
      const float p = __expf(s - mn);
      l[g] = l[g] * corr + p;
#pragma unroll
      for (int j = 0; j < DPL; j++) o[g][j] = o[g][j] * corr + p * vr[j];
      m[g] = mn;
    }
  };

  // four slots in flight per wave
  uint32_t si = s0 + wave;
  for (; si + 3 * ATT_WAVES < s1; si += 4 * ATT_WAVES) {
    float k0[DPL], v0[DPL], k1[DPL], v1[DPL], k2[DPL], v2[DPL], k3[DPL], v3[DPL];
    fetch(si, k0, v0);
    fetch(si + ATT_WAVES, k1, v1);
    fetch(si + 2 * ATT_WAVES, k2, v2);
    fetch(si + 3 * ATT_WAVES, k3, v3);
    consume(k0, v0);
    consume(k1, v1);
    consume(k2, v2);
    consume(k3, v3);
  }
  for (; si < s1; si += ATT_WAVES) {
    float k0[DPL], v0[DPL];
    fetch(si, k0, v0);
    consume(k0, v0);
  }

  // 3. merge the waves of this workgroup
#pragma unroll
  for (int g = 0; g < MAX_G; g++) {
    if (g >= (int)G) break;
    if (lane == 0) {
      wm[wave][g] = m[g];
      wl[wave][g] = l[g];
    }
    if (dl) {
#pragma unroll
      for (int j = 0; j < DPL; j++) wo[wave][g][d0 + j] = o[g][j];
    }
  }
  __syncthreads();
  const uint32_t PS = D + 4;  // partial record: o[D], m, l (+2 pad: float4 rows)
  float* part = a.part + ((size_t)kvh * a.nsplit + split) * G * PS;
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

  // 4. the last split of this kv head merges all partials in split order
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const uint32_t prev = atomicAdd(&a.counters[kvh], 1u);
    last_flag = (prev == a.nsplit - 1) ? 1u : 0u;
  }
  __syncthreads();
  if (!last_flag) return;
  __threadfence();
  __shared__ float sm[MAX_G][MAX_SPLIT], sc[MAX_G][MAX_SPLIT], sL[MAX_G];
  const float* allp = a.part + (size_t)kvh * a.nsplit * G * PS;
  for (uint32_t i = tid; i < G * a.nsplit; i += ATT_NT) {
    const uint32_t g = i / a.nsplit, sp = i % a.nsplit;
    sm[g][sp] = allp[(sp * G + g) * PS + D];
    sc[g][sp] = allp[(sp * G + g) * PS + D + 1];  // l for now
  }
  __syncthreads();
  if (tid < G) {  // per query head: running max, weights c_s, and L
    float M = -INFINITY;
    for (uint32_t sp = 0; sp < a.nsplit; sp++) M = fmaxf(M, sm[tid][sp]);
    float L = 0.f;
    for (uint32_t sp = 0; sp < a.nsplit; sp++) {
      const float c = sm[tid][sp] == -INFINITY ? 0.f : __expf(sm[tid][sp] - M);
      L += sc[tid][sp] * c;
      sc[tid][sp] = c;
    }
    sL[tid] = L;
  }
  __syncthreads();
  const uint32_t D4 = D / 4;
  for (uint32_t i = tid; i < G * D4; i += ATT_NT) {
    const uint32_t g = i / D4, d = (i % D4) * 4;
    float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
    uint32_t sp = 0;
    for (; sp + 8 <= a.nsplit; sp += 8) {
      float4 t[8];
#pragma unroll
      for (int u = 0; u < 8; u++)
        t[u] = *reinterpret_cast<const float4*>(allp + ((sp + u) * G + g) * PS + d);
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const float c = sc[g][sp + u];
        O.x += t[u].x * c;
        O.y += t[u].y * c;
        O.z += t[u].z * c;
        O.w += t[u].w * c;
      }
    }
    for (; sp < a.nsplit; sp++) {
      const float4 t = *reinterpret_cast<const float4*>(allp + (sp * G + g) * PS + d);
      const float c = sc[g][sp];
      O.x += t.x * c;
      O.y += t.y * c;
      O.z += t.z * c;
      O.w += t.w * c;
    }
    const float L = sL[g];
    const float inv = L > 0.f ? 1.0f / L : 0.f;
    float* o = a.out + (size_t)(kvh * G + g) * D + d;
    o[0] = O.x * inv;
    o[1] = O.y * inv;
    o[2] = O.z * inv;
    o[3] = O.w * inv;
  }
  if (tid == 0) a.counters[kvh] = 0;  // ready for the next launch
}

extern "C" __global__ __launch_bounds__(ATT_NT) void gh_attn_d4_k(AttnArgs a) { attn_body<4>(a); }
extern "C" __global__ __launch_bounds__(ATT_NT) void gh_attn_d2_k(AttnArgs a) { attn_body<2>(a); }
extern "C" __global__ __launch_bounds__(ATT_NT) void gh_attn_d8_k(AttnArgs a) { attn_body<8>(a); }
