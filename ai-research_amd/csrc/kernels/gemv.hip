// gemv.hip -- Q4_0 / Q8_0 dequant GEMV and the fused gate+up GeGLU for gfx950.
//
// Semantics: shaders/gemv_q4.wgsl:13-82, shaders/gemv_q8.wgsl:13-82,
// shaders/fused_mlp_q4.wgsl:20-119 (Y = deq(W) . X; act = gelu_tanh(g) * u).
// Layout: the reference's quant.zig rows, unchanged (Q4_0 = 20 B blocks,
// Q8_0 = 36 B blocks, f32 scale first).
//
// Design (HBM-bound, ~3.2 flop/B):
//  * Work unit = one "group" of 4 consecutive blocks of one row: 80 B (Q4) or
//    144 B (Q8), i.e. 5 or 9 aligned 16-byte loads per lane.  A row's groups
//    are spread over a team of TPR lanes of one wavefront; a lane keeps RPT
//    rows in flight at the same group so each x value read from LDS feeds RPT
//    rows.  Teams reduce with cross-lane shuffles, no LDS.
//  * x is staged once per workgroup in LDS with 4 floats of padding per group
//    (group stride 132 floats) so the TPR lanes of a team, which read
//    different groups at the same offset, land on different LDS banks.
//  * In-register dequant without per-weight int->float of a signed value:
//      sum_j (n_j - 8) d x_j = d (sum_j n_j x_j - 8 sum_j x_j)
//    with the per-block sum_j x_j precomputed while staging x.  Q4: masks
//    cut each word into nibble pairs that, read as two fp16 halves, are the
//    exact denormals n 2^-24 (or 16 n 2^-24); v_fma_mix_f32 multiplies a half
//    by an fp32 x into an fp32 sum, and the powers of two come off once per
//    block.  Q8 flips the sign bit of each byte (q + 128), converts it with
//    one v_cvt_f32_ubyte{0..3} and removes 128 sum x the same way.
//  * fp32 accumulation throughout.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../common/stream_args.h"  // XPro

#define GROUP_STRIDE 132  // floats per 128-element x group in LDS (+4 pad)

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }

// 16-byte weight loads.  Plain loads, not non-temporal: lanes read 80 B
// (Q4) or 144 B (Q8) apart, so each 128-B line is touched by several load
// instructions of the same wave, and the streaming hint evicts it between
// them (measured: 3.4 vs 6.4 TB/s on MI355X for this pattern).
// Explicitly in the global address space: a pointer chosen at run time
// between two arguments otherwise degrades to a FLAT load, which also counts
// against lgkmcnt and so is drained by every LDS wait.
typedef const u32x4 __attribute__((address_space(1)))* gvec_ptr;
__device__ __forceinline__ u32x4 ldw(const void* p) {
  return *(gvec_ptr)(p);
}

// Cross-lane sums with DPP row operations and the gfx950 permlane swaps (a
// few cycles each) instead of __shfl_xor, which lowers to an LDS-crossbar
// ds_bpermute per step.  Every
// step adds a commutative pair, so all participating lanes end with the
// same bit-identical value.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// sum over the 8 lanes of each half-row (lanes 8k .. 8k+7)
__device__ __forceinline__ float sum8(float v) {
  v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp<0x141>(v);  // row_half_mirror
  return v;
}
// v + (v of lane l ^ 16): v_permlane16_swap exchanges rows 1 and 3 of one
// operand with rows 0 and 2 of the other, so with both operands = v the two
// results hold the values of lanes l and l ^ 16 (one VALU op, no LDS).
__device__ __forceinline__ float add_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// v + (v of lane l ^ 32), with v_permlane32_swap (halves of the wavefront)
__device__ __forceinline__ float add_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// sum over the 64 lanes of the wavefront
__device__ __forceinline__ float sum64(float v) {
  v = sum8(v);
  v += dpp<0x140>(v);  // row_mirror
  v = add_xor16(v);
  return add_xor32(v);
}

// Stage x[K] into LDS (padded by group) and write the per-block sums.
// K % 128 == 0.  Called by the first NT threads of the block (whole
// wavefronts); the caller synchronises.  The loads of a
// chunk of U float4 per thread are all issued before any is consumed, so
// staging costs one L2 round trip per chunk.  The loads are unconditional
// (indices clamped into range) and every loaded value is consumed within its
// chunk: a load left pending across the loop's back edge, or one issued
// under a branch, makes the compiler wait for every earlier load -- the
// weight loads in flight included -- before issuing the next.
template <int NT>
__device__ __forceinline__ void stage_x(const float* __restrict__ X, uint32_t K,
                                        float* xs, float* bsum) {
  constexpr uint32_t U = 8;  // float4 per thread per round
  const uint32_t n4 = K >> 2;
  const float4* X4 = reinterpret_cast<const float4*>(X);
  for (uint32_t base = 0; base < n4; base += NT * U) {
    float4 v[U];
#pragma unroll
    for (uint32_t u = 0; u < U; u++) {
      const uint32_t i = base + u * NT + threadIdx.x;
      v[u] = X4[i < n4 ? i : n4 - 1];
    }
#pragma unroll
    for (uint32_t u = 0; u < U; u++) {
      const uint32_t i = base + u * NT + threadIdx.x;
      const uint32_t e = i << 2;               // element index
      const uint32_t g = e >> 7, o = e & 127;  // group, offset in group
      float s = (v[u].x + v[u].y) + (v[u].z + v[u].w);
      if (i < n4) *reinterpret_cast<float4*>(xs + g * GROUP_STRIDE + o) = v[u];
      // a block is 8 consecutive float4s = the 8 lanes of a half-row (n4 % 8
      // == 0, so a half-row is either fully in range or fully out)
      s = sum8(s);
      if (i < n4 && (i & 7) == 0) bsum[i >> 3] = s;
    }
  }
}

// Nibble/byte masks go through an opaque v_and_b32: when the compiler sees
// the 0x0F0F0F0F mask it folds "(lo >> 8) & 0xFF" into a 4-bit field extract
// and loses the one-instruction v_cvt_f32_ubyte{0..3} form.  With the mask
// hidden it selects v_cvt_f32_ubyteN for every byte itself and schedules it.
__device__ __forceinline__ uint32_t opaque_and(uint32_t w, uint32_t m) {
  uint32_t r;
  asm("v_and_b32 %0, %1, %2" : "=v"(r) : "v"(m), "v"(w));
  return r;
}

__device__ __forceinline__ float ub0(uint32_t x) { return (float)(x & 0xFFu); }
__device__ __forceinline__ float ub1(uint32_t x) { return (float)((x >> 8) & 0xFFu); }
__device__ __forceinline__ float ub2(uint32_t x) { return (float)((x >> 16) & 0xFFu); }
__device__ __forceinline__ float ub3(uint32_t x) { return (float)(x >> 24); }

// Nibble pairs as fp16 denormals: (w & 0x000F000F) read as two halves is
// exactly (n_a 2^-24, n_b 2^-24), and v_fma_mix_f32 multiplies one half by an
// fp32 x into an fp32 sum, so no weight needs its own conversion: 8 weights
// cost 4 masks, 1 shift and 8 FMAs (v_cvt_f32_ubyte per weight: 2 + 8 + 8).
// Every product and partial sum is the conversion form's times 2^-24 (exact),
// in the same order, so the results are bit-identical to it.
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ h2_t nib_pair(uint32_t w, uint32_t m) {
  return __builtin_bit_cast(h2_t, opaque_and(w, m));
}
// One word (elements 8k .. 8k+7, xa = x[8k..8k+3], xc = x[8k+4..8k+7]):
// sl += 2^-24 (n0 x0 + n2 x2 + n4 x4 + n6 x6), sh += 2^-20 (n1 x1 + ... + n7 x7)
__device__ __forceinline__ void q4_word(uint32_t w, const float4& xa, const float4& xc, float& sl,
                                        float& sh) {
  const uint32_t t = w >> 8;
  const h2_t p0 = nib_pair(w, 0x000F000Fu);  // elements 0, 4
  const h2_t p1 = nib_pair(w, 0x00F000F0u);  // 16 x elements 1, 5
  const h2_t p2 = nib_pair(t, 0x000F000Fu);  // elements 2, 6
  const h2_t p3 = nib_pair(t, 0x00F000F0u);  // 16 x elements 3, 7
  sl = __builtin_fmaf((float)p0.x, xa.x, sl);
  sh = __builtin_fmaf((float)p1.x, xa.y, sh);
  sl = __builtin_fmaf((float)p2.x, xa.z, sl);
  sh = __builtin_fmaf((float)p3.x, xa.w, sh);
  sl = __builtin_fmaf((float)p0.y, xc.x, sl);
  sh = __builtin_fmaf((float)p1.y, xc.y, sh);
  sl = __builtin_fmaf((float)p2.y, xc.z, sl);
  sh = __builtin_fmaf((float)p3.y, xc.w, sh);
}
// sum_j n_j x_j from a block's two q4_word sums
__device__ __forceinline__ float q4_sum(float sl, float sh) {
  return (sl + sh * 0.0625f) * 16777216.0f;
}

// sum_j n_j x_j over one Q4 block, n_j = nibble j (0..15).
__device__ __forceinline__ float q4_nx(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3,
                                       const float* __restrict__ xb) {
  const uint32_t w[4] = {w0, w1, w2, w3};
  float sl = 0.f, sh = 0.f;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const float4 xa = *reinterpret_cast<const float4*>(xb + 8 * k);
    const float4 xc = *reinterpret_cast<const float4*>(xb + 8 * k + 4);
    q4_word(w[k], xa, xc, sl, sh);
  }
  return q4_sum(sl, sh);
}

// sum_j (q_j + 128) x_j over one Q8 block given its 8 packed words.
__device__ __forceinline__ float q8_ux(const uint32_t* w, const float* __restrict__ xb) {
  float s0 = 0.f, s1 = 0.f;
#pragma unroll
  for (int k = 0; k < 8; k++) {
    const uint32_t u = opaque_and(w[k] ^ 0x80808080u, 0xFFFFFFFFu);  // int8 q -> uint8 q + 128
    const float4 xa = *reinterpret_cast<const float4*>(xb + 4 * k);
    s0 += ub0(u) * xa.x;
    s1 += ub1(u) * xa.y;
    s0 += ub2(u) * xa.z;
    s1 += ub3(u) * xa.w;
  }
  return s0 + s1;
}

struct Q4G {
  u32x4 a0, a1, a2, a3, a4;
};

__device__ __forceinline__ Q4G load_q4g(const uint8_t* p) {
  Q4G g;
  g.a0 = ldw(p + 0);
  g.a1 = ldw(p + 16);
  g.a2 = ldw(p + 32);
  g.a3 = ldw(p + 48);
  g.a4 = ldw(p + 64);
  return g;
}

// Dot of one 4-block Q4 group with x; words: block j at 5j .. 5j+4.
__device__ __forceinline__ float q4_group_dot(const Q4G& g, const float* __restrict__ xg,
                                              const float* __restrict__ bs) {
  float r;
  r = u2f(g.a0.x) * (q4_nx(g.a0.y, g.a0.z, g.a0.w, g.a1.x, xg) - 8.0f * bs[0]);
  r += u2f(g.a1.y) * (q4_nx(g.a1.z, g.a1.w, g.a2.x, g.a2.y, xg + 32) - 8.0f * bs[1]);
  r += u2f(g.a2.z) * (q4_nx(g.a2.w, g.a3.x, g.a3.y, g.a3.z, xg + 64) - 8.0f * bs[2]);
  r += u2f(g.a3.w) * (q4_nx(g.a4.x, g.a4.y, g.a4.z, g.a4.w, xg + 96) - 8.0f * bs[3]);
  return r;
}

// Sum over a row team of TPR (16, 32 or 64) consecutive lanes.
template <int TPR>
__device__ __forceinline__ float team_sum(float v) {
  static_assert(TPR == 16 || TPR == 32 || TPR == 64, "team of 16, 32 or 64 lanes");
  v = sum8(v);
  v += dpp<0x140>(v);  // row_mirror: the two half-rows of a row of 16
  if (TPR >= 32) v = add_xor16(v);
  if (TPR == 64) v = add_xor32(v);
  return v;
}

__device__ __forceinline__ float gelu_tanh(float x) {
  // kernels.zig:94-97 / fused_mlp_q4.wgsl:15-18
  const float inner = 0.7978845608f * (x + 0.044715f * x * x * x);
  return 0.5f * x * (1.0f + tanhf(inner));
}

// ------------------------------------------------------------------------
// x prologue.  The decode step fuses the reference's separate norm
// dispatches (src/gpu/model_dispatch.zig:21,32-34,39-41,122) into the GEMV
// that consumes their output; every workgroup recomputes the (cheap) norm of
// one hidden vector while its first weight loads are in flight.
//   mode 0: x as given
//   mode 1: RMSNorm(x) * w                                   (input / final norm)
//   mode 2: xn = (x + r') * s with r' = RMSNorm(r) * wr (r as given when wr
//           is null); workgroup 0 writes xn to xout (the residual stream);
//           the GEMV consumes RMSNorm(xn) * w                  (add + norm)
// Every norm is in * (mean(in^2) + eps)^-1/2 * w, as src/kernels.zig:46-52
// (which divides 1 by the square root; here v_rsq_f32, within 1 ulp of it).
// ------------------------------------------------------------------------
// (mean + eps)^-1/2 of a norm: v_rsq_f32 (1 ulp) instead of the correctly
// rounded sqrt and divide (about 40 instructions per wavefront, which every
// wavefront of every workgroup runs on the launch's critical path; with the
// scale folded below, 0.25 us less per normed stream launch).
__device__ __forceinline__ float norm_rsqrt(float mean_sq_eps) {
  return __builtin_amdgcn_rsqf(mean_sq_eps);
}

// Block-wide sums of NV values per thread; every thread gets the totals.
// red holds (NT / 64) * NV floats and must not be reused before a barrier.
template <int NT, int NV>
__device__ __forceinline__ void block_sums(float (&v)[NV], float* red) {
#pragma unroll
  for (int j = 0; j < NV; j++) v[j] = sum64(v[j]);
  if ((threadIdx.x & 63) == 0) {
#pragma unroll
    for (int j = 0; j < NV; j++) red[(threadIdx.x >> 6) * NV + j] = v[j];
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < NV; j++) {
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < NT / 64; w++) t += red[w * NV + j];
    v[j] = t;
  }
}

// Extra LDS (floats) the prologue and epilogues need beyond the padded x and
// block sums (the host adds 4 * this many bytes).
__host__ __device__ constexpr uint32_t pro_extra_floats() { return 64; }

// Largest K of a normed prologue: each thread holds its float4 slices of x,
// r and the two norm weights in registers (PRO_U per vector).
#define PRO_U 4

// The normed prologue takes one block-wide reduction, not two: for mode 2,
// with q = r * wr and c = (mean(r^2) + eps)^-1/2 (q = r, c = 1 without wr),
//   sum(xn^2) = s^2 (sum x^2 + 2 c sum x q + c^2 sum q^2)
// so the four sums go through one reduction.  Only if that expansion
// cancels (the total below 1e-3 of its positive terms) is sum(xn^2)
// reduced directly from xn, as a second pass.
// The prologue's inputs (float4 slices of x, r, wr and w per thread).
struct ProIn {
  float4 vx[PRO_U], vr[PRO_U], vwr[PRO_U], vw[PRO_U];
};

// Issue the loads of the vectors the mode reads (clamped indices, branches
// uniform over the launch), so they go out before the stream's first weight
// loads and complete first.  Each 15 KB vector every workgroup reads costs
// about 0.5 us in a 15360 x 3840 gate+up stream on MI355X (L2 traffic of
// 768 workgroups), so vectors a mode does not use are not loaded.
template <int NT>
__device__ __forceinline__ void pro_load(const XPro& p, uint32_t K, ProIn& in) {
  const uint32_t n4 = K >> 2;
  const bool add = p.mode == 2, norm = p.mode >= 1, has_wr = add && p.wr;
  const float4* x = reinterpret_cast<const float4*>(p.x);
  const float4* w = reinterpret_cast<const float4*>(p.w);
  const float4* r = reinterpret_cast<const float4*>(p.r);
  const float4* wr = reinterpret_cast<const float4*>(p.wr);
#pragma unroll
  for (uint32_t u = 0; u < PRO_U; u++) {
    uint32_t i = u * NT + threadIdx.x;
    i = i < n4 ? i : n4 - 1;
    in.vx[u] = x[i];
    if (norm) in.vw[u] = w[i];
    if (add) in.vr[u] = r[i];
    if (has_wr) in.vwr[u] = wr[i];
  }
}

template <int NT>
__device__ __forceinline__ void pro_finish(const XPro& p, uint32_t K, ProIn& in, float* xs,
                                           float* bsum, float* ext) {
  const uint32_t n4 = K >> 2;
  float4* vx = in.vx;
  const float4* vr = in.vr;
  const float4* vwr = in.vwr;
  const float4* vw = in.vw;
  if (p.mode == 0) {  // x as given
#pragma unroll
    for (uint32_t u = 0; u < PRO_U; u++) {
      const uint32_t i = u * NT + threadIdx.x;
      const uint32_t e = i << 2, g = e >> 7, o = e & 127;
      if (i < n4) *reinterpret_cast<float4*>(xs + g * GROUP_STRIDE + o) = vx[u];
      const float s = sum8((vx[u].x + vx[u].y) + (vx[u].z + vx[u].w));
      if (i < n4 && (i & 7) == 0) bsum[i >> 3] = s;
    }
    __syncthreads();
    return;
  }
  const bool add = p.mode == 2;
  const bool has_wr = p.wr != nullptr;
  float inv;
  if (add) {
    float t[4] = {0.f, 0.f, 0.f, 0.f};  // sum r^2, x^2, x q, q^2
#pragma unroll
    for (uint32_t u = 0; u < PRO_U; u++) {
      if (u * NT + threadIdx.x < n4) {
        const float r[4] = {vr[u].x, vr[u].y, vr[u].z, vr[u].w};
        const float x[4] = {vx[u].x, vx[u].y, vx[u].z, vx[u].w};
        const float w[4] = {vwr[u].x, vwr[u].y, vwr[u].z, vwr[u].w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const float q = has_wr ? r[e] * w[e] : r[e];
          t[0] += r[e] * r[e];
          t[1] += x[e] * x[e];
          t[2] += x[e] * q;
          t[3] += q * q;
        }
      }
    }
    block_sums<NT, 4>(t, ext);
    const float c = has_wr ? norm_rsqrt(t[0] / (float)K + p.eps) : 1.0f;
    const float pos = t[1] + c * c * t[3];
    float s2 = p.s * p.s * (pos + 2.0f * c * t[2]);
    // vx becomes x + r' and xn = s (x + r'): the scale s is applied once, in
    // inv below, except in workgroup 0's residual write
#pragma unroll
    for (uint32_t u = 0; u < PRO_U; u++) {
      const uint32_t i = u * NT + threadIdx.x;
      if (i < n4) {
        float4 rv = vr[u];
        if (has_wr) {
          rv.x = rv.x * c * vwr[u].x;
          rv.y = rv.y * c * vwr[u].y;
          rv.z = rv.z * c * vwr[u].z;
          rv.w = rv.w * c * vwr[u].w;
        }
        vx[u].x += rv.x;
        vx[u].y += rv.y;
        vx[u].z += rv.z;
        vx[u].w += rv.w;
        if (blockIdx.x == 0)
          reinterpret_cast<float4*>(p.xout)[i] =
              make_float4(vx[u].x * p.s, vx[u].y * p.s, vx[u].z * p.s, vx[u].w * p.s);
      }
    }
    if (!(s2 > 1e-3f * p.s * p.s * pos)) {  // cancellation (uniform branch): reduce xn^2 itself
      float d[1] = {0.f};
#pragma unroll
      for (uint32_t u = 0; u < PRO_U; u++)
        if (u * NT + threadIdx.x < n4)
          d[0] += vx[u].x * vx[u].x + vx[u].y * vx[u].y + vx[u].z * vx[u].z + vx[u].w * vx[u].w;
      block_sums<NT, 1>(d, ext + 4 * (NT / 64));
      s2 = p.s * p.s * d[0];
    }
    inv = norm_rsqrt(s2 / (float)K + p.eps) * p.s;
  } else {
    float d[1] = {0.f};
#pragma unroll
    for (uint32_t u = 0; u < PRO_U; u++)
      if (u * NT + threadIdx.x < n4)
        d[0] += vx[u].x * vx[u].x + vx[u].y * vx[u].y + vx[u].z * vx[u].z + vx[u].w * vx[u].w;
    block_sums<NT, 1>(d, ext);
    inv = norm_rsqrt(d[0] / (float)K + p.eps);
  }
#pragma unroll
  for (uint32_t u = 0; u < PRO_U; u++) {
    const uint32_t i = u * NT + threadIdx.x;
    float s = 0.f;
    if (i < n4) {
      const uint32_t e = i << 2, g = e >> 7, o = e & 127;
      float4 v;
      v.x = vx[u].x * inv * vw[u].x;
      v.y = vx[u].y * inv * vw[u].y;
      v.z = vx[u].z * inv * vw[u].z;
      v.w = vx[u].w * inv * vw[u].w;
      *reinterpret_cast<float4*>(xs + g * GROUP_STRIDE + o) = v;
      s = (v.x + v.y) + (v.z + v.w);
    }
    // block sums: the 8 lanes of a half-row hold one block (NT and n4 are multiples of 8)
    s = sum8(s);
    if (i < n4 && (i & 7) == 0) bsum[i >> 3] = s;
  }
  __syncthreads();
}

// Mode 4: the gated layer's input and its gate (quiescence).  Each thread
// loads its slices of x, r, wr, w and xa and the previous layer's run flag
// up front; one block-wide reduction gives sum r^2, x^2, x q, q^2 and xa^2,
// from which A' and its norm follow as in mode 2 (or A' = xa).  Workgroup 0
// alone then reads xprev, reduces mean((A' - xprev)^2), writes the run flag
// and stores A' as xprev, so no workgroup reads an xprev another writes.
struct ProGIn {
  ProIn p;
  float4 va[PRO_U];
  uint32_t prun;
};

template <int NT>
__device__ __forceinline__ void pro_gate_load(const XPro& p, uint32_t K, ProGIn& in) {
  const uint32_t n4 = K >> 2;
  const float4* x = reinterpret_cast<const float4*>(p.x);
  const float4* r = reinterpret_cast<const float4*>(p.r);
  const float4* wr = reinterpret_cast<const float4*>(p.wr ? p.wr : p.r);
  const float4* w = reinterpret_cast<const float4*>(p.w);
  const float4* xa = reinterpret_cast<const float4*>(p.xa);
  in.prun = p.pmode == 2u ? *p.prun : 1u;
#pragma unroll
  for (uint32_t u = 0; u < PRO_U; u++) {
    uint32_t i = u * NT + threadIdx.x;
    i = i < n4 ? i : n4 - 1;
    in.p.vx[u] = x[i];
    in.p.vr[u] = r[i];
    in.p.vwr[u] = wr[i];
    in.p.vw[u] = w[i];
    in.va[u] = xa[i];
  }
}

template <int NT>
__device__ __forceinline__ void pro_gate_finish(const XPro& p, uint32_t K, ProGIn& in, float* xs,
                                                float* bsum, float* ext) {
  const uint32_t n4 = K >> 2;
  const bool add = p.pmode == 1u || (p.pmode == 2u && in.prun != 0u);  // uniform
  const bool has_wr = p.wr != nullptr;
  float4* vx = in.p.vx;
  const float4* vr = in.p.vr;
  const float4* vwr = in.p.vwr;
  const float4* vw = in.p.vw;
  float t[5] = {0.f, 0.f, 0.f, 0.f, 0.f};  // sum r^2, x^2, x q, q^2, xa^2
#pragma unroll
  for (uint32_t u = 0; u < PRO_U; u++) {
    if (u * NT + threadIdx.x < n4) {
      const float r[4] = {vr[u].x, vr[u].y, vr[u].z, vr[u].w};
      const float x[4] = {vx[u].x, vx[u].y, vx[u].z, vx[u].w};
      const float w[4] = {vwr[u].x, vwr[u].y, vwr[u].z, vwr[u].w};
      const float a[4] = {in.va[u].x, in.va[u].y, in.va[u].z, in.va[u].w};
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const float q = has_wr ? r[e] * w[e] : r[e];
        t[0] += r[e] * r[e];
        t[1] += x[e] * x[e];
        t[2] += x[e] * q;
        t[3] += q * q;
        t[4] += a[e] * a[e];
      }
    }
  }
  block_sums<NT, 5>(t, ext);
  float s2;
  if (add) {
    const float c = has_wr ? norm_rsqrt(t[0] / (float)K + p.eps) : 1.0f;
    const float pos = t[1] + c * c * t[3];
    s2 = p.s * p.s * (pos + 2.0f * c * t[2]);
#pragma unroll
    for (uint32_t u = 0; u < PRO_U; u++) {
      float4 rv = vr[u];
      if (has_wr) {
        rv.x = rv.x * c * vwr[u].x;
        rv.y = rv.y * c * vwr[u].y;
        rv.z = rv.z * c * vwr[u].z;
        rv.w = rv.w * c * vwr[u].w;
      }
      vx[u].x = (vx[u].x + rv.x) * p.s;
      vx[u].y = (vx[u].y + rv.y) * p.s;
      vx[u].z = (vx[u].z + rv.z) * p.s;
      vx[u].w = (vx[u].w + rv.w) * p.s;
    }
    if (!(s2 > 1e-3f * p.s * p.s * pos)) {  // cancellation (uniform branch): reduce A'^2 itself
      float d[1] = {0.f};
#pragma unroll
      for (uint32_t u = 0; u < PRO_U; u++)
        if (u * NT + threadIdx.x < n4)
          d[0] += vx[u].x * vx[u].x + vx[u].y * vx[u].y + vx[u].z * vx[u].z + vx[u].w * vx[u].w;
      block_sums<NT, 1>(d, ext + 5 * (NT / 64));
      s2 = d[0];
    }
  } else {
#pragma unroll
    for (uint32_t u = 0; u < PRO_U; u++) vx[u] = in.va[u];
    s2 = t[4];
  }
  const float inv = norm_rsqrt(s2 / (float)K + p.eps);
#pragma unroll
  for (uint32_t u = 0; u < PRO_U; u++) {
    const uint32_t i = u * NT + threadIdx.x;
    float sb = 0.f;
    if (i < n4) {
      const uint32_t e = i << 2, g = e >> 7, o = e & 127;
      float4 v;
      v.x = vx[u].x * inv * vw[u].x;
      v.y = vx[u].y * inv * vw[u].y;
      v.z = vx[u].z * inv * vw[u].z;
      v.w = vx[u].w * inv * vw[u].w;
      *reinterpret_cast<float4*>(xs + g * GROUP_STRIDE + o) = v;
      sb = (v.x + v.y) + (v.z + v.w);
    }
    sb = sum8(sb);
    if (i < n4 && (i & 7) == 0) bsum[i >> 3] = sb;
  }
  if (blockIdx.x == 0) {  // the gate (uniform per workgroup)
    float4* xprev = reinterpret_cast<float4*>(p.xprev);
    float d[1] = {0.f};
#pragma unroll
    for (uint32_t u = 0; u < PRO_U; u++) {
      const uint32_t i = u * NT + threadIdx.x;
      if (i < n4) {
        const float4 pv = xprev[i];
        const float a = vx[u].x - pv.x, b = vx[u].y - pv.y, e = vx[u].z - pv.z,
                    f = vx[u].w - pv.w;
        d[0] += a * a + b * b + e * e + f * f;
        xprev[i] = vx[u];
        if (add) reinterpret_cast<float4*>(p.xout)[i] = vx[u];
      }
    }
    block_sums<NT, 1>(d, ext + 6 * (NT / 64));
    if (threadIdx.x == 0) *p.run_out = (d[0] / (float)K >= p.thr || p.thr <= 0.0f) ? 1u : 0u;
  }
  __syncthreads();
}

// ------------------------------------------------------------------------
// Weight formats: one "item" = one 4-block group of one row.
// init() sets the whole accumulator, zero() resets it for the next row,
// finish() reduces a row over its team, block_end() runs once per workgroup
// after the stream (all threads).
// ------------------------------------------------------------------------
struct Q4Fmt {  // shaders/gemv_q4.wgsl
  static constexpr uint32_t kGroupBytes = 80, kBlockBytes = 20;
  struct Item {
    Q4G w;
  };
  struct Acc {
    float s;
  };
  struct Args {
    const uint8_t* W;
    float* Y;
  };
  __device__ static void load(Item& it, const Args& a, size_t off) {
    it.w = load_q4g(a.W + off);
  }
  __device__ static void init(Acc& c) { c.s = 0.f; }
  __device__ static void zero(Acc& c) { c.s = 0.f; }
  __device__ static void fma(Acc& c, const Item& it, const float* xg, const float* bs, float valid) {
    c.s += valid * q4_group_dot(it.w, xg, bs);
  }
  template <int TPR>
  __device__ static void finish(Acc& c, const Args& a, uint32_t row, bool writer) {
    const float v = team_sum<TPR>(c.s);
    if (writer) a.Y[row] = v;
  }
  template <int NT>
  __device__ static void block_end(const Acc&, const Args&, float*) {}
};

// Gate and up rows of the same (row, group) travel as one item, so every x
// value read from LDS feeds both matrices.
__device__ __forceinline__ void q4_group_dot2(const Q4G& a, const Q4G& b, const float* __restrict__ xg,
                                              const float* __restrict__ bs, float& ra, float& rb) {
  const uint32_t A[20] = {a.a0.x, a.a0.y, a.a0.z, a.a0.w, a.a1.x, a.a1.y, a.a1.z, a.a1.w,
                          a.a2.x, a.a2.y, a.a2.z, a.a2.w, a.a3.x, a.a3.y, a.a3.z, a.a3.w,
                          a.a4.x, a.a4.y, a.a4.z, a.a4.w};
  const uint32_t B[20] = {b.a0.x, b.a0.y, b.a0.z, b.a0.w, b.a1.x, b.a1.y, b.a1.z, b.a1.w,
                          b.a2.x, b.a2.y, b.a2.z, b.a2.w, b.a3.x, b.a3.y, b.a3.z, b.a3.w,
                          b.a4.x, b.a4.y, b.a4.z, b.a4.w};
  ra = 0.f;
  rb = 0.f;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const uint32_t* wa = &A[5 * j + 1];
    const uint32_t* wb = &B[5 * j + 1];
    const float* xb = xg + 32 * j;
    float al = 0.f, ah = 0.f, bl = 0.f, bh = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const float4 xa = *reinterpret_cast<const float4*>(xb + 8 * k);
      const float4 xc = *reinterpret_cast<const float4*>(xb + 8 * k + 4);
      q4_word(wa[k], xa, xc, al, ah);
      q4_word(wb[k], xa, xc, bl, bh);
    }
    // same operation order as q4_group_dot for each matrix
    const float sa = q4_sum(al, ah), sb = q4_sum(bl, bh);
    if (j == 0) {
      ra = u2f(A[0]) * (sa - 8.0f * bs[0]);
      rb = u2f(B[0]) * (sb - 8.0f * bs[0]);
    } else {
      ra += u2f(A[5 * j]) * (sa - 8.0f * bs[j]);
      rb += u2f(B[5 * j]) * (sb - 8.0f * bs[j]);
    }
  }
}

struct GateUpFmt {  // shaders/fused_mlp_q4.wgsl: act = gelu_tanh(Wg x) * (Wu x)
  static constexpr uint32_t kGroupBytes = 80, kBlockBytes = 20;
  struct Item {
    Q4G g, u;
  };
  struct Acc {
    float g, u;
  };
  struct Args {
    const uint8_t* Wg;
    const uint8_t* Wu;
    float* Y;
  };
  __device__ static void load(Item& it, const Args& a, size_t off) {
    it.g = load_q4g(a.Wg + off);
    it.u = load_q4g(a.Wu + off);
  }
  __device__ static void init(Acc& c) { c.g = c.u = 0.f; }
  __device__ static void zero(Acc& c) { c.g = c.u = 0.f; }
  __device__ static void fma(Acc& c, const Item& it, const float* xg, const float* bs, float valid) {
    float g, u;
    q4_group_dot2(it.g, it.u, xg, bs, g, u);
    c.g += valid * g;
    c.u += valid * u;
  }
  template <int TPR>
  __device__ static void finish(Acc& c, const Args& a, uint32_t row, bool writer) {
    const float g = team_sum<TPR>(c.g);
    const float u = team_sum<TPR>(c.u);
    if (writer) a.Y[row] = gelu_tanh(g) * u;
  }
  template <int NT>
  __device__ static void block_end(const Acc&, const Args&, float*) {}
};

struct Q8G {
  u32x4 v[9];
};

__device__ __forceinline__ void load_q8g(Q8G& g, const uint8_t* p) {
#pragma unroll
  for (int k = 0; k < 9; k++) g.v[k] = ldw(p + 16 * k);
}

__device__ __forceinline__ float q8_group_dot(const Q8G& g, const float* xg, const float* bs) {
  uint32_t w[36];
#pragma unroll
  for (int k = 0; k < 9; k++) {
    w[4 * k + 0] = g.v[k].x;
    w[4 * k + 1] = g.v[k].y;
    w[4 * k + 2] = g.v[k].z;
    w[4 * k + 3] = g.v[k].w;
  }
  float r = 0.f;
#pragma unroll
  for (int j = 0; j < 4; j++) r += u2f(w[9 * j]) * (q8_ux(&w[9 * j + 1], xg + 32 * j) - 128.0f * bs[j]);
  return r;
}

struct Q8Fmt {  // shaders/gemv_q8.wgsl
  static constexpr uint32_t kGroupBytes = 144, kBlockBytes = 36;
  struct Item {
    Q8G w;
  };
  struct Acc {
    float s;
  };
  struct Args {
    const uint8_t* W;
    float* Y;
  };
  __device__ static void load(Item& it, const Args& a, size_t off) {
    load_q8g(it.w, a.W + off);
  }
  __device__ static void init(Acc& c) { c.s = 0.f; }
  __device__ static void zero(Acc& c) { c.s = 0.f; }
  __device__ static void fma(Acc& c, const Item& it, const float* xg, const float* bs, float valid) {
    c.s += valid * q8_group_dot(it.w, xg, bs);
  }
  template <int TPR>
  __device__ static void finish(Acc& c, const Args& a, uint32_t row, bool writer) {
    const float v = team_sum<TPR>(c.s);
    if (writer) a.Y[row] = v;
  }
  template <int NT>
  __device__ static void block_end(const Acc&, const Args&, float*) {}
};

__device__ __forceinline__ void q8_group_dot2(const Q8G& a, const Q8G& b, const float* xg,
                                              const float* bs, float& ra, float& rb) {
  uint32_t A[36], B[36];
#pragma unroll
  for (int k = 0; k < 9; k++) {
    A[4 * k + 0] = a.v[k].x;
    A[4 * k + 1] = a.v[k].y;
    A[4 * k + 2] = a.v[k].z;
    A[4 * k + 3] = a.v[k].w;
    B[4 * k + 0] = b.v[k].x;
    B[4 * k + 1] = b.v[k].y;
    B[4 * k + 2] = b.v[k].z;
    B[4 * k + 3] = b.v[k].w;
  }
  ra = 0.f;
  rb = 0.f;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const float* xb = xg + 32 * j;
    float a0 = 0.f, a1 = 0.f, b0 = 0.f, b1 = 0.f;
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const uint32_t ua = opaque_and(A[9 * j + 1 + k] ^ 0x80808080u, 0xFFFFFFFFu);
      const uint32_t ub = opaque_and(B[9 * j + 1 + k] ^ 0x80808080u, 0xFFFFFFFFu);
      const float4 xa = *reinterpret_cast<const float4*>(xb + 4 * k);
      a0 += ub0(ua) * xa.x;
      a1 += ub1(ua) * xa.y;
      a0 += ub2(ua) * xa.z;
      a1 += ub3(ua) * xa.w;
      b0 += ub0(ub) * xa.x;
      b1 += ub1(ub) * xa.y;
      b0 += ub2(ub) * xa.z;
      b1 += ub3(ub) * xa.w;
    }
    ra += u2f(A[9 * j]) * ((a0 + a1) - 128.0f * bs[j]);
    rb += u2f(B[9 * j]) * ((b0 + b1) - 128.0f * bs[j]);
  }
}

struct GateUpQ8Fmt {  // shaders/fused_mlp_q8.wgsl (--q8 layers)
  static constexpr uint32_t kGroupBytes = 144, kBlockBytes = 36;
  struct Item {
    Q8G g, u;
  };
  using Acc = GateUpFmt::Acc;
  using Args = GateUpFmt::Args;
  __device__ static void load(Item& it, const Args& a, size_t off) {
    load_q8g(it.g, a.Wg + off);
    load_q8g(it.u, a.Wu + off);
  }
  __device__ static void init(Acc& c) { c.g = c.u = 0.f; }
  __device__ static void zero(Acc& c) { c.g = c.u = 0.f; }
  __device__ static void fma(Acc& c, const Item& it, const float* xg, const float* bs, float valid) {
    float g, u;
    q8_group_dot2(it.g, it.u, xg, bs, g, u);
    c.g += valid * g;
    c.u += valid * u;
  }
  template <int TPR>
  __device__ static void finish(Acc& c, const Args& a, uint32_t row, bool writer) {
    GateUpFmt::finish<TPR>(c, a, row, writer);
  }
  template <int NT>
  __device__ static void block_end(const Acc&, const Args&, float*) {}
};

// (value, index) order of the greedy pick: larger value wins, equal values go
// to the smaller index (src/kernels.zig:164-174).
__device__ __forceinline__ bool better(float v, uint32_t i, float bv, uint32_t bi) {
  return v > bv || (v == bv && i < bi);
}

// Q8_0 vocab projection with the argmax fused in (shaders/gemv_q8.wgsl then
// shaders/argmax.wgsl, src/gpu/model_dispatch.zig:124-126): every lane keeps
// the best (logit, row) of its team's rows and block_end writes the block's
// best as one partial.  gh_argmax_final_k, launched right after, reduces the
// partials to the token.  (A "last block reduces" scheme inside the stream
// needs a device-scope fence per workgroup, which costs more than the whole
// second launch.)  Logits are stored only when Y != null.
__device__ __forceinline__ void wave_best(float& v, uint32_t& i) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(v, off, 64);
    const uint32_t oi = __shfl_xor(i, off, 64);
    if (better(ov, oi, v, i)) {
      v = ov;
      i = oi;
    }
  }
}

// Best (value, index) of the block: every thread passes its candidate;
// thread 0 returns the result.  red holds 2 * NT / 64 words.
template <int NT>
__device__ __forceinline__ void block_best(float& bv, uint32_t& bi, float* red) {
  constexpr int W = NT / 64;
  float* rv = red;
  uint32_t* ri = reinterpret_cast<uint32_t*>(red + W);
  wave_best(bv, bi);
  if ((threadIdx.x & 63) == 0) {
    rv[threadIdx.x >> 6] = bv;
    ri[threadIdx.x >> 6] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < W; w++)
      if (better(rv[w], ri[w], bv, bi)) {
        bv = rv[w];
        bi = ri[w];
      }
  }
}

struct Q8ArgmaxFmt {
  static constexpr uint32_t kGroupBytes = 144, kBlockBytes = 36;
  using Item = Q8Fmt::Item;
  struct Acc {
    float s, bv;
    uint32_t bi;
  };
  struct Args {
    const uint8_t* W;
    float* Y;
    uint32_t* partial;  // 2 words per block: best value bits, its row
  };
  __device__ static void load(Item& it, const Args& a, size_t off) {
    load_q8g(it.w, a.W + off);
  }
  __device__ static void init(Acc& c) {
    c.s = 0.f;
    c.bv = -INFINITY;
    c.bi = 0xFFFFFFFFu;
  }
  __device__ static void zero(Acc& c) { c.s = 0.f; }
  __device__ static void fma(Acc& c, const Item& it, const float* xg, const float* bs, float valid) {
    c.s += valid * q8_group_dot(it.w, xg, bs);
  }
  template <int TPR>
  __device__ static void finish(Acc& c, const Args& a, uint32_t row, bool writer) {
    const float v = team_sum<TPR>(c.s);
    if (a.Y && writer) a.Y[row] = v;
    if (better(v, row, c.bv, c.bi)) {
      c.bv = v;
      c.bi = row;
    }
  }
  template <int NT>
  __device__ static void block_end(const Acc& c, const Args& a, float* red) {
    float bv = c.bv;
    uint32_t bi = c.bi;
    block_best<NT>(bv, bi, red);
    if (threadIdx.x == 0) {
      a.partial[2 * blockIdx.x] = __float_as_uint(bv);
      a.partial[2 * blockIdx.x + 1] = bi;
    }
  }
};

// ------------------------------------------------------------------------
// bf16 weights (the reference's --gpu mode, mode none: src/gpu/kernels.zig:36
// selects shaders/gemv_bf16.wgsl).  Rows are the plain row-major bf16 of the
// checkpoint, K / 8 chunks of 16 bytes.  The stream is interleaved: item j of
// lane l of a row team holds chunks (8 j + k) TPR + l, k = 0..7, so each of
// the 8 loads of a wavefront reads TPR consecutive chunks (whole cache lines;
// 256 contiguous bytes per lane instead measured 8.1 vs 5.4 us for 19.7 MB).
// A chunk's 8 weights widen exactly to fp32 (low half first) and meet x in
// fp32, as the shader's bf16_to_f32(p & 0xFFFF) * X[2i] + ... does.
// ------------------------------------------------------------------------
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// x of chunk c (8 floats) in the group-padded LDS staging
__device__ __forceinline__ const float* x_of_chunk(const float* xs, uint32_t c) {
  return xs + (c >> 4) * GROUP_STRIDE + ((c & 15u) << 3);
}

__device__ __forceinline__ float bf16_chunk_dot(const u32x4& w, const float* xc) {
  const float4 xa = *reinterpret_cast<const float4*>(xc);
  const float4 xb = *reinterpret_cast<const float4*>(xc + 4);
  float s = bf_lo(w.x) * xa.x + bf_hi(w.x) * xa.y;
  s += bf_lo(w.y) * xa.z + bf_hi(w.y) * xa.w;
  s += bf_lo(w.z) * xb.x + bf_hi(w.z) * xb.y;
  s += bf_lo(w.w) * xb.z + bf_hi(w.w) * xb.w;
  return s;
}

constexpr uint32_t kBfChunks = 8;  // 16-byte chunks per lane per item (64 weights)

template <int TPR>
__device__ __forceinline__ void load_bf_item(u32x4 (&w)[kBfChunks], const uint8_t* row,
                                             uint32_t c0, uint32_t nch) {
#pragma unroll
  for (uint32_t k = 0; k < kBfChunks; k++) {
    uint32_t c = c0 + k * TPR;
    c = c < nch ? c : nch - 1;  // past the row: an in-range duplicate, weighted 0
    w[k] = ldw(row + (size_t)c * 16);
  }
}

// Sum of an item's chunk dots into acc (chunks past the row add 0).
template <int TPR>
__device__ __forceinline__ void bf_item_dot(float& acc, const u32x4 (&w)[kBfChunks],
                                            const float* xs, uint32_t c0, uint32_t nch) {
#pragma unroll
  for (uint32_t k = 0; k < kBfChunks; k++) {
    const uint32_t ch = c0 + k * TPR;
    const float d = bf16_chunk_dot(w[k], x_of_chunk(xs, ch < nch ? ch : nch - 1));
    acc += ch < nch ? d : 0.0f;
  }
}

struct Bf16Fmt {  // shaders/gemv_bf16.wgsl
  static constexpr uint32_t kChunks = kBfChunks, kBlockBytes = 64;  // 32 weights = 64 B
  struct Item {
    u32x4 w[kBfChunks];
  };
  using Acc = Q4Fmt::Acc;
  using Args = Q4Fmt::Args;
  template <int TPR>
  __device__ static void load(Item& it, const Args& a, size_t row_off, uint32_t c0, uint32_t nch) {
    load_bf_item<TPR>(it.w, a.W + row_off, c0, nch);
  }
  __device__ static void init(Acc& c) { c.s = 0.f; }
  __device__ static void zero(Acc& c) { c.s = 0.f; }
  template <int TPR>
  __device__ static void fma(Acc& c, const Item& it, const float* xs, uint32_t c0, uint32_t nch) {
    bf_item_dot<TPR>(c.s, it.w, xs, c0, nch);
  }
  template <int TPR>
  __device__ static void finish(Acc& c, const Args& a, uint32_t row, bool writer) {
    Q4Fmt::finish<TPR>(c, a, row, writer);
  }
  template <int NT>
  __device__ static void block_end(const Acc&, const Args&, float*) {}
};

// bf16 gate and up rows of the same (row, item) travel together, so every x
// value read from LDS feeds both.  (In the reference's mode none the fused
// MLP pipeline is the Q4 shader, src/gpu/kernels.zig:41, which reads bf16
// rows as Q4 blocks; this computes what the CPU path computes,
// src/kernels.zig:100-129: act = gelu_tanh(Wg x) * (Wu x).)
struct GateUpBf16Fmt {
  static constexpr uint32_t kChunks = kBfChunks, kBlockBytes = 64;
  struct Item {
    u32x4 g[kBfChunks], u[kBfChunks];
  };
  using Acc = GateUpFmt::Acc;
  using Args = GateUpFmt::Args;
  template <int TPR>
  __device__ static void load(Item& it, const Args& a, size_t row_off, uint32_t c0, uint32_t nch) {
    load_bf_item<TPR>(it.g, a.Wg + row_off, c0, nch);
    load_bf_item<TPR>(it.u, a.Wu + row_off, c0, nch);
  }
  __device__ static void init(Acc& c) { c.g = c.u = 0.f; }
  __device__ static void zero(Acc& c) { c.g = c.u = 0.f; }
  template <int TPR>
  __device__ static void fma(Acc& c, const Item& it, const float* xs, uint32_t c0, uint32_t nch) {
#pragma unroll
    for (uint32_t k = 0; k < kBfChunks; k++) {
      const uint32_t ch = c0 + k * TPR;
      const float* xc = x_of_chunk(xs, ch < nch ? ch : nch - 1);
      const float dg = bf16_chunk_dot(it.g[k], xc);
      const float du = bf16_chunk_dot(it.u[k], xc);
      c.g += ch < nch ? dg : 0.0f;
      c.u += ch < nch ? du : 0.0f;
    }
  }
  template <int TPR>
  __device__ static void finish(Acc& c, const Args& a, uint32_t row, bool writer) {
    GateUpFmt::finish<TPR>(c, a, row, writer);
  }
  template <int NT>
  __device__ static void block_end(const Acc&, const Args&, float*) {}
};

// bf16 vocab projection with the argmax fused in: the head of mode none is
// the bf16 embedding itself (src/gpu/model_gpu.zig:160-161; the logits
// pipeline is the bf16 GEMV, src/gpu/kernels.zig:38).
struct Bf16ArgmaxFmt {
  static constexpr uint32_t kChunks = kBfChunks, kBlockBytes = 64;
  using Item = Bf16Fmt::Item;
  using Acc = Q8ArgmaxFmt::Acc;
  using Args = Q8ArgmaxFmt::Args;
  template <int TPR>
  __device__ static void load(Item& it, const Args& a, size_t row_off, uint32_t c0, uint32_t nch) {
    load_bf_item<TPR>(it.w, a.W + row_off, c0, nch);
  }
  __device__ static void init(Acc& c) { Q8ArgmaxFmt::init(c); }
  __device__ static void zero(Acc& c) { c.s = 0.f; }
  template <int TPR>
  __device__ static void fma(Acc& c, const Item& it, const float* xs, uint32_t c0, uint32_t nch) {
    bf_item_dot<TPR>(c.s, it.w, xs, c0, nch);
  }
  template <int TPR>
  __device__ static void finish(Acc& c, const Args& a, uint32_t row, bool writer) {
    Q8ArgmaxFmt::finish<TPR>(c, a, row, writer);
  }
  template <int NT>
  __device__ static void block_end(const Acc& c, const Args& a, float* red) {
    Q8ArgmaxFmt::block_end<NT>(c, a, red);
  }
};

// Formats with kChunks stream interleaved (stream_rows_il), the others by
// 4-block groups (stream_rows).
template <class F>
constexpr auto interleaved(int) -> decltype(F::kChunks, bool()) { return true; }
template <class F>
constexpr bool interleaved(long) { return false; }

// ------------------------------------------------------------------------
// Persistent row-team streaming.  Team t (TPR lanes) owns rows t, t + T,
// t + 2T, ... (T = teams in the grid); lane l of a team owns groups
// l, l + TPR, ..., l + (GPL-1) TPR of each of its rows.  A lane walks its
// items in order through a ring of D item buffers: while item i is reduced,
// items i+1 .. i+D-1 are in flight.  D = 1 keeps one item per lane in flight
// and relies on the other waves of the CU to cover the latency; on MI355X
// that reads faster than deeper per-lane look-ahead at these sizes (more
// outstanding requests per CU than the memory system serves well).  The
// ring is unrolled so no register copies (which would force an early wait)
// are needed.  Items past the end of a row (group >= ng) load an in-range
// duplicate and contribute zero; nothing is loaded beyond a team's last
// item.  Teams with no rows skip the stream but still take part in the
// block-wide prologue and epilogue.
// ------------------------------------------------------------------------
// The prologue of a stream and its first weight loads (issue()).  run
// non-null (a gated layer's stream): the layer's run flag, read at entry and
// tested once the first loads are in flight, before the prologue writes
// anything to global memory; returns false when the layer is gated off
// (every thread of the workgroup reads the same flag).  Testing it at entry
// instead made every gated launch wait for the flag before its first load.
template <int NT, int PRO, class Issue>
__device__ __forceinline__ bool stream_start(const XPro& xp, uint32_t K, float* xs, float* bsum,
                                             float* ext, Issue issue,
                                             const uint32_t* run = nullptr) {
  const uint32_t go = run ? *run : 1u;
  // A wave's loads complete in order, so x loads issued behind its own
  // weight loads would wait for them (barriers do not wait for outstanding
  // loads).  Every thread therefore issues its prologue loads (x, and for
  // the normed streams r and the norm weights) first, then its weight loads,
  // then runs the prologue (whose reductions need every thread).
  if constexpr (PRO == 2) {
    ProGIn pin;
    pro_gate_load<NT>(xp, K, pin);
    issue();
    pro_gate_finish<NT>(xp, K, pin, xs, bsum, ext);
  } else if constexpr (PRO == 1) {
    ProIn pin;
    pro_load<NT>(xp, K, pin);
    issue();
    if (go == 0u) return false;
    pro_finish<NT>(xp, K, pin, xs, bsum, ext);
  } else if (K <= PRO_U * 4 * NT) {
    // x first: every thread issues its slices of x, then its first weight
    // loads, then stages x (the x loads return first; measured 14.8 vs
    // 15.2 us against splitting the workgroup into stagers and streamers)
    ProIn pin;
    XPro x_only = xp;
    x_only.mode = 0;
    pro_load<NT>(x_only, K, pin);
    issue();
    if (go == 0u) return false;
    pro_finish<NT>(x_only, K, pin, xs, bsum, ext);
  } else {
    // longer x than the registers hold: the first NS threads stage x while
    // the others' first weight loads are in flight, then issue their own
    constexpr uint32_t NS = NT >= 1024 ? 256 : NT / 2;
    const bool late = threadIdx.x < NS;
    if (!late) issue();
    if (late) stage_x<NS>(xp.x, K, xs, bsum);
    __syncthreads();
    if (late) issue();
    if (go == 0u) return false;
  }
  return true;
}

template <class F, int TPR, int GPL, int D, int NT, int PRO>
__device__ __forceinline__ void stream_rows(const typename F::Args& a, const XPro& xp, uint32_t M,
                                            uint32_t K, const uint32_t* run) {
  extern __shared__ float lds[];
  const uint32_t nb = K >> 5, ng = nb >> 2;
  float* xs = lds;
  float* bsum = lds + ng * GROUP_STRIDE;
  float* ext = bsum + nb;  // prologue scratch / epilogue reduction space

  constexpr uint32_t TEAMS = NT / TPR;
  const uint32_t lr = threadIdx.x % TPR;
  const uint32_t team = blockIdx.x * TEAMS + threadIdx.x / TPR;
  const uint32_t nteams = gridDim.x * TEAMS;
  const bool active = team < M;
  constexpr uint32_t PER_ROW = GPL;  // items per row for one lane
  const uint32_t n_items = active ? ((M - 1 - team) / nteams + 1) * PER_ROW : 0;
  const size_t row_bytes = (size_t)nb * F::kBlockBytes;

  // item i -> row (i / PER_ROW), lane group slot (i % PER_ROW)
  auto group_of = [&](uint32_t i) -> uint32_t { return lr + (i % PER_ROW) * TPR; };
  auto offset_of = [&](uint32_t i) -> size_t {
    const uint32_t row = team + (i / PER_ROW) * nteams;
    uint32_t g = group_of(i);
    g = g < ng ? g : ng - 1;
    return (size_t)row * row_bytes + (size_t)g * F::kGroupBytes;
  };
  // the same with the row clamped into the matrix (for loads that may not be used)
  auto offset_in = [&](uint32_t i) -> size_t {
    uint32_t row = team + (i / PER_ROW) * nteams;
    row = row < M ? row : M - 1;
    uint32_t g = group_of(i);
    g = g < ng ? g : ng - 1;
    return (size_t)row * row_bytes + (size_t)g * F::kGroupBytes;
  };

  // Plain streams load their first items unconditionally (a team past the
  // last row, or an item past a lane's last, loads an in-range duplicate that
  // is never used): the compiler then knows how many weight loads follow the
  // x loads, and its waits for x no longer wait for the weights (8192 x 2048:
  // 4.53 against 5.00 us; 3840 x 15360: 10.0 against 10.5 us).  The normed
  // streams keep them under the branch: with the same change their prologue
  // overlaps the first weight loads, yet they measured slower (15360 x 3840
  // gate+up 15.5 against 15.2 us, decode 370 against 372.5 tok/s).
  typename F::Item buf[D];
  if (!stream_start<NT, PRO>(xp, K, xs, bsum, ext, [&]() {
#pragma unroll
    for (int d = 0; d < D; d++) {
      if constexpr (PRO != 0) {
        if (d < n_items) F::load(buf[d], a, offset_of(d));
      } else {
        F::load(buf[d], a, offset_in(d));
      }
    }
  }, run))
    return;
  typename F::Acc acc;
  F::init(acc);
#pragma unroll 1
  for (uint32_t base = 0; base < n_items; base += D) {
#pragma unroll
    for (int d = 0; d < D; d++) {
      const uint32_t i = base + d;
      if (i < n_items) {  // uniform within a team
        const uint32_t g = group_of(i);
        const uint32_t gc = g < ng ? g : ng - 1;
        F::fma(acc, buf[d], xs + gc * GROUP_STRIDE, bsum + gc * 4, g < ng ? 1.0f : 0.0f);
        if (i % PER_ROW == PER_ROW - 1) {
          F::template finish<TPR>(acc, a, team + (i / PER_ROW) * nteams, lr == 0);
          F::zero(acc);
        }
      }
      if (i + D < n_items) F::load(buf[d], a, offset_of(i + D));
    }
  }
  F::template block_end<NT>(acc, a, ext);
}

// ------------------------------------------------------------------------
// Interleaved row-team streaming (bf16 rows): as stream_rows, but item j of
// lane l covers the row's 16-byte chunks (kChunks j + k) TPR + l, so the
// team reads whole cache lines per load instruction.  GPL items per row per
// lane, TPR GPL kChunks >= K / 8.
// ------------------------------------------------------------------------
template <class F, int TPR, int GPL, int D, int NT, int PRO>
__device__ __forceinline__ void stream_rows_il(const typename F::Args& a, const XPro& xp,
                                               uint32_t M, uint32_t K, const uint32_t* run) {
  extern __shared__ float lds[];
  const uint32_t nb = K >> 5, ng = nb >> 2, nch = K >> 3;
  float* xs = lds;
  float* bsum = lds + ng * GROUP_STRIDE;
  float* ext = bsum + nb;
  constexpr uint32_t TEAMS = NT / TPR, C = F::kChunks;
  const uint32_t lr = threadIdx.x % TPR;
  const uint32_t team = blockIdx.x * TEAMS + threadIdx.x / TPR;
  const uint32_t nteams = gridDim.x * TEAMS;
  const uint32_t n_items = team < M ? ((M - 1 - team) / nteams + 1) * GPL : 0;
  const size_t row_bytes = (size_t)K * 2;
  auto row_of = [&](uint32_t i) -> uint32_t { return team + (i / GPL) * nteams; };
  auto c0_of = [&](uint32_t i) -> uint32_t { return (i % GPL) * C * TPR + lr; };
  typename F::Item buf[D];
  // first items: unconditional in the plain streams, as in stream_rows
  if (!stream_start<NT, PRO>(xp, K, xs, bsum, ext, [&]() {
#pragma unroll
    for (int d = 0; d < D; d++) {
      if constexpr (PRO != 0) {
        if (d < n_items) F::template load<TPR>(buf[d], a, row_of(d) * row_bytes, c0_of(d), nch);
      } else {
        const uint32_t r = row_of(d) < M ? row_of(d) : M - 1;
        F::template load<TPR>(buf[d], a, r * row_bytes, c0_of(d), nch);
      }
    }
  }, run))
    return;
  typename F::Acc acc;
  F::init(acc);
#pragma unroll 1
  for (uint32_t base = 0; base < n_items; base += D) {
#pragma unroll
    for (int d = 0; d < D; d++) {
      const uint32_t i = base + d;
      if (i < n_items) {  // uniform within a team
        F::template fma<TPR>(acc, buf[d], xs, c0_of(i), nch);
        if (i % GPL == GPL - 1) {
          F::template finish<TPR>(acc, a, row_of(i), lr == 0);
          F::zero(acc);
        }
      }
      if (i + D < n_items)
        F::template load<TPR>(buf[d], a, row_of(i + D) * row_bytes, c0_of(i + D), nch);
    }
  }
  F::template block_end<NT>(acc, a, ext);
}

template <class F, int TPR, int GPL, int D, int NT, int PRO>
__device__ __forceinline__ void stream(const typename F::Args& a, const XPro& xp, uint32_t M,
                                       uint32_t K, const uint32_t* run = nullptr) {
  if constexpr (interleaved<F>(0))
    stream_rows_il<F, TPR, GPL, D, NT, PRO>(a, xp, M, K, run);
  else
    stream_rows<F, TPR, GPL, D, NT, PRO>(a, xp, M, K, run);
}

// Kernel names: gh_<family>[n|g]_t<TPR>_g<GPL>_d<D>; the "n" variants carry
// the normed x prologue (modes 1 and 2, PRO = 1), the "g" variants a gated
// layer's input and gate (mode 4, PRO = 2), the others stage x as given
// (mode 0) and keep the prologue's registers out of the stream.  Weight and output
// pointers are separate kernel parameters: loaded out of a by-value struct
// parameter they lose the kernel-argument address-space and alignment facts,
// and the stream then needs ~100 more VGPRs (220 vs 126 for the Q4 d3 form).
// Gated forms (suffix _q): the decode graph's gated layers (quiescence on)
// launch these; they take the layer's run flag and do nothing when it is 0
// (tested once their first loads are in flight, stream_start).  The ungated
// kernels carry no gating code at all: even a null-pointer test at entry
// measured +0.3 us per launch.
#define GH_STREAM_KERNEL_NT(NAME, FMT, PARAMS, ARGS, T, G, D, PRO, NT, SUFFIX)        \
  extern "C" __global__ __launch_bounds__(NT) void NAME##_t##T##_g##G##_d##D##SUFFIX(     \
      GH_UNPAREN PARAMS, XPro xp, uint32_t M, uint32_t K) {                               \
    stream<FMT, T, G, D, NT, PRO>(FMT::Args{GH_UNPAREN ARGS}, xp, M, K);               \
  }
#define GH_STREAM_KERNEL_NT_Q(NAME, FMT, PARAMS, ARGS, T, G, D, PRO, NT, SUFFIX)      \
  GH_STREAM_KERNEL_NT(NAME, FMT, PARAMS, ARGS, T, G, D, PRO, NT, SUFFIX)              \
  extern "C" __global__ __launch_bounds__(NT) void NAME##_t##T##_g##G##_d##D##SUFFIX##_q( \
      GH_UNPAREN PARAMS, XPro xp, uint32_t M, uint32_t K, const uint32_t* run) {          \
    stream<FMT, T, G, D, NT, PRO>(FMT::Args{GH_UNPAREN ARGS}, xp, M, K, run);          \
  }
#define GH_STREAM_KERNEL(NAME, FMT, PARAMS, ARGS, T, G, D, PRO) \
  GH_STREAM_KERNEL_NT(NAME, FMT, PARAMS, ARGS, T, G, D, PRO, 256, )
#define GH_STREAM_KERNEL_Q(NAME, FMT, PARAMS, ARGS, T, G, D, PRO) \
  GH_STREAM_KERNEL_NT_Q(NAME, FMT, PARAMS, ARGS, T, G, D, PRO, 256, )
#define GH_UNPAREN(...) __VA_ARGS__

#define GH_P_W (const uint8_t* W, float* Y)
#define GH_A_W (W, Y)
#define GH_P_GU (const uint8_t* Wg, const uint8_t* Wu, float* Y)
#define GH_A_GU (Wg, Wu, Y)
#define GH_P_AM (const uint8_t* W, float* Y, uint32_t* partial)
#define GH_A_AM (W, Y, partial)

// Depth 1 (the default) has gated forms too; depth 2 is for tuning only.
#define GH_PLAIN_K(T, G, D, K)                                                   \
  K(gh_gemv_q4, Q4Fmt, GH_P_W, GH_A_W, T, G, D, false)                           \
  K(gh_gemv_q8, Q8Fmt, GH_P_W, GH_A_W, T, G, D, false)                           \
  K(gh_gateup_q4, GateUpFmt, GH_P_GU, GH_A_GU, T, G, D, false)                   \
  K(gh_gateup_q8, GateUpQ8Fmt, GH_P_GU, GH_A_GU, T, G, D, false)                 \
  GH_STREAM_KERNEL(gh_argmax_q8, Q8ArgmaxFmt, GH_P_AM, GH_A_AM, T, G, D, false)
#define GH_NORMED_K(T, G, D, K)                                                  \
  K(gh_gemv_q4n, Q4Fmt, GH_P_W, GH_A_W, T, G, D, true)                           \
  K(gh_gemv_q8n, Q8Fmt, GH_P_W, GH_A_W, T, G, D, true)                           \
  K(gh_gateup_q4n, GateUpFmt, GH_P_GU, GH_A_GU, T, G, D, true)                   \
  K(gh_gateup_q8n, GateUpQ8Fmt, GH_P_GU, GH_A_GU, T, G, D, true)                 \
  GH_STREAM_KERNEL(gh_argmax_q8n, Q8ArgmaxFmt, GH_P_AM, GH_A_AM, T, G, D, true)
#define GH_PLAIN(T, G, D) GH_PLAIN_K(T, G, D, GH_STREAM_KERNEL)
#define GH_PLAIN_Q(T, G, D) GH_PLAIN_K(T, G, D, GH_STREAM_KERNEL_Q)
#define GH_NORMED(T, G, D) GH_NORMED_K(T, G, D, GH_STREAM_KERNEL)
#define GH_NORMED_Q(T, G, D) GH_NORMED_K(T, G, D, GH_STREAM_KERNEL_Q)

#define GH_SHAPES(X, D) X(16, 1, D) X(32, 1, D) X(64, 1, D) X(32, 2, D) X(64, 2, D) X(32, 4, D) X(64, 4, D)

// bf16 rows (64 weights per lane item): the shapes the default pick can
// choose (one item per lane per row first, ties to the wider team).
#define GH_BF16_K(T, G, D, NORMED, SFX)                                                     \
  GH_STREAM_KERNEL_Q(gh_gemv_bf16##SFX, Bf16Fmt, GH_P_W, GH_A_W, T, G, D, NORMED)           \
  GH_STREAM_KERNEL_Q(gh_gateup_bf16##SFX, GateUpBf16Fmt, GH_P_GU, GH_A_GU, T, G, D, NORMED) \
  GH_STREAM_KERNEL(gh_argmax_bf16##SFX, Bf16ArgmaxFmt, GH_P_AM, GH_A_AM, T, G, D, NORMED)
#define GH_BF16_PLAIN(T, G, D) GH_BF16_K(T, G, D, false, )
#define GH_BF16_NORMED(T, G, D) GH_BF16_K(T, G, D, true, n)
#define GH_BF16_SHAPES(X) X(16, 1, 1) X(32, 1, 1) X(64, 1, 1) X(64, 2, 1) X(64, 4, 1)

// Wide workgroups (1024 threads) for long rows: one x staging (up to 64 KB
// of LDS for K = 15360) serves 16 wavefronts instead of 4.  (At K ~ 4096
// they measured slower than 256-thread workgroups, so only these exist.)
#define GH_WIDE(T, G, D)                                                                   \
  GH_STREAM_KERNEL_NT_Q(gh_gemv_q4, Q4Fmt, GH_P_W, GH_A_W, T, G, D, false, 1024, _w)       \
  GH_STREAM_KERNEL_NT_Q(gh_gemv_q8, Q8Fmt, GH_P_W, GH_A_W, T, G, D, false, 1024, _w)

// Depth 1 is the default everywhere; depth 2 stays for tuning (GH_GEMV_CFG).
#if defined(GH_GEMV_NORMED)
GH_SHAPES(GH_NORMED_Q, 1)
GH_SHAPES(GH_NORMED, 2)
GH_BF16_SHAPES(GH_BF16_NORMED)
// The first projection of a gated layer (QKV) with the gate in its prologue
// (mode 4, PRO = 2): "g" variants, depth 1, no run-flag test at entry
#define GH_GATED_K(T, G, D)                                          \
  GH_STREAM_KERNEL(gh_gemv_q4g, Q4Fmt, GH_P_W, GH_A_W, T, G, D, 2)   \
  GH_STREAM_KERNEL(gh_gemv_q8g, Q8Fmt, GH_P_W, GH_A_W, T, G, D, 2)
#define GH_GATED_BF16_K(T, G, D) GH_STREAM_KERNEL(gh_gemv_bf16g, Bf16Fmt, GH_P_W, GH_A_W, T, G, D, 2)
GH_SHAPES(GH_GATED_K, 1)
GH_BF16_SHAPES(GH_GATED_BF16_K)
#else
GH_SHAPES(GH_PLAIN_Q, 1)
GH_SHAPES(GH_PLAIN, 2)
GH_BF16_SHAPES(GH_BF16_PLAIN)
GH_WIDE(32, 4, 1) GH_WIDE(64, 2, 1) GH_WIDE(64, 4, 1)  // depth 2 at 1024 threads spills
// bf16 rows of K >= 8192 (64 lanes x 2 or 4 items of 64 weights): 1024-thread
// workgroups as for the quantized rows (3840 x 15360: a 61 KB x staging
// otherwise leaves two 256-thread workgroups per CU)
GH_STREAM_KERNEL_NT_Q(gh_gemv_bf16, Bf16Fmt, GH_P_W, GH_A_W, 64, 2, 1, false, 1024, _w)
GH_STREAM_KERNEL_NT_Q(gh_gemv_bf16, Bf16Fmt, GH_P_W, GH_A_W, 64, 4, 1, false, 1024, _w)

// The token from the n block partials of a fused argmax stream: the largest
// value, the lowest row among equals (src/kernels.zig:164-174).  One block.
extern "C" __global__ __launch_bounds__(256) void gh_argmax_final_k(const uint32_t* partial,
                                                                   uint32_t n, uint32_t* token) {
  __shared__ float red[8];
  float bv = -INFINITY;
  uint32_t bi = 0xFFFFFFFFu;
  for (uint32_t b = threadIdx.x; b < n; b += 256) {
    const float v = __uint_as_float(partial[2 * b]);
    const uint32_t i = partial[2 * b + 1];
    if (better(v, i, bv, bi)) {
      bv = v;
      bi = i;
    }
  }
  block_best<256>(bv, bi, red);
  if (threadIdx.x == 0) token[0] = bi == 0xFFFFFFFFu ? 0u : bi;
}
#endif
