// norm.hip -- RMSNorm, residual add + RMSNorm and greedy argmax for gfx950.
//
//   rmsnorm      shaders/rmsnorm.wgsl:13-48, src/kernels.zig:46-52
//                Y = X * (mean(X^2) + eps)^-1/2 * W
//   add_rmsnorm  shaders/add_rmsnorm.wgsl:15-51
//                X <- (X + R) * scalar (in place); Y = RMSNorm(X) * W
//   argmax       shaders/argmax.wgsl:12-48, src/kernels.zig:164-174
//                index of the largest logit; ties go to the LOWEST index, as
//                the CPU path does (the reference shader does not guarantee it)
//
// The decode step fuses the norms into the GEMV prologues and the argmax
// into the vocab GEMV; these standalone kernels are the reference-shaped
// entry points (one workgroup for a norm, as in the reference) and the
// building blocks they share.
#include <hip/hip_runtime.h>
#include <stdint.h>

#define NORM_NT 1024

__device__ __forceinline__ float block_sum(float v, float* red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = 0.f;
  const uint32_t nw = blockDim.x >> 6;
  for (uint32_t w = 0; w < nw; w++) t += red[w];
  __syncthreads();
  return t;
}

extern "C" __global__ __launch_bounds__(NORM_NT) void gh_rmsnorm_k(const float* X,
                                                                   const float* __restrict__ W,
                                                                   float* Y, uint32_t dim,
                                                                   float eps) {
  __shared__ float red[NORM_NT / 64];
  float ss = 0.f;
  for (uint32_t i = threadIdx.x; i < dim; i += blockDim.x) ss += X[i] * X[i];
  const float r = 1.0f / sqrtf(block_sum(ss, red) / (float)dim + eps);
  for (uint32_t i = threadIdx.x; i < dim; i += blockDim.x) Y[i] = X[i] * r * W[i];
}

extern "C" __global__ __launch_bounds__(NORM_NT) void gh_add_rmsnorm_k(
    float* X, const float* __restrict__ R, const float* __restrict__ W, float* Y, uint32_t dim,
    float eps, float scalar) {
  __shared__ float red[NORM_NT / 64];
  float ss = 0.f;
  for (uint32_t i = threadIdx.x; i < dim; i += blockDim.x) {
    const float v = (X[i] + R[i]) * scalar;
    X[i] = v;
    ss += v * v;
  }
  const float r = 1.0f / sqrtf(block_sum(ss, red) / (float)dim + eps);
  for (uint32_t i = threadIdx.x; i < dim; i += blockDim.x) Y[i] = X[i] * r * W[i];
}

// (value, index) order for the greedy pick: larger value wins, equal values
// go to the smaller index.
__device__ __forceinline__ bool better(float v, uint32_t i, float bv, uint32_t bi) {
  return v > bv || (v == bv && i < bi);
}

__device__ __forceinline__ void wave_argmax(float& v, uint32_t& i) {
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

// shaders/argmax.wgsl split over workgroups: each workgroup writes the best
// (value, index) of its contiguous chunk to partial[2 b], [2 b + 1];
// gh_argmax_final_k then reduces the partials to the token (no device-scope
// fence per workgroup, see the fused LM-head stream).
extern "C" __global__ __launch_bounds__(256) void gh_argmax_k(const float* __restrict__ logits,
                                                              uint32_t n, uint32_t* partial) {
  __shared__ float sv[4];
  __shared__ uint32_t si[4];
  const uint32_t per = (n + gridDim.x - 1) / gridDim.x;
  const uint32_t b0 = blockIdx.x * per, b1 = min(n, b0 + per);
  float bv = -INFINITY;
  uint32_t bi = 0xFFFFFFFFu;
  for (uint32_t i = b0 + threadIdx.x; i < b1; i += blockDim.x) {
    const float v = logits[i];
    if (better(v, i, bv, bi)) {
      bv = v;
      bi = i;
    }
  }
  wave_argmax(bv, bi);
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    sv[wave] = bv;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; w++)
      if (better(sv[w], si[w], bv, bi)) {
        bv = sv[w];
        bi = si[w];
      }
    partial[2 * blockIdx.x] = __float_as_uint(bv);
    partial[2 * blockIdx.x + 1] = bi;
  }
}

// Layer gate of the decode graph with quiescence on (shaders/
// quiescence_gate.wgsl:16-62 with the layer input it gates,
// src/gpu/model_dispatch.zig:45-101).  One workgroup.
//  1. The layer's input x: with prev_mode 1 (the previous layer ran) or 2
//     with *prev_run set, the previous layer's post-FFN add,
//       x = (xmid + RMSNorm(m) * wpost) * s      (m as given without wpost),
//     written to A; otherwise (no previous layer, or it was gated off) x is
//     A as it stands.
//  2. With gate set: mean((x - xprev)^2) over H, xprev <- x, and *run_out =
//     (mean >= thr || thr <= 0).  Without gate only step 1 runs (the
//     residual for the LM head after the last layer).
// H <= 4096 * 4 (four float4 per thread).
#define QG_U 4
extern "C" __global__ __launch_bounds__(NORM_NT) void gh_qgate_k(
    const float* xmid, const float* m, const float* __restrict__ wpost, float s,
    uint32_t prev_mode, const uint32_t* prev_run, float* A, float* xprev, float thr,
    uint32_t* run_out, uint32_t H, float eps, uint32_t gate) {
  __shared__ float red[NORM_NT / 64];
  const uint32_t n4 = H >> 2;
  // every input is loaded up front (one memory round trip; all pointers but
  // wpost are valid in every mode), then the mode picks what it uses
  const uint32_t prun = prev_mode == 2u ? *prev_run : 1u;
  float4 xv[QG_U], mv[QG_U], wv[QG_U], pv[QG_U], av[QG_U];
#pragma unroll
  for (int u = 0; u < QG_U; u++) {
    const uint32_t i = u * NORM_NT + threadIdx.x;
    const uint32_t ic = i < n4 ? i : n4 - 1;
    xv[u] = reinterpret_cast<const float4*>(xmid)[ic];
    mv[u] = reinterpret_cast<const float4*>(m)[ic];
    wv[u] = wpost ? reinterpret_cast<const float4*>(wpost)[ic] : make_float4(1.f, 1.f, 1.f, 1.f);
    pv[u] = reinterpret_cast<const float4*>(xprev)[ic];
    av[u] = reinterpret_cast<const float4*>(A)[ic];
  }
  const bool add = prev_mode == 1u || (prev_mode == 2u && prun != 0u);
  if (add) {
    float ss = 0.f;
#pragma unroll
    for (int u = 0; u < QG_U; u++)
      if (u * NORM_NT + threadIdx.x < n4)
        ss += mv[u].x * mv[u].x + mv[u].y * mv[u].y + mv[u].z * mv[u].z + mv[u].w * mv[u].w;
    const float c = wpost ? 1.0f / sqrtf(block_sum(ss, red) / (float)H + eps) : 1.0f;
#pragma unroll
    for (int u = 0; u < QG_U; u++) {
      const uint32_t i = u * NORM_NT + threadIdx.x;
      const float4 r = wpost ? make_float4(mv[u].x * c * wv[u].x, mv[u].y * c * wv[u].y,
                                           mv[u].z * c * wv[u].z, mv[u].w * c * wv[u].w)
                             : mv[u];
      av[u] = make_float4((xv[u].x + r.x) * s, (xv[u].y + r.y) * s, (xv[u].z + r.z) * s,
                          (xv[u].w + r.w) * s);
      if (i < n4) reinterpret_cast<float4*>(A)[i] = av[u];
    }
  }
  if (!gate) return;
  float d = 0.f;
#pragma unroll
  for (int u = 0; u < QG_U; u++) {
    const uint32_t i = u * NORM_NT + threadIdx.x;
    if (i < n4) {
      const float a = av[u].x - pv[u].x, b = av[u].y - pv[u].y, e = av[u].z - pv[u].z,
                  f = av[u].w - pv[u].w;
      d += a * a + b * b + e * e + f * f;
      reinterpret_cast<float4*>(xprev)[i] = av[u];
    }
  }
  const float ms = block_sum(d, red) / (float)H;
  if (threadIdx.x == 0) *run_out = (ms >= thr || thr <= 0.0f) ? 1u : 0u;
}
