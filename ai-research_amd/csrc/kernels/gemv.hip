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
//    with the per-block sum_j x_j precomputed while staging x.  Nibbles are
//    split with two ANDs (0x0F0F0F0F / 0xF0F0F0F0); each byte converts with
//    one v_cvt_f32_ubyte{0..3}; the high nibbles carry a factor 16 that is
//    removed once per block (exact power-of-two scale).  Q8 flips the sign
//    bit of each byte (q + 128) and removes 128 sum x the same way.
//  * fp32 accumulation throughout.
#include <hip/hip_runtime.h>
#include <stdint.h>

#define WG 256
#define GROUP_STRIDE 132  // floats per 128-element x group in LDS (+4 pad)

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }

// Weights are streamed once per token: non-temporal 16-byte loads.
__device__ __forceinline__ u32x4 ldnt(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// Stage x[K] into LDS (padded by group) and write the per-block sums.
// K % 128 == 0.  All threads of the block must call it.
__device__ __forceinline__ void stage_x(const float* __restrict__ X, uint32_t K,
                                        float* xs, float* bsum) {
  const uint32_t n4 = K >> 2;
  for (uint32_t i = threadIdx.x; i < n4; i += WG) {
    float4 v = reinterpret_cast<const float4*>(X)[i];
    uint32_t e = i << 2;                     // element index
    uint32_t g = e >> 7, o = e & 127;        // group, offset in group
    *reinterpret_cast<float4*>(xs + g * GROUP_STRIDE + o) = v;
    float s = (v.x + v.y) + (v.z + v.w);
    // a block is 8 consecutive float4s = 8 consecutive lanes (n4 % 8 == 0,
    // so a lane group of 8 is either fully active or fully inactive)
    s += __shfl_xor(s, 1, 8);
    s += __shfl_xor(s, 2, 8);
    s += __shfl_xor(s, 4, 8);
    if ((i & 7) == 0) bsum[i >> 3] = s;
  }
  __syncthreads();
}

// v_cvt_f32_ubyte{0..3}: byte k of a dword to float in one instruction.  The
// compiler folds the 0x0F0F0F0F masks into bit-field extracts and loses this
// form, so it is spelled out.
#define GH_CVT_UB(N)                                                    \
  __device__ __forceinline__ float cvt_ub##N(uint32_t x) {              \
    float r;                                                            \
    asm("v_cvt_f32_ubyte" #N " %0, %1" : "=v"(r) : "v"(x));             \
    return r;                                                           \
  }
GH_CVT_UB(0)
GH_CVT_UB(1)
GH_CVT_UB(2)
GH_CVT_UB(3)

// sum_j n_j x_j over one Q4 block, n_j = nibble j (0..15).
__device__ __forceinline__ float q4_nx(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3,
                                       const float* __restrict__ xb) {
  const uint32_t w[4] = {w0, w1, w2, w3};
  float sl = 0.f, sh = 0.f;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const uint32_t lo = w[k] & 0x0F0F0F0Fu;  // nibbles 0,2,4,6 -> elements 8k+0,2,4,6
    const uint32_t hi = w[k] & 0xF0F0F0F0u;  // 16 x nibbles 1,3,5,7
    const float4 xa = *reinterpret_cast<const float4*>(xb + 8 * k);
    const float4 xc = *reinterpret_cast<const float4*>(xb + 8 * k + 4);
    sl += cvt_ub0(lo) * xa.x;
    sh += cvt_ub0(hi) * xa.y;
    sl += cvt_ub1(lo) * xa.z;
    sh += cvt_ub1(hi) * xa.w;
    sl += cvt_ub2(lo) * xc.x;
    sh += cvt_ub2(hi) * xc.y;
    sl += cvt_ub3(lo) * xc.z;
    sh += cvt_ub3(hi) * xc.w;
  }
  return sl + sh * 0.0625f;
}

// sum_j (q_j + 128) x_j over one Q8 block given its 8 packed words.
__device__ __forceinline__ float q8_ux(const uint32_t* w, const float* __restrict__ xb) {
  float s0 = 0.f, s1 = 0.f;
#pragma unroll
  for (int k = 0; k < 8; k++) {
    const uint32_t u = w[k] ^ 0x80808080u;  // int8 q -> uint8 q + 128
    const float4 xa = *reinterpret_cast<const float4*>(xb + 4 * k);
    s0 += cvt_ub0(u) * xa.x;
    s1 += cvt_ub1(u) * xa.y;
    s0 += cvt_ub2(u) * xa.z;
    s1 += cvt_ub3(u) * xa.w;
  }
  return s0 + s1;
}

struct Q4G {
  u32x4 a0, a1, a2, a3, a4;
};

__device__ __forceinline__ Q4G load_q4g(const uint8_t* p) {
  Q4G g;
  g.a0 = ldnt(p + 0);
  g.a1 = ldnt(p + 16);
  g.a2 = ldnt(p + 32);
  g.a3 = ldnt(p + 48);
  g.a4 = ldnt(p + 64);
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

template <int TPR>
__device__ __forceinline__ float team_sum(float v) {
#pragma unroll
  for (int off = TPR / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, TPR);
  return v;
}

__device__ __forceinline__ float gelu_tanh(float x) {
  // kernels.zig:94-97 / fused_mlp_q4.wgsl:15-18
  const float inner = 0.7978845608f * (x + 0.044715f * x * x * x);
  return 0.5f * x * (1.0f + tanhf(inner));
}

// ------------------------------------------------------------------------
// Q4_0 GEMV
// ------------------------------------------------------------------------
template <int TPR, int RPT>
__device__ __forceinline__ void gemv_q4_body(const uint8_t* __restrict__ W,
                                             const float* __restrict__ X,
                                             float* __restrict__ Y, uint32_t M, uint32_t K) {
  extern __shared__ float lds[];
  const uint32_t nb = K >> 5, ng = nb >> 2;
  float* xs = lds;
  float* bsum = lds + ng * GROUP_STRIDE;
  stage_x(X, K, xs, bsum);

  constexpr int TEAMS = WG / TPR;
  const uint32_t lr = threadIdx.x % TPR;
  const uint32_t row0 = (blockIdx.x * TEAMS + threadIdx.x / TPR) * RPT;
  const size_t row_bytes = (size_t)nb * 20;
  float acc[RPT];
#pragma unroll
  for (int r = 0; r < RPT; r++) acc[r] = 0.f;

  for (uint32_t g = lr; g < ng; g += TPR) {
    Q4G q[RPT];
#pragma unroll
    for (int r = 0; r < RPT; r++) {
      const uint32_t row = row0 + r < M ? row0 + r : M - 1;  // clamp: tail rows are discarded
      q[r] = load_q4g(W + (size_t)row * row_bytes + (size_t)g * 80);
    }
    const float* xg = xs + g * GROUP_STRIDE;
    const float* bs = bsum + g * 4;
#pragma unroll
    for (int r = 0; r < RPT; r++) acc[r] += q4_group_dot(q[r], xg, bs);
  }
#pragma unroll
  for (int r = 0; r < RPT; r++) {
    const float v = team_sum<TPR>(acc[r]);
    if (lr == 0 && row0 + r < M) Y[row0 + r] = v;
  }
}

// ------------------------------------------------------------------------
// fused gate + up GeGLU on Q4_0 rows
// ------------------------------------------------------------------------
template <int TPR, int RPT>
__device__ __forceinline__ void gateup_q4_body(const uint8_t* __restrict__ Wg,
                                               const uint8_t* __restrict__ Wu,
                                               const float* __restrict__ X,
                                               float* __restrict__ Y, uint32_t M, uint32_t K) {
  extern __shared__ float lds[];
  const uint32_t nb = K >> 5, ng = nb >> 2;
  float* xs = lds;
  float* bsum = lds + ng * GROUP_STRIDE;
  stage_x(X, K, xs, bsum);

  constexpr int TEAMS = WG / TPR;
  const uint32_t lr = threadIdx.x % TPR;
  const uint32_t row0 = (blockIdx.x * TEAMS + threadIdx.x / TPR) * RPT;
  const size_t row_bytes = (size_t)nb * 20;
  float ag[RPT], au[RPT];
#pragma unroll
  for (int r = 0; r < RPT; r++) ag[r] = au[r] = 0.f;

  for (uint32_t g = lr; g < ng; g += TPR) {
    Q4G qg[RPT], qu[RPT];
#pragma unroll
    for (int r = 0; r < RPT; r++) {
      const uint32_t row = row0 + r < M ? row0 + r : M - 1;
      const size_t off = (size_t)row * row_bytes + (size_t)g * 80;
      qg[r] = load_q4g(Wg + off);
      qu[r] = load_q4g(Wu + off);
    }
    const float* xg = xs + g * GROUP_STRIDE;
    const float* bs = bsum + g * 4;
#pragma unroll
    for (int r = 0; r < RPT; r++) {
      ag[r] += q4_group_dot(qg[r], xg, bs);
      au[r] += q4_group_dot(qu[r], xg, bs);
    }
  }
#pragma unroll
  for (int r = 0; r < RPT; r++) {
    const float gsum = team_sum<TPR>(ag[r]);
    const float usum = team_sum<TPR>(au[r]);
    if (lr == 0 && row0 + r < M) Y[row0 + r] = gelu_tanh(gsum) * usum;
  }
}

// ------------------------------------------------------------------------
// Q8_0 GEMV
// ------------------------------------------------------------------------
template <int TPR, int RPT>
__device__ __forceinline__ void gemv_q8_body(const uint8_t* __restrict__ W,
                                             const float* __restrict__ X,
                                             float* __restrict__ Y, uint32_t M, uint32_t K) {
  extern __shared__ float lds[];
  const uint32_t nb = K >> 5, ng = nb >> 2;
  float* xs = lds;
  float* bsum = lds + ng * GROUP_STRIDE;
  stage_x(X, K, xs, bsum);

  constexpr int TEAMS = WG / TPR;
  const uint32_t lr = threadIdx.x % TPR;
  const uint32_t row0 = (blockIdx.x * TEAMS + threadIdx.x / TPR) * RPT;
  const size_t row_bytes = (size_t)nb * 36;
  float acc[RPT];
#pragma unroll
  for (int r = 0; r < RPT; r++) acc[r] = 0.f;

  for (uint32_t g = lr; g < ng; g += TPR) {
    uint32_t w[RPT][36];
#pragma unroll
    for (int r = 0; r < RPT; r++) {
      const uint32_t row = row0 + r < M ? row0 + r : M - 1;
      const uint8_t* p = W + (size_t)row * row_bytes + (size_t)g * 144;
#pragma unroll
      for (int v = 0; v < 9; v++) {
        const u32x4 t = ldnt(p + 16 * v);
        w[r][4 * v + 0] = t.x;
        w[r][4 * v + 1] = t.y;
        w[r][4 * v + 2] = t.z;
        w[r][4 * v + 3] = t.w;
      }
    }
    const float* xg = xs + g * GROUP_STRIDE;
    const float* bs = bsum + g * 4;
#pragma unroll
    for (int r = 0; r < RPT; r++) {
#pragma unroll
      for (int j = 0; j < 4; j++)
        acc[r] += u2f(w[r][9 * j]) * (q8_ux(&w[r][9 * j + 1], xg + 32 * j) - 128.0f * bs[j]);
    }
  }
#pragma unroll
  for (int r = 0; r < RPT; r++) {
    const float v = team_sum<TPR>(acc[r]);
    if (lr == 0 && row0 + r < M) Y[row0 + r] = v;
  }
}

#define GH_GEMV_INST(T, R)                                                                     \
  extern "C" __global__ __launch_bounds__(WG) void gh_gemv_q4_t##T##_r##R(                      \
      const uint8_t* W, const float* X, float* Y, uint32_t M, uint32_t K) {                     \
    gemv_q4_body<T, R>(W, X, Y, M, K);                                                          \
  }                                                                                             \
  extern "C" __global__ __launch_bounds__(WG) void gh_gateup_q4_t##T##_r##R(                    \
      const uint8_t* Wg, const uint8_t* Wu, const float* X, float* Y, uint32_t M, uint32_t K) { \
    gateup_q4_body<T, R>(Wg, Wu, X, Y, M, K);                                                   \
  }                                                                                             \
  extern "C" __global__ __launch_bounds__(WG) void gh_gemv_q8_t##T##_r##R(                      \
      const uint8_t* W, const float* X, float* Y, uint32_t M, uint32_t K) {                     \
    gemv_q8_body<T, R>(W, X, Y, M, K);                                                          \
  }

GH_GEMV_INST(8, 1)
GH_GEMV_INST(8, 2)
GH_GEMV_INST(8, 4)
GH_GEMV_INST(16, 1)
GH_GEMV_INST(16, 2)
GH_GEMV_INST(16, 4)
GH_GEMV_INST(32, 1)
GH_GEMV_INST(32, 2)
GH_GEMV_INST(32, 4)
GH_GEMV_INST(64, 1)
GH_GEMV_INST(64, 2)
GH_GEMV_INST(64, 4)
