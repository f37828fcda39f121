// prefill.hip -- batched prefill for gfx950: the MFMA Q4_0 / Q8_0 dequant GEMM
// and the row-wise norm that feeds it.
//
// The reference has no batched prefill: it runs prompt tokens one at a time
// through its decode graph without logits (src/interactive.zig:33-37,
// src/gpu/model_dispatch.zig:144).  Here the T prompt tokens of a layer go
// through each projection as one dense contraction
//     C[T][N] = A[T][K] . deq(W)[N][K]^T
// on the matrix cores (v_mfma_f32_32x32x16_f16), keeping the decode path's
// accuracy:
//  * weights enter exactly: the MFMA B operand is the integer n - 8 (Q4) or
//    q (Q8), exact in fp16, and each 32-block's f32 scale d is applied to the
//    block's fp32 partial sum (acc += d * block_sum), as the GEMV does;
//  * activations are split a = s (hi + lo) with hi = fp16(a / s),
//    lo = fp16(a / s - hi) and s a power of two per row that puts the row's
//    largest |a| / s in [2^13, 2^14) (no fp16 overflow for any row), and both
//    halves go through the MFMA (22+ significant bits of a).  The split is
//    made once per row (gh_pf_halves_k, or gh_pf_norm_k for normed rows),
//    not in every tile that reads the row, and s is applied in the epilogue
//    (exact: a power of two);
//  * accumulation is fp32.
//
// Tiling: a workgroup of 256 threads (2 x 2 wavefronts) owns a BM x BN tile
// of C; each wavefront a (BM/2) x (BN/2) sub-tile of 32 x 32 MFMA blocks (the
// _w8 forms of the 128-row tiles: 512 threads, 4 x 2 wavefronts of
// (BM/4) x (BN/2), so a CU's two tiles run four waves per SIMD).  K
// advances one quant block (32) per step: the A slice (as hi and lo) and the
// integer W slice with its scales go to LDS in unpadded, XOR-swizzled rows
// (bank-conflict-free operand reads and stage writes).  Two LDS stages:
// while the MFMAs of step s read one, step s+1's global loads are in flight
// and then stored into the other, one barrier per step.  Workgroups take
// their tiles in an XCD-aware order (the tiles of one XCD share A rows).
//
// MFMA 32x32x16 f16 operand layout (checked on the device): lane l holds
// A[l % 32][8 (l / 32) + e] and B[8 (l / 32) + e][l % 32], e = 0..7; result
// register r of lane l is C[8 (r / 4) + 4 (l / 32) + r % 4][l % 32].
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

#define PF_NT 256

// Weight words through an explicit global-address-space pointer: the matrix
// is picked at run time (gate or up), which would otherwise degrade to FLAT.
typedef const uint32_t __attribute__((address_space(1)))* gword_ptr;

struct Q4W {  // src/quant.zig:55-90: {f32 d, 4 words of nibbles}
  static constexpr uint32_t kBlockBytes = 20;
  static constexpr int kWords = 3;
  static constexpr bool kBf16 = false;
  // half h (elements 16h .. 16h+15) of a block: scale and its 16 values
  __device__ static void load(const uint8_t* blk, uint32_t h, uint32_t* w) {
    gword_ptr p = (gword_ptr)(blk);
    w[0] = p[0];
    w[1] = p[1 + 2 * h];
    w[2] = p[2 + 2 * h];
  }
  // n - 8 as fp16 pairs, exactly: (w >> 4j) & 0x000F000F | 0x64006400 read as
  // two halves is (1024 + n_j, 1024 + n_{j+4}), and one packed subtract of
  // 1032 leaves (n_j - 8, n_{j+4} - 8).  So the 8 elements of a word come out
  // in the K order (0,4,1,5,2,6,3,7); the A operand is stored in the same
  // order (pf_ax_pos with perm).  out: 8 words = the half-block's 16 halves.
  __device__ static void ints(const uint32_t* w, uint32_t* out) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 bias = {(_Float16)-1032.0f, (_Float16)-1032.0f};
#pragma unroll
    for (int k = 0; k < 2; k++)
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const uint32_t pr = ((w[1 + k] >> (4 * j)) & 0x000F000Fu) | 0x64006400u;
        out[4 * k + j] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, pr) + bias);
      }
  }
};

struct Q8W {  // src/quant.zig:20-51: {f32 d, 8 words of int8}
  static constexpr uint32_t kBlockBytes = 36;
  static constexpr int kWords = 5;
  static constexpr bool kBf16 = false;
  __device__ static void load(const uint8_t* blk, uint32_t h, uint32_t* w) {
    gword_ptr p = (gword_ptr)(blk);
    w[0] = p[0];
#pragma unroll
    for (int k = 0; k < 4; k++) w[1 + k] = p[1 + 4 * h + k];
  }
  __device__ static void ints(const uint32_t* w, uint32_t* out) {  // q as fp16, in K order
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int k = 0; k < 4; k++)
#pragma unroll
      for (int n = 0; n < 4; n += 2) {
        const h2 v = {(_Float16)(int)(int8_t)((w[1 + k] >> (8 * n)) & 0xFFu),
                      (_Float16)(int)(int8_t)((w[1 + k] >> (8 * n + 8)) & 0xFFu)};
        out[2 * k + n / 2] = __builtin_bit_cast(uint32_t, v);
      }
  }
};

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef const u32x4_t __attribute__((address_space(1)))* gvec_ptr;

// bf16 rows as stored (mode none, the reference's --gpu weights): 32 bf16 of
// a row per K step go to the stage as they are and feed the bf16 MFMA
// directly; there is no unpacking and no block scale (kBf16).
struct Bf16W {
  static constexpr uint32_t kBlockBytes = 64;
  static constexpr int kWords = 8;
  static constexpr bool kBf16 = true;
  // half h (elements 16h .. 16h+15) of a 32-element segment: 8 words
  __device__ static void load(const uint8_t* blk, uint32_t h, uint32_t* w) {
    gvec_ptr p = (gvec_ptr)(blk + 32 * h);
    const u32x4_t a = p[0], b = p[1];
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
    w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
  }
  __device__ static void ints(const uint32_t* w, uint32_t* out) {
#pragma unroll
    for (int k = 0; k < 8; k++) out[k] = w[k];
  }
};

__device__ __forceinline__ float gelu_tanh(float x) {
  // kernels.zig:94-97 / fused_mlp_q4.wgsl:15-18
  const float inner = 0.7978845608f * (x + 0.044715f * x * x * x);
  return 0.5f * x * (1.0f + tanhf(inner));
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// The GEMM's A operand layout ("ax"): row t of K elements is 2K halves, the
// hi halves of block b (elements 32b .. 32b+31) at 64b, their lo halves at
// 64b + 32.  With perm (Q4_0 weights) the 8 elements of each group sit in the
// order Q4W::ints unpacks a word: position 2m holds element m, 2m + 1 element
// m + 4.  Offset of element e's hi half within its row:
__device__ __forceinline__ uint32_t pf_ax_pos(uint32_t e, bool perm) {
  const uint32_t j = e & 7;
  return (e >> 5) * 64 + (e & 24) + (perm ? ((j & 3) << 1) | (j >> 2) : j);
}

// NMAT = 1: C = A W^T.  NMAT = 2: C = gelu_tanh(A Wg^T) * (A Wu^T).  A as its
// fp16 hi/lo halves interleaved per 32-element block (pf_ax: a row's K step
// is one contiguous 128-byte segment) and row scales rs; C f32.
// Each step covers KB quant blocks (32 KB elements of K).
// SPLIT (split-K, for few tiles): workgroup z of gridDim.z runs K steps
// [z S / Z, (z + 1) S / Z) and writes its raw sums to C as partial plane
// (z, matrix) of [Z][NMAT][T][N]; gh_pf_splitk_k adds the planes in z order
// and applies the epilogue.
// NW: waves per workgroup, 4 (2 x 2, each (BM/2) x (BN/2)) or 8 (4 x 2, each
// (BM/4) x (BN/2)).
template <class F, int BM, int BN, int NMAT, int KB, bool SPLIT, int NW = 4>
__device__ __forceinline__ void gemm_tile(const _Float16* __restrict__ Ax,
                                          const float* __restrict__ rs,
                                          const uint8_t* __restrict__ W0,
                                          const uint8_t* __restrict__ W1, float* __restrict__ C,
                                          uint32_t T, uint32_t N, uint32_t K) {
  static_assert(KB == 1, "one quant block per K step (the LDS swizzle assumes it)");
  static_assert(NW == 4 || NW == 8, "2 x 2 or 4 x 2 waves");
  constexpr int NT = 64 * NW;
  constexpr int TM = BM / (16 * NW), TN = BN / 64;  // 32x32 blocks per wave in M and N
  static_assert(TM >= 1, "a wave holds at least one 32-row block");
  constexpr int A_CH = 8 * KB;                               // 16-B chunks per row and step
  constexpr int A_PER = BM * A_CH / NT;                      // 16-B chunks per thread
  constexpr int B_ROWS = NMAT * BN;                          // weight rows per step
  constexpr int B_HALVES = 2 * KB * B_ROWS;                  // 16-element half-blocks
  constexpr int B_PER = (B_HALVES + NT - 1) / NT;
  static_assert(A_PER >= 1 && (BM * A_CH) % NT == 0, "A chunks divide the workgroup");
  // Two LDS stages: the MFMAs of step s read one while step s+1 is stored
  // into the other, so a K step needs one barrier.  A row of a stage is 128 B
  // (8 chunks of 8 halves: hi 0-3, lo 4-7), a weight row 64 B (4 chunks), with
  // no padding; chunk k of row r sits at k ^ sa(r) (A) or k ^ sb(r) (weights).
  // The swizzles keep every ds_read_b128 of the MFMA operands (16 rows at one
  // chunk) and every ds_write_b128 of a stage (2 A rows, or 8 weight rows at
  // two chunks) on distinct banks, for 8-lane phases over 32 banks as well as
  // 16-lane phases over 64.  (An 80-byte padded row was conflict-free to read
  // but not to write: write conflicts cost as many LDS cycles as the reads.)
  __shared__ _Float16 SA[2][BM * 64];
  __shared__ _Float16 Bs[2][B_ROWS * 32];
  __shared__ float Ds[2][B_ROWS * KB];
  auto a_at = [](uint32_t r, uint32_t k) { return r * 64 + 8 * (k ^ ((r & 7) ^ ((r >> 3) & 1))); };
  auto b_at = [](uint32_t r, uint32_t k) { return r * 32 + 8 * (k ^ (((r >> 1) ^ (r >> 2)) & 3)); };

  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // XCD-aware tile order: workgroups go to the 8 XCDs round-robin (w % 8), so
  // XCD c takes the c-th contiguous eighth of the tiles in (split, m, n)
  // order, n fastest.  The tiles of one XCD then share their A rows (one
  // 128-row block of a 512-token prompt is 2 MB: it stays in the XCD's L2)
  // instead of every XCD cycling through all of A.
  const uint32_t gx = gridDim.x, gy = gridDim.y, gz = SPLIT ? gridDim.z : 1u;
  const uint32_t G = gx * gy * gz;
  uint32_t w = blockIdx.x + gx * (blockIdx.y + gy * (SPLIT ? blockIdx.z : 0u));
  if (G % 8 == 0) w = (w % 8) * (G / 8) + w / 8;
  const uint32_t tn = w % gx, tm = (w / gx) % gy;
  const uint32_t m0 = tm * BM, n0 = tn * BN;
  const uint32_t wm = (wave >> 1) * (BM / (NW / 2)), wn = (wave & 1) * (BN / 2);
  const uint32_t nb = K / 32, nsteps = (nb + KB - 1) / KB;
  const size_t row_bytes = (size_t)nb * F::kBlockBytes;

  // global -> register staging of one K step (blocks past K load block nb - 1
  // and are multiplied by a zero scale)
  u32x4 ra[A_PER];  // a native vector: plain loads and stores, kept in registers
  uint32_t rb[B_PER][F::kWords];
  auto load_step = [&](uint32_t step) {
#pragma unroll
    for (int i = 0; i < A_PER; i++) {
      // chunk c: row c / A_CH; q = c % A_CH -> block q / 8 of the step, plane
      // (q / 4) % 2, 8 halves at (q % 4) * 8
      const uint32_t c = tid + i * NT, q = c % A_CH;
      uint32_t r = m0 + c / A_CH;
      r = r < T ? r : T - 1;
      uint32_t blk = step * KB + q / 8;
      blk = blk < nb ? blk : nb - 1;
      ra[i] = *reinterpret_cast<const u32x4*>(Ax + (size_t)r * 2 * K + (size_t)blk * 64 + 8 * (q % 8));
    }
#pragma unroll
    for (int i = 0; i < B_PER; i++) {
      const uint32_t hb = tid + i * NT;  // ((row * KB) + block) * 2 + half
      if (hb < (uint32_t)B_HALVES) {
        const uint32_t lr = hb / (2 * KB), kq = (hb / 2) % KB, mat = lr / BN;
        uint32_t r = n0 + lr % BN;
        r = r < N ? r : N - 1;
        uint32_t blk = step * KB + kq;
        blk = blk < nb ? blk : nb - 1;
        const uint8_t* W = mat ? W1 : W0;
        F::load(W + (size_t)r * row_bytes + (size_t)blk * F::kBlockBytes, hb % 2, rb[i]);
      }
    }
  };
  auto store_step = [&](int sb, uint32_t step) {
#pragma unroll
    for (int i = 0; i < A_PER; i++) {
      const uint32_t c = tid + i * NT;
      *reinterpret_cast<u32x4*>(&SA[sb][a_at(c / A_CH, c % A_CH)]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_PER; i++) {
      const uint32_t hb = tid + i * NT;
      if (hb < (uint32_t)B_HALVES) {
        const uint32_t lr = hb / (2 * KB), kq = (hb / 2) % KB;
        uint32_t v[8];
        F::ints(rb[i], v);
        *reinterpret_cast<u32x4*>(&Bs[sb][b_at(lr, 2 * (hb % 2))]) = u32x4{v[0], v[1], v[2], v[3]};
        *reinterpret_cast<u32x4*>(&Bs[sb][b_at(lr, 2 * (hb % 2) + 1)]) = u32x4{v[4], v[5], v[6], v[7]};
        if constexpr (!F::kBf16)
          if (hb % 2 == 0) Ds[sb][lr * KB + kq] = step * KB + kq < nb ? __uint_as_float(rb[i][0]) : 0.f;
      }
    }
  };

  f32x16 acc[NMAT][TM][TN];
#pragma unroll
  for (int q = 0; q < NMAT; q++)
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int j = 0; j < TN; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[q][i][j][r] = 0.f;

  const uint32_t nz = gz, z = w / (gx * gy);
  const uint32_t s_begin = (uint32_t)((uint64_t)nsteps * z / nz);
  const uint32_t s_end = (uint32_t)((uint64_t)nsteps * (z + 1) / nz);
  if (s_begin < s_end) {
    load_step(s_begin);
    store_step(0, s_begin);
  }
  __syncthreads();
  for (uint32_t step = s_begin; step < s_end; step++) {
    const int cb = (step - s_begin) & 1;
    if (step + 1 < s_end) load_step(step + 1);  // in flight through this step's MFMAs
#pragma unroll
    for (int kq = 0; kq < KB; kq++) {
      half8 ah[2][TM], al[2][TM];
#pragma unroll
      for (int h = 0; h < 2; h++)
#pragma unroll
        for (int i = 0; i < TM; i++) {
          const uint32_t r = wm + 32 * i + lane % 32, k = 2 * h + lane / 32;
          ah[h][i] = *reinterpret_cast<const half8*>(&SA[cb][a_at(r, k)]);
          al[h][i] = *reinterpret_cast<const half8*>(&SA[cb][a_at(r, 4 + k)]);
        }
#pragma unroll
      for (int q = 0; q < NMAT; q++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
          const uint32_t brow = q * BN + wn + 32 * j + lane % 32;
          const half8 b0 = *reinterpret_cast<const half8*>(&Bs[cb][b_at(brow, lane / 32)]);
          const half8 b1 = *reinterpret_cast<const half8*>(&Bs[cb][b_at(brow, 2 + lane / 32)]);
          if constexpr (F::kBf16) {
            // exact bf16 weights and bf16 activation halves: every product
            // accumulates straight into the tile (one block per step, so no
            // step lies past K)
            const bf16x8 c0 = __builtin_bit_cast(bf16x8, b0), c1 = __builtin_bit_cast(bf16x8, b1);
#pragma unroll
            for (int i = 0; i < TM; i++) {
              f32x16 t = acc[q][i][j];
              t = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, ah[0][i]), c0, t, 0, 0, 0);
              t = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, al[0][i]), c0, t, 0, 0, 0);
              t = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, ah[1][i]), c1, t, 0, 0, 0);
              t = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, al[1][i]), c1, t, 0, 0, 0);
              acc[q][i][j] = t;
            }
            continue;
          }
          const float d = Ds[cb][brow * KB + kq];
#pragma unroll
          for (int i = 0; i < TM; i++) {
            f32x16 blk = {};
            blk = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[0][i], b0, blk, 0, 0, 0);
            blk = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[0][i], b0, blk, 0, 0, 0);
            blk = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[1][i], b1, blk, 0, 0, 0);
            blk = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[1][i], b1, blk, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 16; r++) acc[q][i][j][r] += d * blk[r];
          }
        }
    }
    if (step + 1 < s_end) store_step(cb ^ 1, step + 1);
    // the next step reads the stage just stored, and then stores into the
    // stage read here
    __syncthreads();
  }

  // epilogue: result register r of lane l -> row 8 (r/4) + 4 (l/32) + r%4, col l % 32
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++) {
      const uint32_t col = n0 + wn + 32 * j + lane % 32;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const uint32_t row = m0 + wm + 32 * i + 8 * (r / 4) + 4 * (lane / 32) + r % 4;
        if (row < T && col < N) {
          const float sr = rs[row];
          if constexpr (SPLIT) {
#pragma unroll
            for (int q = 0; q < NMAT; q++)
              C[((size_t)(z * NMAT + q) * T + row) * N + col] = acc[q][i][j][r] * sr;
          } else if constexpr (NMAT == 1) {
            C[(size_t)row * N + col] = acc[0][i][j][r] * sr;
          } else {
            C[(size_t)row * N + col] = gelu_tanh(acc[0][i][j][r] * sr) * (acc[1][i][j][r] * sr);
          }
        }
      }
    }
}

#define GH_GEMM(NAME, F, BM, BN, KB, SPLIT, SUFFIX)                                       \
  extern "C" __global__ __launch_bounds__(PF_NT) GH_PF_OCC_##BM void NAME##_k##KB##SUFFIX( \
      const _Float16* Ax, const float* rs, const uint8_t* W, float* C, uint32_t T,         \
      uint32_t N, uint32_t K) {                                                            \
    gemm_tile<F, BM, BN, 1, KB, SPLIT>(Ax, rs, W, W, C, T, N, K);                          \
  }
#define GH_GEMM_W8(NAME, F, BM, BN, KB, SPLIT, SUFFIX)                                    \
  extern "C" __global__ __launch_bounds__(512) GH_PF_OCC_W8 void NAME##_k##KB##SUFFIX(     \
      const _Float16* Ax, const float* rs, const uint8_t* W, float* C, uint32_t T,         \
      uint32_t N, uint32_t K) {                                                            \
    gemm_tile<F, BM, BN, 1, KB, SPLIT, 8>(Ax, rs, W, W, C, T, N, K);                       \
  }
#define GH_GEMM_PAIR_W8(NAME, F, BM, BN, KB, SPLIT, SUFFIX)                               \
  extern "C" __global__ __launch_bounds__(512) GH_PF_OCC_W8 void NAME##_k##KB##SUFFIX(     \
      const _Float16* Ax, const float* rs, const uint8_t* Wg, const uint8_t* Wu,           \
      float* Act, uint32_t T, uint32_t N, uint32_t K) {                                    \
    gemm_tile<F, BM, BN, 2, KB, SPLIT, 8>(Ax, rs, Wg, Wu, Act, T, N, K);                   \
  }
#define GH_PF_OCC_W8 __attribute__((amdgpu_waves_per_eu(4, 4)))
#define GH_GEMM_PAIR(NAME, F, BM, BN, KB, SPLIT, SUFFIX)                                  \
  extern "C" __global__ __launch_bounds__(PF_NT) GH_PF_OCC_##BM void NAME##_k##KB##SUFFIX( \
      const _Float16* Ax, const float* rs, const uint8_t* Wg, const uint8_t* Wu,           \
      float* Act, uint32_t T, uint32_t N, uint32_t K) {                                    \
    gemm_tile<F, BM, BN, 2, KB, SPLIT>(Ax, rs, Wg, Wu, Act, T, N, K);                      \
  }
// The 128-row tiles are held to 2 waves per SIMD: at 3 (the register count
// allows it) they measured ~2x slower, the third workgroup's tiles evicting
// the first two's operands.
#define GH_PF_OCC_128 __attribute__((amdgpu_waves_per_eu(1, 2)))
#define GH_PF_OCC_64
#define GH_GEMM_ALL                                                       \
  GH_GEMM(gh_pf_gemm_q4_m128_n128, Q4W, 128, 128, 1, false, )             \
  GH_GEMM(gh_pf_gemm_q4_m128_n64, Q4W, 128, 64, 1, false, )               \
  GH_GEMM(gh_pf_gemm_q4_m64_n64, Q4W, 64, 64, 1, false, )                 \
  GH_GEMM(gh_pf_gemm_q8_m128_n128, Q8W, 128, 128, 1, false, )             \
  GH_GEMM(gh_pf_gemm_q8_m128_n64, Q8W, 128, 64, 1, false, )               \
  GH_GEMM(gh_pf_gemm_q8_m64_n64, Q8W, 64, 64, 1, false, )                 \
  GH_GEMM_PAIR(gh_pf_gateup_q4_m128_n64, Q4W, 128, 64, 1, false, )        \
  GH_GEMM_PAIR(gh_pf_gateup_q4_m64_n64, Q4W, 64, 64, 1, false, )          \
  GH_GEMM_PAIR(gh_pf_gateup_q8_m128_n64, Q8W, 128, 64, 1, false, )        \
  GH_GEMM_PAIR(gh_pf_gateup_q8_m64_n64, Q8W, 64, 64, 1, false, )

// One quant block per K step measured fastest (12B prefill 62.7 ms vs 65.9
// and 68.4 ms at 2 and 4 blocks), and loading 2 or 3 steps ahead in a
// register ring slower (72-77 ms vs 64): the step is bound by its barriers
// and MFMA dependency chains, not by load latency.
GH_GEMM_ALL

// Split-K forms, for products whose tiles alone cannot fill the CUs: the
// small tile for a few prompt tokens (without the split each workgroup walks
// all of K one block per step, and that serial chain, not bandwidth, sets the
// time), and the large plain tile for the narrow products of a long prompt
// (o and down, N = 3840), which otherwise fall back to the small tile.
GH_GEMM(gh_pf_gemm_bf16_m128_n128, Bf16W, 128, 128, 1, false, )
GH_GEMM(gh_pf_gemm_bf16_m128_n64, Bf16W, 128, 64, 1, false, )
GH_GEMM(gh_pf_gemm_bf16_m64_n64, Bf16W, 64, 64, 1, false, )
GH_GEMM_PAIR(gh_pf_gateup_bf16_m128_n64, Bf16W, 128, 64, 1, false, )
GH_GEMM_PAIR(gh_pf_gateup_bf16_m64_n64, Bf16W, 64, 64, 1, false, )
GH_GEMM(gh_pf_gemm_bf16_m64_n64, Bf16W, 64, 64, 1, true, _s)
GH_GEMM(gh_pf_gemm_bf16_m128_n128, Bf16W, 128, 128, 1, true, _s)
GH_GEMM_PAIR(gh_pf_gateup_bf16_m64_n64, Bf16W, 64, 64, 1, true, _s)
GH_GEMM(gh_pf_gemm_q4_m64_n64, Q4W, 64, 64, 1, true, _s)
GH_GEMM(gh_pf_gemm_q8_m64_n64, Q8W, 64, 64, 1, true, _s)
GH_GEMM(gh_pf_gemm_q4_m128_n128, Q4W, 128, 128, 1, true, _s)
GH_GEMM(gh_pf_gemm_q8_m128_n128, Q8W, 128, 128, 1, true, _s)
GH_GEMM_PAIR(gh_pf_gateup_q4_m64_n64, Q4W, 64, 64, 1, true, _s)
GH_GEMM_PAIR(gh_pf_gateup_q4_m128_n64, Q4W, 128, 64, 1, true, _s)  // 65-128 tokens
GH_GEMM_PAIR(gh_pf_gateup_q8_m64_n64, Q8W, 64, 64, 1, true, _s)

// 8-wave forms of the 128-row tiles (names end in _w8)
#define GH_GEMM_W8_FMT(FMT, F)                                                  \
  GH_GEMM_W8(gh_pf_gemm_##FMT##_m128_n128, F, 128, 128, 1, false, _w8)          \
  GH_GEMM_W8(gh_pf_gemm_##FMT##_m128_n64, F, 128, 64, 1, false, _w8)            \
  GH_GEMM_W8(gh_pf_gemm_##FMT##_m128_n128, F, 128, 128, 1, true, _s_w8)         \
  GH_GEMM_PAIR_W8(gh_pf_gateup_##FMT##_m128_n64, F, 128, 64, 1, false, _w8)
GH_GEMM_W8_FMT(q4, Q4W)
GH_GEMM_W8_FMT(q8, Q8W)
GH_GEMM_W8_FMT(bf16, Bf16W)
GH_GEMM_PAIR_W8(gh_pf_gateup_q4_m128_n64, Q4W, 128, 64, 1, true, _s_w8)

// The row scale of the GEMM's A operand for a row whose largest |x| is m:
// s = 2^(e - 14) with 2^(e-1) <= m < 2^e (1 for m = 0), so every |x| / s
// < 2^14 fits fp16; returns s and sets *inv = 1 / s (both exact).
__device__ __forceinline__ float row_scale(float m, float* inv) {
  int e = 0;
  if (m > 0.f) frexpf(m, &e);
  const int sh = m > 0.f ? e - 14 : 0;
  *inv = ldexpf(1.f, -sh);
  return ldexpf(1.f, sh);
}

// The MFMA A operand of one f32 row (K <= PF_HALVES_K): hi = fp16(a / s),
// lo = fp16(a / s - hi) with s = row_scale(max|a|), in the ax layout
// (pf_ax_pos).  One workgroup per row; rs[t] = s.
#define PF_HALVES_NT 1024
#define PF_HALVES_G 2  // 8-element groups per thread
#define PF_HALVES_K (8 * PF_HALVES_NT * PF_HALVES_G)

// Round-to-nearest-even bf16 bits of a finite float.
__device__ __forceinline__ uint32_t pf_bf16_bits(float f) {
  const uint32_t b = __float_as_uint(f);
  return (b + 0x7FFFu + ((b >> 16) & 1u)) >> 16;
}

// hi = fp16(x), lo = fp16(x - hi) of one 8-element group, stored in the ax
// layout at dst (16-byte aligned): the group's hi halves, and 32 halves on its
// lo halves, each as one 16-byte store.  fmt 0: fp16 in K order; 1: fp16 in
// the Q4 unpacking's K order; 2: bf16 halves (hi = bf16(x), lo = bf16(x - hi),
// about 16 significant bits) in K order, for the bf16 weights' MFMA.
__device__ __forceinline__ void pf_store_group(const float (&x)[8], uint32_t fmt, _Float16* dst) {
  half8 hi, lo;
  if (fmt == 2u) {
    uint32_t hw[4], lw[4];
#pragma unroll
    for (int k = 0; k < 8; k += 2) {
      const uint32_t h0 = pf_bf16_bits(x[k]), h1 = pf_bf16_bits(x[k + 1]);
      const uint32_t l0 = pf_bf16_bits(x[k] - __uint_as_float(h0 << 16));
      const uint32_t l1 = pf_bf16_bits(x[k + 1] - __uint_as_float(h1 << 16));
      hw[k / 2] = h0 | (h1 << 16);
      lw[k / 2] = l0 | (l1 << 16);
    }
    *reinterpret_cast<u32x4*>(dst) = u32x4{hw[0], hw[1], hw[2], hw[3]};
    *reinterpret_cast<u32x4*>(dst + 32) = u32x4{lw[0], lw[1], lw[2], lw[3]};
    return;
  }
#pragma unroll
  for (int k = 0; k < 8; k++) {
    const int p = fmt == 1u ? ((k & 3) << 1) | (k >> 2) : k;
    const _Float16 h = (_Float16)x[k];
    hi[p] = h;
    lo[p] = (_Float16)(x[k] - (float)h);
  }
  *reinterpret_cast<half8*>(dst) = hi;
  *reinterpret_cast<half8*>(dst + 32) = lo;
}

extern "C" __global__ __launch_bounds__(PF_HALVES_NT) void gh_pf_halves_k(
    const float* __restrict__ A, _Float16* __restrict__ Ax,
    float* __restrict__ rs, uint32_t K, uint32_t perm) {
  __shared__ float red[PF_HALVES_NT / 64];
  const uint32_t t = blockIdx.x, tid = threadIdx.x, n8 = K / 8;
  const float4* a = reinterpret_cast<const float4*>(A + (size_t)t * K);
  float4 v[PF_HALVES_G][2];
  float m = 0.f;
#pragma unroll
  for (int u = 0; u < PF_HALVES_G; u++) {
    const uint32_t g = tid + u * PF_HALVES_NT, gc = g < n8 ? g : n8 - 1;
    v[u][0] = a[2 * gc];
    v[u][1] = a[2 * gc + 1];
#pragma unroll
    for (int h = 0; h < 2; h++)
      if (g < n8)
        m = fmaxf(m, fmaxf(fmaxf(fabsf(v[u][h].x), fabsf(v[u][h].y)), fmaxf(fabsf(v[u][h].z), fabsf(v[u][h].w))));
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  if ((tid & 63) == 0) red[tid >> 6] = m;
  __syncthreads();
  m = 0.f;
#pragma unroll
  for (int w = 0; w < PF_HALVES_NT / 64; w++) m = fmaxf(m, red[w]);
  float inv;
  const float sc = row_scale(m, &inv);
#pragma unroll
  for (int u = 0; u < PF_HALVES_G; u++) {
    const uint32_t g = tid + u * PF_HALVES_NT;
    if (g < n8) {
      const float x[8] = {v[u][0].x * inv, v[u][0].y * inv, v[u][0].z * inv, v[u][0].w * inv,
                          v[u][1].x * inv, v[u][1].y * inv, v[u][1].z * inv, v[u][1].w * inv};
      pf_store_group(x, perm, Ax + (size_t)t * 2 * K + pf_ax_pos(8 * g, false));
    }
  }
  if (tid == 0) rs[t] = sc;
}

// C[T][N] from the Z partial planes of a split-K GEMM, added in z order (so
// the result does not depend on scheduling): the plain sum (nmat 1) or
// gelu_tanh(sum of gate planes) * (sum of up planes) (nmat 2).
extern "C" __global__ __launch_bounds__(PF_NT) void gh_pf_splitk_k(const float* __restrict__ P,
                                                                  float* __restrict__ C,
                                                                  uint32_t T, uint32_t N,
                                                                  uint32_t nz, uint32_t nmat) {
  const size_t tn = (size_t)T * N;
  for (size_t i = (size_t)blockIdx.x * PF_NT + threadIdx.x; i < tn; i += (size_t)gridDim.x * PF_NT) {
    float g = 0.f, u = 0.f;
#pragma unroll 4
    for (uint32_t z = 0; z < nz; z++) {
      g += P[(size_t)z * nmat * tn + i];
      if (nmat == 2) u += P[((size_t)z * 2 + 1) * tn + i];
    }
    C[i] = nmat == 2 ? gelu_tanh(g) * u : g;
  }
}

// ---------------------------------------------------------------------------
// Short batches (at most 48 tokens): the weight-streaming GEMM.
//
// With a few tokens the tile GEMM above spends each K step on one barrier
// and one load round trip for a tile that is mostly padding, and reads its
// weights at 0.8-1.5 TB/s.  Here every wavefront streams its own weight rows,
// one register set of 16 rows x SB quant blocks in flight while the previous
// set feeds the matrix cores, and the tokens take the MFMA's other
// dimension: v_mfma_f32_16x16x32_f16 (or _bf16) with A = 16 tokens x 32 K
// (the activation halves, as the tile GEMM reads them) and B = 32 K x 16
// weight rows (one quant block of each row, exact integers), so one MFMA
// pair (hi, lo) covers one block of 16 rows and the rows' block scales apply
// to its results.  With TG groups of 16 tokens each group is its own MFMA
// pair on the same weight fragment.
//
// MFMA 16x16x32 operand layout: lane l holds A[l % 16][8 (l / 16) + e] and
// B[8 (l / 16) + e][l % 16], e = 0..7; result register r of lane l is
// D[4 (l / 16) + r][l % 16].  So lane group g = l / 16 takes elements
// 8g .. 8g + 7 of each block (Q4_0: word 1 + g, unpacked in the order the ax
// layout keeps them), and D holds tokens 4g + r of weight row l % 16: one
// block scale per lane.
//
// A set is loaded as the decode streams load: lane l takes PB consecutive
// blocks (16-byte loads) of row l % 16, piece l / 16, so each row's SB
// blocks arrive as one contiguous run.  (Loading each lane's MFMA fragment
// directly, one scale and one word per block from 16 rows 2400 bytes apart,
// reads at about 1.3 TB/s against 5.4-6.0 TB/s for these runs.)  The wave
// then writes the set to its
// own LDS rows and reads the fragments back; LDS keeps a wave's operations in
// order, so no barrier is involved.  Bank conflicts: each 16-lane phase of a
// set write covers 16 rows (one piece), and the row strides (84, 148 and 132
// dwords) are 4 x odd modulo the 64 banks, so those writes and the fragment
// reads (16 rows, 4 lane groups) land on distinct banks.  (With lane l on
// row l / 4 a phase held 4 rows x 4 pieces at bank 20 (row + piece); the
// gate+up's conflict cycles fell by a quarter with this mapping, its time
// did not move.)
//
// Workgroup (x, z) of NW waves owns row groups [NW RGW x, NW RGW (x + 1)) of
// 16 rows and K blocks [z KR, z KR + KR) (KR and K / 32 multiples of 4): it
// stages that slice of the T <= 16 TG activation rows in LDS once, and wave
// w then streams row groups w, w + NW, ... with no further barrier.
// gridDim.z > 1: plane z of [Z][NMAT][T][N] takes the raw sums times the row
// scale, as the tile GEMM's split form writes them; gridDim.z = 1: C takes
// the epilogue.
//
// AF (the o and down inputs, and the kernel-level f32 entry points): A comes
// as f32 rows, and the staging splits each token's slice itself, with a
// power-of-two scale of its own (row_scale of the slice's largest |a|, 16
// threads per token); plane z then carries that scale instead of the row's.
// This saves the separate split launch (gh_pf_halves_k).
// ---------------------------------------------------------------------------
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct SQ4 {  // Q4_0 (src/quant.zig:55-90): {f32 d, 4 words of nibbles}
  static constexpr uint32_t kBlockBytes = 20;
  static constexpr int kPB = 4;  // blocks per lane and set (80 bytes)
  static constexpr bool kBf16 = false;
  static constexpr uint32_t kFmt = 1;  // pf_store_group format of the A halves
  // the fragment of block kb from an LDS row: scale d, word 1 + g as the
  // fp16 pairs (n_j - 8, n_{j+4} - 8), j = 0..3, as Q4W::ints unpacks it
  __device__ static half8 frag(const uint8_t* row, uint32_t kb, uint32_t g, float* d) {
    const uint32_t* p = reinterpret_cast<const uint32_t*>(row + kb * kBlockBytes);
    *d = __uint_as_float(p[0]);
    const uint32_t w = p[1 + g];
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 bias = {(_Float16)-1032.0f, (_Float16)-1032.0f};
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t pr = ((w >> (4 * j)) & 0x000F000Fu) | 0x64006400u;
      o[j] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, pr) + bias);
    }
    return __builtin_bit_cast(half8, o);
  }
};

struct SQ8 {  // Q8_0 (src/quant.zig:20-51): {f32 d, 8 words of int8}
  static constexpr uint32_t kBlockBytes = 36;
  static constexpr int kPB = 4;  // 144 bytes
  static constexpr bool kBf16 = false;
  static constexpr uint32_t kFmt = 0;
  __device__ static half8 frag(const uint8_t* row, uint32_t kb, uint32_t g, float* d) {
    const uint32_t* p = reinterpret_cast<const uint32_t*>(row + kb * kBlockBytes);
    *d = __uint_as_float(p[0]);
    const uint32_t w[2] = {p[1 + 2 * g], p[2 + 2 * g]};
    half8 o;  // q as fp16, in K order
#pragma unroll
    for (int k = 0; k < 2; k++)
#pragma unroll
      for (int n = 0; n < 4; n++) o[4 * k + n] = (_Float16)(int)(int8_t)((w[k] >> (8 * n)) & 0xFFu);
    return o;
  }
};

struct SBf16 {  // bf16 rows: 32-element segments of 64 bytes, no scale
  static constexpr uint32_t kBlockBytes = 64;
  static constexpr int kPB = 2;  // 128 bytes
  static constexpr bool kBf16 = true;
  static constexpr uint32_t kFmt = 2;
  __device__ static half8 frag(const uint8_t* row, uint32_t kb, uint32_t g, float* d) {
    *d = 1.f;
    return *reinterpret_cast<const half8*>(row + kb * kBlockBytes + 16 * g);
  }
};

template <class F>
struct SSet {
  static constexpr int SB = 4 * F::kPB;                          // blocks per set
  static constexpr int NV = F::kPB * (int)F::kBlockBytes / 16;   // 16-byte loads per lane
  static constexpr uint32_t RS = SB * F::kBlockBytes + 16;       // LDS row stride (bytes)
  static constexpr uint32_t kWaveBytes = 16 * RS;                // one matrix's set
};

#define PF_SLICE_MAX 32  // quant blocks per K slice (the AF staging holds 8 groups per thread)

// NW waves per workgroup (NW * 64 threads), TG groups of 16 tokens (T <= 16 TG).
template <class F, int NMAT, bool AF, int NW, int TG>
__device__ __forceinline__ void stream_gemm(const _Float16* __restrict__ Ax,
                                            const float* __restrict__ rs,
                                            const uint8_t* __restrict__ W0,
                                            const uint8_t* __restrict__ W1,
                                            float* __restrict__ C, uint32_t T, uint32_t N,
                                            uint32_t K, uint32_t KR, uint32_t RGW) {
  using S = SSet<F>;
  constexpr int SB = S::SB, NV = S::NV, PB = F::kPB;
  constexpr uint32_t NT = 64 * NW;
  extern __shared__ __attribute__((aligned(16))) uint8_t pf_slice[];
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t g = lane >> 4, li = lane & 15;
  const uint32_t nb = K / 32, z = blockIdx.z;
  const uint32_t b0 = z * KR, nk = min(nb - b0, KR);  // the host keeps b0 < nb, 4 | nk
  const uint32_t stride = KR * 128 + 16;              // bytes per staged token row
  const size_t row_bytes = (size_t)nb * F::kBlockBytes;
  const uint32_t kchunks = (nk + SB - 1) / SB;  // sets per row group
  const uint32_t nchunks = RGW * kchunks;
  const uint32_t rg0 = blockIdx.x * NW * RGW + wave;  // row group j of this wave: rg0 + NW j
  // this wave's set rows, after the T staged token rows
  uint8_t* wl = pf_slice + T * stride + wave * NMAT * S::kWaveBytes;
  // token rows of this lane's A fragments (one per group of 16 tokens):
  // tokens past T read token T - 1 (their D rows are never stored)
  const uint8_t* al_row[TG];
#pragma unroll
  for (int h = 0; h < TG; h++) al_row[h] = pf_slice + min(16 * h + li, T - 1) * stride + 16 * g;

  // Set c: row group j = c / kchunks, blocks kb0 .. kb0 + SB - 1 of the
  // slice.  Lane l loads blocks kb0 + PB (l / 16) .. + PB - 1 of row l % 16
  // (a piece that starts past the slice loads its last piece instead; those
  // blocks are skipped).
  u32x4 ra[NMAT][NV], rb[NMAT][NV];
  auto load = [&](uint32_t c, u32x4(&r)[NMAT][NV]) {
    const uint32_t j = c / kchunks, kb0 = (c % kchunks) * SB;
    uint32_t row = (rg0 + NW * j) * 16 + li;
    row = row < N ? row : N - 1;
    const uint32_t kb = min(kb0 + PB * g, nk - PB);
    const size_t off = (size_t)row * row_bytes + (size_t)(b0 + kb) * F::kBlockBytes;
#pragma unroll
    for (int i = 0; i < NV; i++) r[0][i] = *(gvec_ptr)(W0 + off + 16 * i);
    if constexpr (NMAT == 2) {
#pragma unroll
      for (int i = 0; i < NV; i++) r[1][i] = *(gvec_ptr)(W1 + off + 16 * i);
    }
  };

  // the first set is in flight while the slice is staged
  load(0, ra);
  __shared__ float slice_scale[16 * TG];  // AF: each token's scale for this slice
  if constexpr (AF) {
    // 16 threads per token, NT / 16 tokens per pass; thread `sub` takes
    // 8-element groups sub, sub + 16, ... of the slice (nk / 4 of them: nk
    // is a multiple of 4)
    constexpr uint32_t TPP = NT / 16, PASSES = (16 * TG + TPP - 1) / TPP;
    const float* A = reinterpret_cast<const float*>(Ax);
#pragma unroll 1
    for (uint32_t pass = 0; pass < PASSES; pass++) {
      const uint32_t t = (tid >> 4) + pass * TPP, sub = tid & 15, per = nk / 4;
      const bool on = t < T;
      const float* src = A + (size_t)min(t, T - 1) * K + (size_t)b0 * 32;
      float xv[PF_SLICE_MAX / 4][8];
      float m = 0.f;
#pragma unroll
      for (int i = 0; i < PF_SLICE_MAX / 4; i++) {
        if ((uint32_t)i < per) {
          const float4 a = *reinterpret_cast<const float4*>(src + 8 * (sub + 16 * i));
          const float4 b = *reinterpret_cast<const float4*>(src + 8 * (sub + 16 * i) + 4);
          xv[i][0] = a.x; xv[i][1] = a.y; xv[i][2] = a.z; xv[i][3] = a.w;
          xv[i][4] = b.x; xv[i][5] = b.y; xv[i][6] = b.z; xv[i][7] = b.w;
#pragma unroll
          for (int k = 0; k < 8; k++) m = fmaxf(m, fabsf(xv[i][k]));
        }
      }
#pragma unroll
      for (int off = 8; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
      float inv;
      const float sc = row_scale(m, &inv);
      if (on) {
#pragma unroll
        for (int i = 0; i < PF_SLICE_MAX / 4; i++) {
          if ((uint32_t)i < per) {
            const uint32_t gi = sub + 16 * i;  // group gi: block gi / 4, part gi % 4
            float y[8];
#pragma unroll
            for (int k = 0; k < 8; k++) y[k] = xv[i][k] * inv;
            pf_store_group(y, F::kFmt,
                           reinterpret_cast<_Float16*>(pf_slice + t * stride + (gi >> 2) * 128 +
                                                       (gi & 3) * 16));
          }
        }
        if (sub == 0) slice_scale[t] = sc;
      }
    }
  } else {
    const uint32_t per_row = nk * 8;  // 16-byte chunks of one token's slice
    const uint32_t total = T * per_row;
#pragma unroll 4
    for (uint32_t c = tid; c < total; c += NT) {
      const uint32_t t = c / per_row, q = c % per_row;
      const u32x4 v = *reinterpret_cast<const u32x4*>(Ax + (size_t)t * 2 * K + (size_t)b0 * 64 + 8 * q);
      *reinterpret_cast<u32x4*>(pf_slice + t * stride + 16 * q) = v;
    }
  }
  __syncthreads();

  f32x4 acc[NMAT][TG];
#pragma unroll
  for (int q = 0; q < NMAT; q++)
#pragma unroll
    for (int h = 0; h < TG; h++) acc[q][h] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto epilogue = [&](uint32_t j) {
    const uint32_t n = (rg0 + NW * j) * 16 + li;
    if (n >= N) return;
#pragma unroll
    for (int h = 0; h < TG; h++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const uint32_t t = 16 * h + 4 * g + r;
        if (t >= T) continue;
        const float sr = AF ? slice_scale[t] : rs[t];
        if (gridDim.z > 1) {
#pragma unroll
          for (int q = 0; q < NMAT; q++)
            C[((size_t)(z * NMAT + q) * T + t) * N + n] = acc[q][h][r] * sr;
        } else if constexpr (NMAT == 1) {
          C[(size_t)t * N + n] = acc[0][h][r] * sr;
        } else {
          C[(size_t)t * N + n] = gelu_tanh(acc[0][h][r] * sr) * (acc[1][h][r] * sr);
        }
      }
  };

  auto compute = [&](uint32_t c, const u32x4(&r)[NMAT][NV]) {
    const uint32_t j = c / kchunks, kb0 = (c % kchunks) * SB;
    // the set into this wave's LDS rows: lane l's piece l / 16 of row l % 16
#pragma unroll
    for (int q = 0; q < NMAT; q++)
#pragma unroll
      for (int i = 0; i < NV; i++)
        *reinterpret_cast<u32x4*>(wl + q * S::kWaveBytes + li * S::RS + g * PB * F::kBlockBytes +
                                  16 * i) = r[q][i];
#pragma unroll
    for (int u = 0; u < SB; u++) {
      const uint32_t kb = kb0 + u;
      if (kb < nk) {  // uniform over the wave
        half8 ah[TG], al[TG];
#pragma unroll
        for (int h = 0; h < TG; h++) {
          ah[h] = *reinterpret_cast<const half8*>(al_row[h] + kb * 128);
          al[h] = *reinterpret_cast<const half8*>(al_row[h] + kb * 128 + 64);
        }
#pragma unroll
        for (int q = 0; q < NMAT; q++) {
          float d;
          const half8 b = F::frag(wl + q * S::kWaveBytes + li * S::RS, (uint32_t)u, g, &d);
#pragma unroll
          for (int h = 0; h < TG; h++) {
            if constexpr (F::kBf16) {
              f32x4 t = acc[q][h];
              t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ah[h]),
                                                          __builtin_bit_cast(bf16x8, b), t, 0, 0, 0);
              t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, al[h]),
                                                          __builtin_bit_cast(bf16x8, b), t, 0, 0, 0);
              acc[q][h] = t;
            } else {
              f32x4 blk = {0.f, 0.f, 0.f, 0.f};
              blk = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[h], b, blk, 0, 0, 0);
              blk = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[h], b, blk, 0, 0, 0);
#pragma unroll
              for (int e = 0; e < 4; e++) acc[q][h][e] += d * blk[e];
            }
          }
        }
      }
    }
    if (c % kchunks == kchunks - 1) {  // the row group's last set
      epilogue(j);
#pragma unroll
      for (int q = 0; q < NMAT; q++)
#pragma unroll
        for (int h = 0; h < TG; h++) acc[q][h] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };

  for (uint32_t c = 0; c < nchunks; c += 2) {
    if (c + 1 < nchunks) load(c + 1, rb);
    compute(c, ra);
    if (c + 1 < nchunks) {
      if (c + 2 < nchunks) load(c + 2, ra);
      compute(c + 1, rb);
    }
  }
}

// 4-wave workgroups for up to 16 tokens; 8-wave workgroups for 17-32 tokens
// (two token groups per wave sharing each weight fragment; the 32 staged
// token rows serve 8 waves' row groups, which keeps 16-block slices in LDS)
// and for 33-48 tokens (three groups per wave, narrower slices where LDS
// needs them).
#define GH_SGEMM(NAME, F, NMAT, AF)                                                          \
  extern "C" __global__ __launch_bounds__(256) void NAME##_k(                               \
      const _Float16* Ax, const float* rs, const uint8_t* W0, const uint8_t* W1, float* C,  \
      uint32_t T, uint32_t N, uint32_t K, uint32_t KR, uint32_t RGW) {                      \
    stream_gemm<F, NMAT, AF, 4, 1>(Ax, rs, W0, W1, C, T, N, K, KR, RGW);                    \
  }                                                                                         \
  extern "C" __global__ __launch_bounds__(512) void NAME##_t2_k(                            \
      const _Float16* Ax, const float* rs, const uint8_t* W0, const uint8_t* W1, float* C,  \
      uint32_t T, uint32_t N, uint32_t K, uint32_t KR, uint32_t RGW) {                      \
    stream_gemm<F, NMAT, AF, 8, 2>(Ax, rs, W0, W1, C, T, N, K, KR, RGW);                    \
  }                                                                                         \
  extern "C" __global__ __launch_bounds__(512) void NAME##_t3_k(                            \
      const _Float16* Ax, const float* rs, const uint8_t* W0, const uint8_t* W1, float* C,  \
      uint32_t T, uint32_t N, uint32_t K, uint32_t KR, uint32_t RGW) {                      \
    stream_gemm<F, NMAT, AF, 8, 3>(Ax, rs, W0, W1, C, T, N, K, KR, RGW);                    \
  }
GH_SGEMM(gh_pf_sgemm_q4, SQ4, 1, false)
GH_SGEMM(gh_pf_sgateup_q4, SQ4, 2, false)
GH_SGEMM(gh_pf_sgemm_q8, SQ8, 1, false)
GH_SGEMM(gh_pf_sgateup_q8, SQ8, 2, false)
GH_SGEMM(gh_pf_sgemm_bf16, SBf16, 1, false)
GH_SGEMM(gh_pf_sgateup_bf16, SBf16, 2, false)
GH_SGEMM(gh_pf_sgemm_q4_f, SQ4, 1, true)
GH_SGEMM(gh_pf_sgateup_q4_f, SQ4, 2, true)
GH_SGEMM(gh_pf_sgemm_q8_f, SQ8, 1, true)
GH_SGEMM(gh_pf_sgateup_q8_f, SQ8, 2, true)
GH_SGEMM(gh_pf_sgemm_bf16_f, SBf16, 1, true)
GH_SGEMM(gh_pf_sgateup_bf16_f, SBf16, 2, true)

// ---------------------------------------------------------------------------
// Row-wise x prologue for T tokens (the batched form of the decode GEMVs'
// fused norms, src/gpu/model_dispatch.zig:21,32-34,39-41):
//   mode 1: xn = RMSNorm(x) * w
//   mode 2: x <- (x + RMSNorm(r) * wr) * s  (r as given when wr is null),
//           stored back as the residual stream; xn = RMSNorm(x) * w
// In mode 2, r may arrive as rz unsummed K-split planes of a GEMM ([rz][T][H]);
// they are added in plane order, as gh_pf_splitk_k adds them.
// One workgroup per token row.
// ---------------------------------------------------------------------------
template <int NT>
__device__ __forceinline__ float block_sum(float v, float* red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < NT / 64; w++) t += red[w];
  __syncthreads();
  return t;
}

#define PF_NORM_NT 1024
#define PF_ROW_MAX 8  // elements per thread (one 8-element group): hidden <= 8192

// Every load (x, r, wr, w) is issued before any is used, with clamped
// indices and stand-in pointers for the operands a mode does not read, so
// the row costs one global round trip rather than one per operand.  The
// normed row goes out as the GEMM's A operand: fp16 hi/lo halves in the ax
// layout (pf_ax_pos, [T][2H]) and the row scale rs[t], as gh_pf_halves_k
// makes them.
template <int NT>
__device__ __forceinline__ float block_max(float v, float* red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < NT / 64; w++) t = fmaxf(t, red[w]);
  __syncthreads();
  return t;
}

template <int NT>
__device__ __forceinline__ void pf_norm_row(float* X, const float* R, const float* wr,
                                            const float* w, _Float16* Xa, float* rs, uint32_t H,
                                            float s, float eps, uint32_t mode, uint32_t perm,
                                            uint32_t rz) {
  __shared__ float red[NT / 64];
  // thread t owns the 8-element group t of the row (H <= 8 * NT)
  const uint32_t t = blockIdx.x, tid = threadIdx.x, n8 = H / 8;
  const bool add = mode == 2, has_wr = wr != nullptr, act = tid < n8;
  const uint32_t e0 = 8 * (act ? tid : n8 - 1);
  float* x = X + (size_t)t * H;
  const float* r = add ? R + (size_t)t * H : x;
  const float* wrp = has_wr ? wr : w;
  float v[8], rv[8], wv[8], wrv[8];
  auto load8 = [&](const float* p, float (&o)[8]) {
    const float4 a = *reinterpret_cast<const float4*>(p + e0);
    const float4 b = *reinterpret_cast<const float4*>(p + e0 + 4);
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
    o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
  };
  load8(x, v);
  load8(r, rv);
  load8(w, wv);
  load8(wrp, wrv);
  if (add) {
    // planes 1 .. rz - 1, 8 in flight at a time (clamped indices), added in
    // plane order
    const size_t plane = (size_t)gridDim.x * H;
    for (uint32_t z = 1; z < rz; z += 8) {
      float pv[8][8];
#pragma unroll
      for (int u = 0; u < 8; u++) load8(r + (size_t)min(z + u, rz - 1) * plane, pv[u]);
#pragma unroll
      for (int u = 0; u < 8; u++)
        if (z + u < rz) {  // uniform
#pragma unroll
          for (int k = 0; k < 8; k++) rv[k] += pv[u][k];
        }
    }
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < 8; k++) ss += rv[k] * rv[k];
    ss = act ? ss : 0.f;
    const float inv_r = has_wr ? 1.0f / sqrtf(block_sum<NT>(ss, red) / (float)H + eps) : 1.0f;
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const float rr = has_wr ? rv[k] * inv_r * wrv[k] : rv[k];
      v[k] = (v[k] + rr) * s;
    }
    if (act) {
      *reinterpret_cast<float4*>(x + e0) = make_float4(v[0], v[1], v[2], v[3]);
      *reinterpret_cast<float4*>(x + e0 + 4) = make_float4(v[4], v[5], v[6], v[7]);
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < 8; k++) ss += v[k] * v[k];
  ss = act ? ss : 0.f;
  const float inv = 1.0f / sqrtf(block_sum<NT>(ss, red) / (float)H + eps);
  float m = 0.f;
#pragma unroll
  for (int k = 0; k < 8; k++) {
    v[k] = v[k] * inv * wv[k];
    m = fmaxf(m, fabsf(v[k]));
  }
  float sinv;
  const float sc = row_scale(block_max<NT>(act ? m : 0.f, red), &sinv);
  if (act) {
    float y[8];
#pragma unroll
    for (int k = 0; k < 8; k++) y[k] = v[k] * sinv;
    pf_store_group(y, perm, Xa + (size_t)t * 2 * H + pf_ax_pos(e0, false));
  }
  if (tid == 0) rs[t] = sc;
}

// 1024 threads for rows of up to 8192, 512 for rows of up to 4096 (the 12B
// hidden 3840: 480 groups, so the 1024-thread form idles more than half its
// threads and holds half as many rows per CU)
extern "C" __global__ __launch_bounds__(PF_NORM_NT) void gh_pf_norm_k(
    float* X, const float* R, const float* wr, const float* w, _Float16* Xa,
    float* rs, uint32_t H, float s, float eps, uint32_t mode, uint32_t perm, uint32_t rz) {
  pf_norm_row<PF_NORM_NT>(X, R, wr, w, Xa, rs, H, s, eps, mode, perm, rz);
}
extern "C" __global__ __launch_bounds__(512) void gh_pf_norm_512_k(
    float* X, const float* R, const float* wr, const float* w, _Float16* Xa,
    float* rs, uint32_t H, float s, float eps, uint32_t mode, uint32_t perm, uint32_t rz) {
  pf_norm_row<512>(X, R, wr, w, Xa, rs, H, s, eps, mode, perm, rz);
}
