// util.hip -- device-side synthetic-data generator and the bit-exact block
// quantizer (src/quant.zig:20-90) for gfx950.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../common/quant_block.h"
#include "../common/synth.h"
#include "../common/rope.h"

// 8 consecutive elements per thread: one 32-byte (f32: 2 x 16 B) store run.
extern "C" __global__ __launch_bounds__(256) void gh_synth_normal_f32_k(
    float* dst, uint64_t n, uint64_t key, double mean, double stddev, uint64_t offset) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x * 8;
  for (uint64_t i = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8; i < n; i += stride) {
    if (i + 8 <= n) {
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; j++) v[j] = gh_normal_f32(key, offset + i + j, mean, stddev);
      float4* p = reinterpret_cast<float4*>(dst + i);
      if ((reinterpret_cast<uintptr_t>(p) & 15) == 0) {
        p[0] = make_float4(v[0], v[1], v[2], v[3]);
        p[1] = make_float4(v[4], v[5], v[6], v[7]);
      } else {
        for (int j = 0; j < 8; j++) dst[i + j] = v[j];
      }
    } else {
      for (uint64_t j = i; j < n; j++) dst[j] = gh_normal_f32(key, offset + j, mean, stddev);
    }
  }
}

extern "C" __global__ __launch_bounds__(256) void gh_synth_normal_bf16_k(
    uint16_t* dst, uint64_t n, uint64_t key, double mean, double stddev, uint64_t offset) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x * 8;
  for (uint64_t i = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8; i < n; i += stride) {
    if (i + 8 <= n && (reinterpret_cast<uintptr_t>(dst + i) & 15) == 0) {
      uint32_t w[4];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        uint32_t lo = gh_bf16_rne(gh_normal_f32(key, offset + i + 2 * j, mean, stddev));
        uint32_t hi = gh_bf16_rne(gh_normal_f32(key, offset + i + 2 * j + 1, mean, stddev));
        w[j] = lo | (hi << 16);
      }
      *reinterpret_cast<uint4*>(dst + i) = make_uint4(w[0], w[1], w[2], w[3]);
    } else {
      const uint64_t e = i + 8 < n ? i + 8 : n;
      for (uint64_t j = i; j < e; j++)
        dst[j] = gh_bf16_rne(gh_normal_f32(key, offset + j, mean, stddev));
    }
  }
}

// One thread per 32-element block.  src: bf16 [rows][cols], dst: blocks with
// row stride ceil(cols/32) blocks (quant.zig:164-171); cols % 32 == 0.
extern "C" __global__ __launch_bounds__(256) void gh_quantize_q4_k(
    uint32_t* dst, const uint16_t* src, uint64_t rows, uint32_t cols) {
  const uint32_t nb = cols >> 5;
  const uint64_t total = rows * nb;
  for (uint64_t b = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; b < total;
       b += (uint64_t)gridDim.x * blockDim.x) {
    uint16_t v[32];
    const uint4* p = reinterpret_cast<const uint4*>(src + b * 32);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      uint4 t = p[j];
      const uint32_t ww[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
      for (int k = 0; k < 4; k++) {
        v[8 * j + 2 * k] = (uint16_t)(ww[k] & 0xFFFFu);
        v[8 * j + 2 * k + 1] = (uint16_t)(ww[k] >> 16);
      }
    }
    uint32_t out[5];
    gh_quantize_block_q4(v, out);
    uint32_t* d = dst + b * 5;
#pragma unroll
    for (int j = 0; j < 5; j++) d[j] = out[j];
  }
}

extern "C" __global__ __launch_bounds__(256) void gh_quantize_q8_k(
    uint32_t* dst, const uint16_t* src, uint64_t rows, uint32_t cols) {
  const uint32_t nb = cols >> 5;
  const uint64_t total = rows * nb;
  for (uint64_t b = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; b < total;
       b += (uint64_t)gridDim.x * blockDim.x) {
    uint16_t v[32];
    const uint4* p = reinterpret_cast<const uint4*>(src + b * 32);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      uint4 t = p[j];
      const uint32_t ww[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
      for (int k = 0; k < 4; k++) {
        v[8 * j + 2 * k] = (uint16_t)(ww[k] & 0xFFFFu);
        v[8 * j + 2 * k + 1] = (uint16_t)(ww[k] >> 16);
      }
    }
    uint32_t out[9];
    gh_quantize_block_q8(v, out);
    uint32_t* d = dst + b * 9;
#pragma unroll
    for (int j = 0; j < 9; j++) d[j] = out[j];
  }
}

extern "C" __global__ __launch_bounds__(256) void gh_fill_u32_k(uint32_t* dst, uint32_t value,
                                                                uint64_t n) {
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (uint64_t)gridDim.x * blockDim.x)
    dst[i] = value;
}

extern "C" __global__ __launch_bounds__(256) void gh_copy_u32_k(uint32_t* dst, const uint32_t* src,
                                                                uint64_t n) {
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (uint64_t)gridDim.x * blockDim.x)
    dst[i] = src[i];
}

// HBM read-bandwidth probe: the buffer's n4 16-byte vectors are read once,
// U loads in flight per lane, and each workgroup writes the sum of what it
// read (so no load is dead).  CONTIG = 0: grid-stride over the whole buffer
// (every round of the grid reads one contiguous span); CONTIG = 1: workgroup
// b reads its own contiguous 1/grid share.  n4 is a multiple of 256 U * grid
// (checked by the host), so no bounds test sits in the loop.
template <int U, bool CONTIG>
__device__ __forceinline__ void read_probe(const float4* __restrict__ src, uint64_t n4,
                                           float* sums) {
  __shared__ float red[4];
  const uint64_t T = (uint64_t)gridDim.x * 256;
  const uint64_t per_wg = n4 / gridDim.x;
  const uint64_t start = CONTIG ? blockIdx.x * per_wg + threadIdx.x
                                : (uint64_t)blockIdx.x * 256 + threadIdx.x;
  const uint64_t end = CONTIG ? (blockIdx.x + 1) * per_wg : n4;
  const uint64_t step = CONTIG ? 256 : T;
  float acc = 0.f;
  for (uint64_t i = start; i < end; i += step * U) {
    float4 v[U];
#pragma unroll
    for (int u = 0; u < U; u++) v[u] = src[i + u * step];
#pragma unroll
    for (int u = 0; u < U; u++) acc += (v[u].x + v[u].y) + (v[u].z + v[u].w);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) sums[blockIdx.x] = (red[0] + red[1]) + (red[2] + red[3]);
}
#define GH_READ_PROBE(U, C)                                                                \
  extern "C" __global__ __launch_bounds__(256) void gh_read_probe_u##U##_c##C##_k(         \
      const float4* __restrict__ src, uint64_t n4, float* sums) {                          \
    read_probe<U, C>(src, n4, sums);                                                       \
  }
GH_READ_PROBE(1, 0) GH_READ_PROBE(2, 0) GH_READ_PROBE(4, 0) GH_READ_PROBE(8, 0)
GH_READ_PROBE(1, 1) GH_READ_PROBE(2, 1) GH_READ_PROBE(4, 1) GH_READ_PROBE(8, 1)

// The per-token step kernel at the head of every decode graph.
//
// RoPE tables: for each of the model's two layer types (rot_t, theta_t; rot 0
// = unused) it writes cos then sin of this clock's angles (gh_rope_angle, the
// attention prologue's own definition) to rope_tab[t], so the 48 attention
// launches of a token read angles instead of each recomputing powf/cosf/sinf.
//
// Ring bookkeeping: the layer-0 state of DynamicRingBuffer
// (src/ring_buffer.zig:56-136, as src/model/forward.zig:42-43 drives it).
// step = {clock, slot_idx, S, flags}.  flags bit 0 set: the kernel activates
// the clock's slot (activateSlot: clocks[slot] = clock, flag set), writes
// slot_idx, S and the active list (getActiveSlots), and sets flags bit 1
// when the list is 0 .. S-1.  Bit 0 clear: the host wrote slot_idx, S, the
// list and bit 1; the kernel only records the activation of slot_idx, so the
// device state follows host-driven steps too.  The list is the slot-order
// compaction of one predicate, because the three tiers are contiguous and
// each tier is listed in slot order:
//   anchors  s < min(clock + 1, A) and active
//   window   clock >= A, active, and its clock in [clock - W + 1 (or A), clock]
//   recall   active and its clock <= clock
// One workgroup of 1024 threads; slots are taken 1024 at a time, with a
// ballot prefix per wavefront and the wavefront counts scanned in LDS.
extern "C" __global__ __launch_bounds__(1024) void gh_ring_step_k(
    uint32_t* ring_clock, uint32_t* ring_flag, uint32_t* step, uint32_t* active, uint32_t A,
    uint32_t W, uint32_t R, float* rope_tab, uint32_t rot0, float theta0, uint32_t rot1,
    float theta1) {
  __shared__ uint32_t wave_n[16];
  __shared__ uint32_t base_n, last_on;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t flags = step[3];
  const uint32_t c = step[0];
  {  // RoPE tables: threads [0, 512) type 0, [512, 1024) type 1
    const uint32_t t = tid >> 9, i = tid & 511u;
    const uint32_t rot = t ? rot1 : rot0;
    if (i < rot / 2 && i < ROPE_TAB_HALF) {
      float cs, sn;
      gh_rope_angle(i, rot, t ? theta1 : theta0, c, &cs, &sn);
      rope_tab[t * 2 * ROPE_TAB_HALF + i] = cs;
      rope_tab[t * 2 * ROPE_TAB_HALF + ROPE_TAB_HALF + i] = sn;
    }
  }
  if ((flags & 1u) == 0u) {
    if (tid == 0 && step[1] < A + W + R) {
      ring_clock[step[1]] = c;
      ring_flag[step[1]] = 1u;
    }
    return;
  }
  const uint32_t slot = c < A ? c : A + (c - A) % W;
  const uint32_t total = A + W + R;
  const uint32_t alim = c + 1u < A ? c + 1u : A;
  const uint32_t minc = c >= W ? c - W + 1u : A;
  if (tid == 0) {
    base_n = 0;
    last_on = 0;
  }
  __syncthreads();
  for (uint32_t s0 = 0; s0 < total; s0 += 1024u) {
    const uint32_t s = s0 + tid;
    bool on = false;
    if (s < total) {
      const bool act = s == slot || ring_flag[s] != 0u;
      const uint32_t clk = s == slot ? c : ring_clock[s];
      if (s < A)
        on = s < alim && act;
      else if (s < A + W)
        on = c >= A && act && clk >= minc && clk <= c;
      else
        on = act && clk <= c;
    }
    const uint64_t mask = __ballot(on);
    if (lane == 0) wave_n[wave] = (uint32_t)__popcll(mask);
    if (on) atomicMax(&last_on, s);
    __syncthreads();
    uint32_t off = base_n;
    for (uint32_t w = 0; w < wave; w++) off += wave_n[w];
    if (on) active[off + (uint32_t)__popcll(mask & ((1ull << lane) - 1ull))] = s;
    __syncthreads();
    if (tid == 0) {
      uint32_t n = 0;
      for (uint32_t w = 0; w < 16u; w++) n += wave_n[w];
      base_n += n;
    }
    __syncthreads();
  }
  if (tid == 0) {
    ring_clock[slot] = c;
    ring_flag[slot] = 1u;
    step[1] = slot;
    step[2] = base_n;
    // the list is 0 .. S-1 exactly when its last (largest) slot is S - 1
    step[3] = 1u | (base_n > 0u && last_on == base_n - 1u ? 2u : 0u);
  }
}

// cos then sin of the RoPE angles at the clock step[0] for one (rot, theta):
// the table the fused decode attention reads (gh_rope_table).
extern "C" __global__ __launch_bounds__(256) void gh_rope_table_k(const uint32_t* step,
                                                                  uint32_t rot, float theta,
                                                                  float* tab) {
  const uint32_t c = step[0];
  for (uint32_t i = threadIdx.x; i < rot / 2 && i < ROPE_TAB_HALF; i += blockDim.x) {
    float cs, sn;
    gh_rope_angle(i, rot, theta, c, &cs, &sn);
    tab[i] = cs;
    tab[ROPE_TAB_HALF + i] = sn;
  }
}

// Moves the K/V rows a staged prefill batch wrote past the ring slots into
// their slots: for cache y (base + off[y] bytes, rows of words[y] u32) and
// pair x, row pairs[2x] := row pairs[2x + 1].  Grid (pairs, caches).  The
// destination rows are ring slots and the sources staging rows, disjoint.
extern "C" __global__ __launch_bounds__(256) void gh_rows_scatter_k(uint8_t* base,
                                                                    const uint64_t* off,
                                                                    const uint32_t* words,
                                                                    const uint32_t* pairs) {
  uint32_t* buf = reinterpret_cast<uint32_t*>(base + off[blockIdx.y]);
  const uint32_t w = words[blockIdx.y];
  const uint32_t dst = pairs[2 * blockIdx.x], src = pairs[2 * blockIdx.x + 1];
  for (uint32_t i = threadIdx.x; i < w; i += 256) buf[(size_t)dst * w + i] = buf[(size_t)src * w + i];
}
