// rope.h -- the RoPE angle of one rotated pair, shared by every kernel that
// rotates (attention prologues) or tabulates the angles (the per-token step
// kernel), so a tabulated angle has the bits the kernel would compute.
// applyRopePartial (src/kernels.zig:132-150): pair (i, i + rot/2), i < rot/2,
// freq = 1 / theta^(2i / rot), angle = clock * freq.
#pragma once
#include <stdint.h>

#define ROPE_TAB_HALF 256  // cos[0..256) then sin[0..256) per table (rot <= 512)

__device__ __forceinline__ void gh_rope_angle(uint32_t i, uint32_t rot, float theta,
                                              uint32_t clock, float* c, float* s) {
  const float freq = 1.0f / powf(theta, (2.0f * (float)i) / (float)rot);
  const float ang = (float)clock * freq;
  *c = cosf(ang);
  *s = sinf(ang);
}
