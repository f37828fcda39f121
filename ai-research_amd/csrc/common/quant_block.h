// quant_block.h -- Q4_0 / Q8_0 block quantizers shared by the host library and
// the gfx950 quantize kernel.  Bit-exact restatement of src/quant.zig:20-90:
//   amax = max |v| over the 32 bf16 values (widened to f32)
//   d    = amax / 7 (Q4) or amax / 127 (Q8), stored as the block's first word
//   id   = amax > 0 ? 7 / amax : 0   (a separate division, not 1 / d)
//   q    = clamp(round_half_away(v * id), -8, 7) + 8   (Q4)
//          clamp(round_half_away(v * id), -128, 127)   (Q8)
//   Q4: element j -> word 1 + j/8 at bit 4*(j%8);  Q8: byte j of words 1..8.
// The f32 quotients are formed as double quotients rounded once to f32, which
// equals the correctly rounded f32 quotient (53 >= 2*24 + 2) on both sides.
#pragma once
#include <stdint.h>

#include "synth.h"  // GH_HD

GH_HD float gh_bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}

GH_HD uint32_t gh_f32_bits(float f) {
  uint32_t u;
  __builtin_memcpy(&u, &f, 4);
  return u;
}

GH_HD int32_t gh_round_clamp(float p, int32_t lo, int32_t hi) {
  float r = __builtin_roundf(p);  // half away from zero, exact
  if (!(r >= (float)lo)) r = (float)lo;
  if (r > (float)hi) r = (float)hi;
  return (int32_t)r;
}

GH_HD float gh_block_amax(const float* v) {
  float amax = 0.0f;
  for (int i = 0; i < 32; i++) {
    float a = __builtin_fabsf(v[i]);
    if (a > amax) amax = a;
  }
  return amax;
}

GH_HD void gh_quantize_block_q4(const uint16_t* src, uint32_t* dst) {
  GH_NOCONTRACT
  float v[32];
  for (int i = 0; i < 32; i++) v[i] = gh_bf16_to_f32(src[i]);
  float amax = gh_block_amax(v);
  float d = (float)((double)amax / 7.0);
  float id = amax > 0.0f ? (float)(7.0 / (double)amax) : 0.0f;
  dst[0] = gh_f32_bits(d);
  for (int w = 0; w < 4; w++) {
    uint32_t word = 0;
    for (int k = 0; k < 8; k++) {
      uint32_t nib = (uint32_t)(gh_round_clamp(v[w * 8 + k] * id, -8, 7) + 8);
      word |= nib << (4 * k);
    }
    dst[1 + w] = word;
  }
}

GH_HD void gh_quantize_block_q8(const uint16_t* src, uint32_t* dst) {
  GH_NOCONTRACT
  float v[32];
  for (int i = 0; i < 32; i++) v[i] = gh_bf16_to_f32(src[i]);
  float amax = gh_block_amax(v);
  float d = (float)((double)amax / 127.0);
  float id = amax > 0.0f ? (float)(127.0 / (double)amax) : 0.0f;
  dst[0] = gh_f32_bits(d);
  for (int w = 0; w < 8; w++) {
    uint32_t word = 0;
    for (int k = 0; k < 4; k++) {
      uint32_t byte = (uint32_t)(uint8_t)(int8_t)gh_round_clamp(v[w * 4 + k] * id, -128, 127);
      word |= byte << (8 * k);
    }
    dst[1 + w] = word;
  }
}
