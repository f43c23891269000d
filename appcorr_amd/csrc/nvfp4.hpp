// NVFP4 element arithmetic shared by the quantize / dequantize kernels (nvfp4.hip) and the producers
// that write the NVFP4 operand directly (the LayerNorm kernels, the SwiGLU epilogue). The format and
// the rounding choices are described at the top of nvfp4.hip.
#pragma once

#include "common.hpp"

namespace oudjat {

static constexpr float kE4m3Eps = 1.52587890625e-05f;  // 2^-16
static constexpr float kE4m3Max = 448.0f;
static constexpr float kE2m1Max = 6.0f;

// e4m3fn encoding of a finite value in [0, 448] with round-to-nearest-even.
__device__ __forceinline__ uint32_t e4m3_encode_pos(float v) {
  const uint32_t u = __float_as_uint(v);
  const int e = (int)((u >> 23) & 0xff) - 127;
  if (e < -6) {
    // Subnormal range: value = m * 2^-9, m in [0, 8] (m == 8 is the smallest normal, 0x08).
    return (uint32_t)__builtin_rintf(v * 512.0f);
  }
  const uint32_t r = u + 0x7ffffu + ((u >> 20) & 1u);  // RNE from 23 to 3 mantissa bits
  const int er = (int)((r >> 23) & 0xff) - 127 + 7;
  const uint32_t m = (r >> 20) & 7u;
  uint32_t code = ((uint32_t)er << 3) | m;
  return code > 0x7eu ? 0x7eu : code;  // saturate to 448 (0x7f is NaN)
}

__device__ __forceinline__ float e4m3_decode(uint32_t c) {
  const uint32_t e = (c >> 3) & 0xf, m = c & 7u;
  const float mag = e == 0 ? (float)m * 0.001953125f : __uint_as_float(((e + 120u) << 23) | (m << 20));
  return (c & 0x80u) ? -mag : mag;
}

// e2m1 code (sign in bit 3) of q with round-to-nearest-even and saturation.
__device__ __forceinline__ uint32_t e2m1_encode(float q) {
  const float a = fabsf(q);
  uint32_t c;
  if (a <= 0.25f) c = 0;
  else if (a < 0.75f) c = 1;
  else if (a <= 1.25f) c = 2;
  else if (a < 1.75f) c = 3;
  else if (a <= 2.5f) c = 4;
  else if (a < 3.5f) c = 5;
  else if (a <= 5.0f) c = 6;
  else c = 7;
  return c | ((__float_as_uint(q) >> 28) & 8u);
}

__device__ __forceinline__ float e2m1_decode(uint32_t c) {
  const uint32_t m = c & 7u;
  // 0, 0.5 (subnormal), then 2^(E-1) * (1 + M/2) for code = (E << 1) | M: 1, 1.5, 2, 3, 4, 6
  const float mag = m < 2 ? 0.5f * (float)m : (float)(1u << ((m >> 1) - 1)) * ((m & 1u) ? 1.5f : 1.0f);
  return (c & 8u) ? -mag : mag;
}

// Per-block scale of a 16-element block with maximum magnitude amax: the e4m3 code and the divisor
// ts * e4m3(code) of its elements.
__device__ __forceinline__ void nvfp4_block_scale(float amax, float ts, uint32_t& code, float& tot) {
  const float bs = amax / kE2m1Max;
  const float scaled = fminf(fmaxf(bs / ts, kE4m3Eps), kE4m3Max);
  code = e4m3_encode_pos(scaled);
  tot = ts * e4m3_decode(code);
}

// e2m1 codes of x_e / tot (IEEE quotient, e = 0..7) as one 32-bit word, element e in nibble e.
// Quotient: Markstein's correction step. With y = RN(1 / tot) (one IEEE division per block),
// q0 = RN(x y) is within one ulp of x / tot, the remainder r = x - q0 tot is exact under an FMA,
// and RN(q0 + r y) is the correctly rounded quotient (Markstein's theorem for round-to-nearest;
// checked bitwise against IEEE division on 2.7e8 random pairs on gfx950, all-ones significands
// included). The quotient takes the sign of x, as x / tot does for tot > 0 (the chain alone turns
// x = -0 into +0). Below the normal range the quotient may differ, but only values far below 0.25
// are there and their code is 0 with the sign of x either way. A divisor that is not finite and
// positive (tot == 0 for a block whose scale rounds to e4m3 zero, or a non-positive or non-finite
// tensor scale) takes IEEE division and the integer encoder.
// Codes: v_cvt_scalef32_pk_fp4_f32 with scale 1.0, which was checked on gfx950 to give exactly
// e2m1_encode (round to nearest even, saturation to +-6, -0 -> 0x8) on the neighbourhoods of every
// rounding boundary, ties, zeros, subnormals and huge values; element 2i goes to the low nibble.
__device__ __forceinline__ uint32_t nvfp4_codes8(const float* f, float tot, float y) {
  if (__builtin_expect(!(tot > 0.0f && tot <= 3.40282347e38f), 0)) {
    uint32_t word = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) word |= e2m1_encode(f[e] / tot) << (4 * e);
    return word;
  }
  float q[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float q0 = f[e] * y;
    const float r = __builtin_fmaf(-q0, tot, f[e]);
    q[e] = __builtin_copysignf(__builtin_fmaf(r, y, q0), f[e]);
  }
  uint32_t word = 0;
  word = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(word, q[0], q[1], 1.0f, 0);
  word = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(word, q[2], q[3], 1.0f, 1);
  word = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(word, q[4], q[5], 1.0f, 2);
  word = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(word, q[6], q[7], 1.0f, 3);
  return word;
}

// x_hat = e2m1(code) * e4m3(scale) (the block-scaled value without the tensor scale, exact in bf16)
// of 8 elements f of a 16-element block whose maximum magnitude is amax16 -- the same arithmetic as
// nvfp4_quantize_kernel's x_hat, so a producer holding half a block (and its partner's maximum) writes
// the same bits as the quantizer run on its output.
__device__ __forceinline__ void nvfp4_xhat8(const float* f, float amax16, float ts, float* out) {
  uint32_t code;
  float tot;
  nvfp4_block_scale(amax16, ts, code, tot);
  const uint32_t w = nvfp4_codes8(f, tot, 1.0f / tot);
  const float s = e4m3_decode(code);
  const auto v0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 0);
  const auto v1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 1);
  const auto v2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 2);
  const auto v3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 3);
  const float e2[8] = {v0[0], v0[1], v1[0], v1[1], v2[0], v2[1], v3[0], v3[1]};
#pragma unroll
  for (int e = 0; e < 8; ++e) out[e] = e2[e] * s;
}

// x_hat of 8 bf16 values (fp32 f) whose 16-element block is split between this lane and lane ^ 1
// (which holds the other 8): the block maximum is exchanged between the two lanes. Every lane of the
// wave must execute this (the exchange reads the partner lane); a lane outside the data passes
// zeros and discards the result.
// The SwiGLU pair's fused NVFP4-linear epilogue on 8 elements (token_update.py:620-631): a = x1 s1 + b1
// and b = x2 s2 + b2 in fp32 (one fma each when there are biases), out = (a * sigmoid(a)) * b with
// sigmoid(a) = 1 / (1 + e^-a). Shared by the SwiGLU kernel and the w2 GEMM epilogue (the same bits).
__device__ __forceinline__ void swiglu_scaled8(const float* x1, float s1, const float* ba, const float* x2, float s2,
                                               const float* bb, bool bias, float* out) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float av = bias ? __builtin_fmaf(x1[e], s1, ba[e]) : x1[e] * s1;
    const float bv = bias ? __builtin_fmaf(x2[e], s2, bb[e]) : x2[e] * s2;
    const float silu = av * (1.0f / (1.0f + expf(-av)));
    out[e] = silu * bv;
  }
}

__device__ __forceinline__ void nvfp4_xhat8_pair(const float* f, float ts, float* out) {
  float am = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) am = fmaxf(am, fabsf(f[e]));
  const float amax16 = fmaxf(am, __shfl_xor(am, 1, 64));
  nvfp4_xhat8(f, amax16, ts, out);
}

}  // namespace oudjat
