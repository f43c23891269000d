// OCP e4m3fn encoding shared by the FP8 quantizers and the producers that write FP8 operands directly.
#pragma once

#include "common.hpp"

namespace oudjat {

// e4m3fn code of |v| <= 448 with round-to-nearest-even (subnormals included), OCP 8-bit definition.
__device__ __forceinline__ uint32_t e4m3_code_abs(float a) {
  const uint32_t u = __float_as_uint(a);
  const int e = (int)((u >> 23) & 0xff) - 127;
  if (e < -6) return (uint32_t)__builtin_rintf(a * 512.0f);  // m * 2^-9, m in [0, 8]
  const uint32_t r = u + 0x7ffffu + ((u >> 20) & 1u);      // RNE from 23 to 3 mantissa bits
  const uint32_t code = ((uint32_t)((int)((r >> 23) & 0xff) - 127 + 7) << 3) | ((r >> 20) & 7u);
  return code > 0x7eu ? 0x7eu : code;
}

// The activation code of FastFP8Linear's quantizer (fp8_fast_linear.py:71-73, 183-186): v = x * s in
// fp32 (s the bf16 inverse scale as fp32), clamped to +-448, e4m3fn with round-to-nearest-even; the
// sign bit | magnitude code, NaN -> 0x7f with its sign.
__device__ __forceinline__ uint32_t fp8_act_code(float x, float s) {
  const float v = x * s;
  const uint32_t sign = (__float_as_uint(v) >> 31) << 7;
  return sign | (v != v ? 0x7fu : e4m3_code_abs(fminf(fabsf(v), 448.0f)));
}

}  // namespace oudjat
