// NVFP4 activation quantize / dequantize.
//
// Format (16-element blocks, e4m3 block scale relative to an fp32 tensor scale, packed e2m1):
//   amax  = max |x| over the block                      (fp32)
//   sc    = clamp((amax / 6) / ts, 2^-16, 448)          (two IEEE round-to-nearest divisions)
//   s8    = e4m3(sc)                                    (round to nearest even)
//   q_i   = x_i / (ts * float(s8))                      (IEEE division)
//   code  = e2m1(q_i)                                   (round to nearest even, saturating to +-6,
//                                                        sign kept, -0 -> 0x8)
// Codes are packed two per byte, element 2i in the low nibble. Block scales of a 128x64 tile (128
// rows x 4 blocks) are stored as 32x16 bytes: scale (r, j) of the tile goes to byte
// (r % 32) * 16 + (r / 32) * 4 + j, tiles in row-major tile order. Scales of rows >= M are 0.
//
// Both conversions are integer/compare code written from the OCP 8-bit / MX e2m1 definitions, not
// hardware converts, so the rounding is exactly the one stated above.
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

// One workgroup per 128x64 tile; thread t owns row t/2 and blocks 2*(t%2), 2*(t%2)+1 (32 elements).
__global__ __launch_bounds__(256) void nvfp4_quantize_kernel(const uint16_t* __restrict__ x, int64_t M, int64_t K,
                                                             int64_t sm, const float* __restrict__ tsp,
                                                             uint8_t* __restrict__ qd, uint8_t* __restrict__ sc) {
  const int pn = blockIdx.x, pm = blockIdx.y;
  const int t = threadIdx.x;
  const int r = t >> 1;
  const int jb = (t & 1) * 2;
  const int64_t row = (int64_t)pm * 128 + r;
  const int64_t col0 = (int64_t)pn * 64 + jb * 16;
  const float ts = *tsp;
  const bool row_ok = row < M;
  uint32_t s8[2];
  uint32_t packed[4];
#pragma unroll
  for (int bb = 0; bb < 2; ++bb) {
    const int64_t c0 = col0 + bb * 16;
    const bool ok = row_ok && c0 < K;
    float f[16];
    if (ok) {
      const uint4* p = reinterpret_cast<const uint4*>(x + row * sm + c0);
      unpack8(p[0], f);
      unpack8(p[1], f + 8);
    } else {
#pragma unroll
      for (int e = 0; e < 16; ++e) f[e] = 0.0f;
    }
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; ++e) amax = fmaxf(amax, fabsf(f[e]));
    const float bs = amax / kE2m1Max;
    const float scaled = fminf(fmaxf(bs / ts, kE4m3Eps), kE4m3Max);
    const uint32_t code = e4m3_encode_pos(scaled);
    const float tot = ts * e4m3_decode(code);
    s8[bb] = ok ? code : 0u;
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      uint32_t word = 0;
#pragma unroll
      for (int e = 0; e < 8; ++e) word |= e2m1_encode(f[w * 8 + e] / tot) << (4 * e);
      packed[bb * 2 + w] = word;
    }
  }
  if (row_ok) {
    uint8_t* qrow = qd + row * (K >> 1);
    const int64_t qc = (int64_t)pn * 32 + jb * 8;
    // 8-byte stores: rows of K/2 bytes are only guaranteed 8-byte aligned (K % 16 == 0).
    if (qc < (K >> 1)) *reinterpret_cast<uint2*>(qrow + qc) = make_uint2(packed[0], packed[1]);
    if (qc + 8 < (K >> 1)) *reinterpret_cast<uint2*>(qrow + qc + 8) = make_uint2(packed[2], packed[3]);
  }
  const int64_t tile = (int64_t)pm * gridDim.x + pn;
  uint16_t pair = (uint16_t)(s8[0] | (s8[1] << 8));
  *reinterpret_cast<uint16_t*>(sc + tile * 512 + (r & 31) * 16 + (r >> 5) * 4 + jb) = pair;
}

// One thread per 16-element block.
__global__ __launch_bounds__(256) void nvfp4_dequantize_kernel(const uint8_t* __restrict__ qd,
                                                               const uint8_t* __restrict__ sc,
                                                               const float* __restrict__ tsp, int64_t M, int64_t K,
                                                               uint16_t* __restrict__ out, int64_t os) {
  const int64_t nb = K >> 4;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= M * nb) return;
  const int64_t row = gid / nb;
  const int64_t jg = gid - row * nb;
  const float ts = *tsp;
  const int64_t grid_n = (K + 63) >> 6;
  const int64_t pm = row >> 7, pn = jg >> 2;
  const int r = (int)(row & 127), j = (int)(jg & 3);
  const float s = e4m3_decode(sc[(pm * grid_n + pn) * 512 + (r & 31) * 16 + (r >> 5) * 4 + j]);
  const uint2 w = *reinterpret_cast<const uint2*>(qd + row * (K >> 1) + jg * 8);
  float f[16];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    f[e] = (e2m1_decode((w.x >> (4 * e)) & 15u) * s) * ts;
    f[8 + e] = (e2m1_decode((w.y >> (4 * e)) & 15u) * s) * ts;
  }
  uint4* o = reinterpret_cast<uint4*>(out + row * os + jg * 16);
  o[0] = pack8(f);
  o[1] = pack8(f + 8);
}

}  // namespace oudjat

using namespace oudjat;

extern "C" int oudjat_nvfp4_quantize(const uint16_t* x, int64_t M, int64_t K, int64_t sm, const float* ts,
                                     uint8_t* qdata, uint8_t* scales, oudjat_stream_t stream) {
  OUDJAT_REQUIRE(M >= 0 && K >= 0, OUDJAT_ERR_INVALID_ARGUMENT, "nvfp4_quantize: negative size");
  OUDJAT_REQUIRE(K % 16 == 0, OUDJAT_ERR_UNSUPPORTED_SHAPE, "nvfp4_quantize: K=%lld must be a multiple of 16",
                 (long long)K);
  if (M == 0 || K == 0) return OUDJAT_OK;
  OUDJAT_REQUIRE(x && ts && qdata && scales, OUDJAT_ERR_INVALID_ARGUMENT, "nvfp4_quantize: null pointer");
  OUDJAT_REQUIRE(sm % 8 == 0 && sm >= K && aligned(x, 16) && aligned(qdata, 8) && aligned(scales, 2),
                 OUDJAT_ERR_UNSUPPORTED_LAYOUT, "nvfp4_quantize: 16-byte aligned rows required");
  dim3 grid((unsigned)cdiv(K, 64), (unsigned)cdiv(M, 128));
  nvfp4_quantize_kernel<<<grid, 256, 0, as_stream(stream)>>>(x, M, K, sm, ts, qdata, scales);
  return check_launch("nvfp4_quantize");
}

extern "C" int oudjat_nvfp4_dequantize(const uint8_t* qdata, const uint8_t* scales, const float* ts, int64_t M,
                                       int64_t K, uint16_t* out, int64_t os, oudjat_stream_t stream) {
  OUDJAT_REQUIRE(M >= 0 && K >= 0, OUDJAT_ERR_INVALID_ARGUMENT, "nvfp4_dequantize: negative size");
  OUDJAT_REQUIRE(K % 16 == 0, OUDJAT_ERR_UNSUPPORTED_SHAPE, "nvfp4_dequantize: K=%lld must be a multiple of 16",
                 (long long)K);
  if (M == 0 || K == 0) return OUDJAT_OK;
  OUDJAT_REQUIRE(qdata && scales && ts && out, OUDJAT_ERR_INVALID_ARGUMENT, "nvfp4_dequantize: null pointer");
  OUDJAT_REQUIRE(os % 8 == 0 && os >= K && aligned(out, 16) && aligned(qdata, 8), OUDJAT_ERR_UNSUPPORTED_LAYOUT,
                 "nvfp4_dequantize: 16-byte aligned rows required");
  const int64_t n = M * (K / 16);
  nvfp4_dequantize_kernel<<<(unsigned)cdiv(n, 256), 256, 0, as_stream(stream)>>>(qdata, scales, ts, M, K, out, os);
  return check_launch("nvfp4_dequantize");
}
