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
// The e4m3 scale is encoded by integer code written from the OCP 8-bit definition. The e2m1 codes
// come from gfx950's v_cvt_scalef32_pk_fp4_f32 (scale operand 1.0), whose rounding (nearest even,
// saturating, -0 -> 0x8) was checked against an integer encoder written from the OCP MX definition
// on the neighbourhood of every rounding boundary; blocks whose divisor is not a positive finite
// value keep the integer encoder. Dequantize decodes with v_cvt_scalef32_pk_f32_fp4 (checked against
// the e2m1 table for all 256 code bytes).
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

// One workgroup (256 threads) per 128-row x 64 CT-column region (CT scale tiles side by side),
// 64 / CT rows per pass: lane t of a pass owns row t / (4 CT) and 16-element block t % (4 CT) of the
// region, so 4 CT consecutive lanes read 128 CT contiguous bytes of one row (two 16-byte loads each)
// and write its 32 CT bytes of codes (8 each). The block scale is computed once per block; the 4
// scale bytes of a row within a scale tile are contiguous in the swizzled layout and go to LDS as one
// word from the tile's first lane of the row; the CT finished tiles are stored at the end.
//
// XH: also write xh[row, col] = e2m1(code) * e4m3(scale) as bf16 -- the block-scaled value without the
// tensor scale, exact in bf16 (at most 2 + 4 significant bits, magnitudes 2^-10 .. 2688): the operand
// a bf16 MFMA GEMM multiplies in place of the packed tensor, as a block-scaled FP4 GEMM does. qd / sc
// may then be NULL (only xh written).
template <int CT, bool XH>
__global__ __launch_bounds__(256) void nvfp4_quantize_kernel(const uint16_t* __restrict__ x, int64_t M, int64_t K,
                                                             int64_t sm, const float* __restrict__ tsp,
                                                             uint8_t* __restrict__ qd, uint8_t* __restrict__ sc,
                                                             uint16_t* __restrict__ xh, int64_t xs) {
  constexpr int LPR = 4 * CT;        // lanes per row
  constexpr int RPP = 256 / LPR;     // rows per pass
  const int pm = blockIdx.y;
  const int t = threadIdx.x;
  const int j = t % LPR;
  const int64_t col = ((int64_t)blockIdx.x * CT) * 64 + j * 16;
  const bool col_ok = col < K;  // K % 16 == 0: a block is wholly in or out
  const float ts = *tsp;
  const int64_t tiles_n = (K + 63) >> 6;
  __shared__ __align__(16) uint32_t sscale[CT * 128];  // the CT scale tiles, in their global byte order
#pragma unroll
  for (int pass = 0; pass < 128 / RPP; ++pass) {
    const int r = pass * RPP + t / LPR;  // row within the tile
    const int64_t row = (int64_t)pm * 128 + r;
    const bool ok = col_ok && row < M;
    float f[16];
    if (ok) {
      const uint4* p = reinterpret_cast<const uint4*>(x + row * sm + col);
      unpack8(p[0], f);
      unpack8(p[1], f + 8);
    } else {
#pragma unroll
      for (int e = 0; e < 16; ++e) f[e] = 0.0f;
    }
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; ++e) amax = fmaxf(amax, fabsf(f[e]));
    uint32_t code;
    float tot;
    nvfp4_block_scale(amax, ts, code, tot);
    const float y = 1.0f / tot;
    const uint32_t w0 = nvfp4_codes8(f, tot, y), w1 = nvfp4_codes8(f + 8, tot, y);
    if (ok && qd) *reinterpret_cast<uint2*>(qd + row * (K >> 1) + (col >> 1)) = make_uint2(w0, w1);
    if constexpr (XH) {
      if (ok) {
        const float s = e4m3_decode(code);
        float h[16];
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          const uint32_t w = half ? w1 : w0;
          const auto v0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 0);
          const auto v1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 1);
          const auto v2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 2);
          const auto v3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 3);
          const float e2[8] = {v0[0], v0[1], v1[0], v1[1], v2[0], v2[1], v3[0], v3[1]};
#pragma unroll
          for (int e = 0; e < 8; ++e) h[half * 8 + e] = e2[e] * s;
        }
        uint4* d = reinterpret_cast<uint4*>(xh + row * xs + col);
        d[0] = pack8(h);
        d[1] = pack8(h + 8);
      }
    }
    // Scale bytes of the row's 4 blocks of this tile (zero for blocks past K or rows past M).
    const uint32_t b = ok ? code : 0u;
    const uint32_t b1 = __shfl_down(b, 1, 64), b2 = __shfl_down(b, 2, 64), b3 = __shfl_down(b, 3, 64);
    if ((j & 3) == 0) sscale[(j / 4) * 128 + (r & 31) * 4 + (r >> 5)] = b | (b1 << 8) | (b2 << 16) | (b3 << 24);
  }
  if (!sc) return;  // uniform over the workgroup
  // The workgroup's CT scale tiles (512 bytes each, consecutive in the swizzled layout) leave as
  // whole 16-byte stores instead of 4-byte pieces spread over the passes.
  __syncthreads();
  const int64_t tile0 = (int64_t)pm * tiles_n + (int64_t)blockIdx.x * CT;
  if (t < CT * 32 && (int64_t)blockIdx.x * CT + t / 32 < tiles_n)
    reinterpret_cast<uint4*>(sc + tile0 * 512)[t] = reinterpret_cast<const uint4*>(sscale)[t];
}

// Dequantize: one workgroup per 128-row x 64 CT-column region, lane t of a pass decoding the 8
// codes (4 bytes) of 8-element chunk t % (8 CT) of row t / (8 CT), so every 16-byte store of a wave
// writes 1 KB of consecutive row segments (whole cache lines). e2m1 values by
// v_cvt_scalef32_pk_f32_fp4 with scale 1.0 (checked on gfx950 against the e2m1 table for all 256
// code bytes); x = (e2m1 * s) * ts in fp32 (the first product is exact), then bf16.
template <int CT>
__global__ __launch_bounds__(256) void nvfp4_dequantize_kernel(const uint8_t* __restrict__ qd,
                                                               const uint8_t* __restrict__ sc,
                                                               const float* __restrict__ tsp, int64_t M, int64_t K,
                                                               uint16_t* __restrict__ out, int64_t os) {
  constexpr int LPR = 8 * CT;
  constexpr int RPP = 256 / LPR;
  const int pm = blockIdx.y;
  const int t = threadIdx.x;
  const int c = t % LPR;  // 8-element chunk within the region row
  const int64_t col = ((int64_t)blockIdx.x * CT) * 64 + c * 8;
  if (col >= K) return;
  const float ts = *tsp;
  const int64_t tiles_n = (K + 63) >> 6;
  const int64_t tile = (int64_t)pm * tiles_n + (int64_t)blockIdx.x * CT + c / 8;
  const int jb = (c >> 1) & 3;  // block within the scale tile
  // Every pass's scale byte and code word are loaded first (all loads of the lane in flight at
  // once), then decoded and stored.
  constexpr int NP = 128 / RPP;
  uint32_t wq[NP], sq[NP];
#pragma unroll
  for (int pass = 0; pass < NP; ++pass) {
    const int r = pass * RPP + t / LPR;
    const int64_t row = (int64_t)pm * 128 + r;
    wq[pass] = 0u;
    sq[pass] = 0u;
    if (row < M) {
      sq[pass] = sc[tile * 512 + (r & 31) * 16 + (r >> 5) * 4 + jb];
      wq[pass] = *reinterpret_cast<const uint32_t*>(qd + row * (K >> 1) + (col >> 1));
    }
  }
#pragma unroll
  for (int pass = 0; pass < NP; ++pass) {
    const int r = pass * RPP + t / LPR;
    const int64_t row = (int64_t)pm * 128 + r;
    if (row >= M) break;
    const float s = e4m3_decode((uint8_t)sq[pass]);
    const uint32_t w = wq[pass];
    const auto v0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 0);
    const auto v1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 1);
    const auto v2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 2);
    const auto v3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 3);
    const float e2[8] = {v0[0], v0[1], v1[0], v1[1], v2[0], v2[1], v3[0], v3[1]};
    float f[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = (e2[e] * s) * ts;
    *reinterpret_cast<uint4*>(out + row * os + col) = pack8(f);
  }
}

// Scale tiles per quantize workgroup: 2 if that still leaves >= 1024 workgroups, else 1. (4 tiles,
// whole 128-byte code lines per row, measured slower: 45.0 against 40.9 us at [16464, 4096], 19.6
// against 15.3 us at [16464, 1024]; 1 tile 44.5 / 15.2 us.)
static int nvfp4_quantize_tiles_per_wg(int64_t M, int64_t K) {
  return cdiv(K, 128) * cdiv(M, 128) >= 1024 ? 2 : 1;
}

// Scale tiles per dequantize workgroup: the widest of 4, 2, 1 that still leaves >= 1024 workgroups.
static int nvfp4_tiles_per_wg(int64_t M, int64_t K) {
  for (int ct : {4, 2}) {
    if (cdiv(K, 64 * ct) * cdiv(M, 128) >= 1024) return ct;
  }
  return 1;
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
  OUDJAT_REQUIRE(sm % 8 == 0 && sm >= K && aligned(x, 16) && aligned(qdata, 8) && aligned(scales, 4),
                 OUDJAT_ERR_UNSUPPORTED_LAYOUT, "nvfp4_quantize: 16-byte aligned rows required");
  OUDJAT_REQUIRE(cdiv(M, 128) < 65536, OUDJAT_ERR_TOO_LARGE, "nvfp4_quantize: M too large");
  const int ct = nvfp4_quantize_tiles_per_wg(M, K);
  dim3 grid((unsigned)cdiv(K, 64 * ct), (unsigned)cdiv(M, 128));
  hipStream_t st = as_stream(stream);
  if (ct == 4) nvfp4_quantize_kernel<4, false><<<grid, 256, 0, st>>>(x, M, K, sm, ts, qdata, scales, nullptr, 0);
  else if (ct == 2) nvfp4_quantize_kernel<2, false><<<grid, 256, 0, st>>>(x, M, K, sm, ts, qdata, scales, nullptr, 0);
  else nvfp4_quantize_kernel<1, false><<<grid, 256, 0, st>>>(x, M, K, sm, ts, qdata, scales, nullptr, 0);
  return check_launch("nvfp4_quantize");
}

extern "C" int oudjat_nvfp4_quantize_dequantize(const uint16_t* x, int64_t M, int64_t K, int64_t sm,
                                                const float* ts, uint8_t* qdata, uint8_t* scales, uint16_t* xhat,
                                                int64_t xhat_stride, oudjat_stream_t stream) {
  OUDJAT_REQUIRE(M >= 0 && K >= 0, OUDJAT_ERR_INVALID_ARGUMENT, "nvfp4_quantize_dequantize: negative size");
  OUDJAT_REQUIRE(K % 16 == 0, OUDJAT_ERR_UNSUPPORTED_SHAPE,
                 "nvfp4_quantize_dequantize: K=%lld must be a multiple of 16", (long long)K);
  if (M == 0 || K == 0) return OUDJAT_OK;
  OUDJAT_REQUIRE(x && ts && xhat && ((qdata == nullptr) == (scales == nullptr)), OUDJAT_ERR_INVALID_ARGUMENT,
                 "nvfp4_quantize_dequantize: null pointer (qdata and scales are given together or not at all)");
  OUDJAT_REQUIRE(sm % 8 == 0 && sm >= K && aligned(x, 16) && xhat_stride % 8 == 0 && xhat_stride >= K &&
                     aligned(xhat, 16) && (!qdata || (aligned(qdata, 8) && aligned(scales, 4))),
                 OUDJAT_ERR_UNSUPPORTED_LAYOUT, "nvfp4_quantize_dequantize: 16-byte aligned rows required");
  OUDJAT_REQUIRE(cdiv(M, 128) < 65536, OUDJAT_ERR_TOO_LARGE, "nvfp4_quantize_dequantize: M too large");
  const int ct = nvfp4_quantize_tiles_per_wg(M, K);
  dim3 grid((unsigned)cdiv(K, 64 * ct), (unsigned)cdiv(M, 128));
  hipStream_t st = as_stream(stream);
  if (ct == 4)
    nvfp4_quantize_kernel<4, true><<<grid, 256, 0, st>>>(x, M, K, sm, ts, qdata, scales, xhat, xhat_stride);
  else if (ct == 2)
    nvfp4_quantize_kernel<2, true><<<grid, 256, 0, st>>>(x, M, K, sm, ts, qdata, scales, xhat, xhat_stride);
  else
    nvfp4_quantize_kernel<1, true><<<grid, 256, 0, st>>>(x, M, K, sm, ts, qdata, scales, xhat, xhat_stride);
  return check_launch("nvfp4_quantize_dequantize");
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
  OUDJAT_REQUIRE(cdiv(M, 128) < 65536, OUDJAT_ERR_TOO_LARGE, "nvfp4_dequantize: M too large");
  const int ct = nvfp4_tiles_per_wg(M, K);
  dim3 grid((unsigned)cdiv(K, 64 * ct), (unsigned)cdiv(M, 128));
  hipStream_t st = as_stream(stream);
  if (ct == 4) nvfp4_dequantize_kernel<4><<<grid, 256, 0, st>>>(qdata, scales, ts, M, K, out, os);
  else if (ct == 2) nvfp4_dequantize_kernel<2><<<grid, 256, 0, st>>>(qdata, scales, ts, M, K, out, os);
  else nvfp4_dequantize_kernel<1><<<grid, 256, 0, st>>>(qdata, scales, ts, M, K, out, os);
  return check_launch("nvfp4_dequantize");
}
