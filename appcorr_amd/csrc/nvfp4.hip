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
#include "nvfp4.hpp"

namespace oudjat {

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
