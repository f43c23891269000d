// Low-precision correction linears (the reference's FastFP4Linear / FastFP8Linear,
// offload/server/model/fp4_fast_linear.py and fp8_fast_linear.py) on gfx950.
//
// gfx950 has no MFMA for NVFP4's 16-element blocks with e4m3 scales, and every value such a GEMM
// multiplies -- e2m1 code x e4m3 block scale, or an e4m3 code -- is exact in bf16. So the operands are
// quantized with the reference's rounding, written back as those exact bf16 values, and multiplied by
// the bf16 MFMA GEMM with fp32 accumulation: the products and the accumulation are those of the scaled
// FP4 / FP8 GEMM, up to the order of the fp32 sums. The per-tensor factors are applied where the
// reference applies them:
//   NVFP4 (torch._scaled_mm has no per-tensor output scale): raw = bf16(acc) from the GEMM, then this
//     file's scale_bias (out = raw * s + b, fp32, one rounding) or, for the SwiGLU pair, the fused
//     silu(raw1 * s1 + b1) * (raw2 * s2 + b2) epilogue (token_update.py:571-669);
//   FP8 (scales inside the GEMM): bf16(acc * (sa * sb) + b) by the GEMM's accumulator scale.
#include "fp8.hpp"
#include "nvfp4.hpp"

namespace oudjat {
namespace {

constexpr int kLpThreads = 256;

__device__ __forceinline__ float e4m3_value_abs(uint32_t c) {
  const uint32_t e = (c >> 3) & 0xf, m = c & 7u;
  return e == 0 ? (float)m * 0.001953125f : __uint_as_float(((e + 120u) << 23) | (m << 20));
}

// The e4m3 value of a finite or infinite v clamped to [-448, 448] (NaN stays NaN), as fp32.
__device__ __forceinline__ float e4m3_round(float v) {
  if (v != v) return v;
  const float a = fminf(fabsf(v), 448.0f);
  return __builtin_copysignf(e4m3_value_abs(e4m3_code_abs(a)), v);
}

// FP8 quantize-dequantize of rows [M, K]: out = e4m3(clamp(x * scale, +-448)) as bf16 (mode 0: the
// compiled activation path of FastFP8Linear, fp32 product with the bf16 inverse scale,
// fp8_fast_linear.py:71-73, 183-186), or out = e4m3(clamp(bf16(x / bf16(scale)), +-448)) (mode 1: the
// eager weight path, fp8_fast_linear.py:123-125: the division's result is a bf16 tensor).
__global__ void __launch_bounds__(kLpThreads) fp8_qdq_kernel(const uint16_t* __restrict__ x, int64_t M, int64_t K,
                                                             int64_t sm, const float* __restrict__ scalep, int mode,
                                                             uint16_t* __restrict__ out, int64_t os) {
  const int64_t chunks = K >> 3;
  const int64_t i = (int64_t)blockIdx.x * kLpThreads + threadIdx.x;
  if (i >= M * chunks) return;
  const int64_t row = i / chunks, c = (i - row * chunks) * 8;
  float s = *scalep;
  if (mode == 1) s = round_bf16(s);
  float f[8];
  unpack8(*reinterpret_cast<const uint4*>(x + row * sm + c), f);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float v = mode == 0 ? f[e] * s : round_bf16((float)((double)f[e] / (double)s));
    f[e] = e4m3_round(v);
  }
  *reinterpret_cast<uint4*>(out + row * os + c) = pack8(f);
}

// The same quantizer writing the e4m3fn codes themselves (one byte per element, the operands of the
// native FP8 GEMM): sign bit | magnitude code; NaN gives the NaN code 0x7f with its sign.
__global__ void __launch_bounds__(kLpThreads) fp8_quantize_kernel(const uint16_t* __restrict__ x, int64_t M, int64_t K,
                                                                  int64_t sm, const float* __restrict__ scalep,
                                                                  int mode, uint8_t* __restrict__ out, int64_t os) {
  const int64_t chunks = K >> 3;
  const int64_t i = (int64_t)blockIdx.x * kLpThreads + threadIdx.x;
  if (i >= M * chunks) return;
  const int64_t row = i / chunks, c = (i - row * chunks) * 8;
  float s = *scalep;
  if (mode == 1) s = round_bf16(s);
  float f[8];
  unpack8(*reinterpret_cast<const uint4*>(x + row * sm + c), f);
  uint32_t code[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    if (mode == 0) {
      code[e] = fp8_act_code(f[e], s);
    } else {
      const float v = round_bf16((float)((double)f[e] / (double)s));
      const uint32_t sign = (__float_as_uint(v) >> 31) << 7;
      code[e] = sign | (v != v ? 0x7fu : e4m3_code_abs(fminf(fabsf(v), 448.0f)));
    }
  }
  uint2 w;
  w.x = code[0] | (code[1] << 8) | (code[2] << 16) | (code[3] << 24);
  w.y = code[4] | (code[5] << 8) | (code[6] << 16) | (code[7] << 24);
  *reinterpret_cast<uint2*>(out + row * os + c) = w;
}

// NVFP4 output epilogue: out = bf16(v * s + b) over [M, N] (the fp32 multiply-add contracted to one
// rounding when a bias is present, as the reference's Triton kernel compiles it; v * s without one),
// and with gamma additionally bf16(that * gamma[col]) (the block's LayerScale on the result).
__global__ void __launch_bounds__(kLpThreads) scale_bias_kernel(const uint16_t* __restrict__ x, int64_t M, int64_t N,
                                                                int64_t xs, float s, const uint16_t* __restrict__ bias,
                                                                const uint16_t* __restrict__ gamma,
                                                                uint16_t* __restrict__ out, int64_t os) {
  const int64_t chunks = N >> 3;
  const int64_t i = (int64_t)blockIdx.x * kLpThreads + threadIdx.x;
  if (i >= M * chunks) return;
  const int64_t row = i / chunks, c = (i - row * chunks) * 8;
  float v[8], b[8], g[8];
  unpack8(*reinterpret_cast<const uint4*>(x + row * xs + c), v);
  if (bias) unpack8(*reinterpret_cast<const uint4*>(bias + c), b);
  if (gamma) unpack8(*reinterpret_cast<const uint4*>(gamma + c), g);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float y = bias ? __builtin_fmaf(v[e], s, b[e]) : v[e] * s;
    if (gamma) y = round_bf16(y) * g[e];
    v[e] = y;
  }
  *reinterpret_cast<uint4*>(out + row * os + c) = pack8(v);
}

// The SwiGLU pair's fused NVFP4 epilogue (token_update.py:620-631): a = x1 s1 + b1, b = x2 s2 + b2
// (fp32; contracted with a bias as above), out = bf16((a * sigmoid(a)) * b), sigmoid(a) = 1 / (1 + e^-a).
// XH: the row written is the NVFP4 operand x_hat (tensor scale *xh_ts) of that bf16 output -- the input
// of the NVFP4 w3 linear -- as nvfp4_quantize_dequantize gives it; a 16-element block is the chunk
// pair of threads 2k, 2k + 1 (N % 16 == 0).
template <bool XH>
__global__ void __launch_bounds__(kLpThreads) swiglu_scaled_kernel(const uint16_t* __restrict__ x1, float s1,
                                                                   const uint16_t* __restrict__ b1,
                                                                   const uint16_t* __restrict__ x2, float s2,
                                                                   const uint16_t* __restrict__ b2, int64_t M,
                                                                   int64_t N, uint16_t* __restrict__ out,
                                                                   const float* __restrict__ xh_ts) {
  const int64_t chunks = N >> 3;
  const int64_t i = (int64_t)blockIdx.x * kLpThreads + threadIdx.x;
  if (i >= M * chunks) return;
  const int64_t row = i / chunks, c = (i - row * chunks) * 8;
  float a[8], b[8], ba[8], bb[8];
  unpack8(*reinterpret_cast<const uint4*>(x1 + row * N + c), a);
  unpack8(*reinterpret_cast<const uint4*>(x2 + row * N + c), b);
  if (b1) {
    unpack8(*reinterpret_cast<const uint4*>(b1 + c), ba);
    unpack8(*reinterpret_cast<const uint4*>(b2 + c), bb);
  }
  swiglu_scaled8(a, s1, ba, b, s2, bb, b1 != nullptr, a);
  if constexpr (XH) {
    float h[8];
    unpack8(pack8(a), a);  // the bf16 output the quantizer reads
    nvfp4_xhat8_pair(a, *xh_ts, h);
    *reinterpret_cast<uint4*>(out + row * N + c) = pack8(h);
  } else {
    *reinterpret_cast<uint4*>(out + row * N + c) = pack8(a);
  }
}

// amax[0] = max(amax[0], max |x|) over rows [M, K] (the calibration observer's running maximum).
// |x| is taken as its bit pattern, so the unsigned maximum orders finite values, infinity and NaN the
// way torch.maximum(amax, x.abs().amax()) does (NaN wins).
__global__ void __launch_bounds__(kLpThreads) amax_kernel(const uint16_t* __restrict__ x, int64_t M, int64_t K,
                                                          int64_t sm, float* __restrict__ amax) {
  const int64_t chunks = K >> 3;
  const int64_t n = M * chunks;
  uint32_t m = 0;
  for (int64_t i = (int64_t)blockIdx.x * kLpThreads + threadIdx.x; i < n; i += (int64_t)gridDim.x * kLpThreads) {
    const int64_t row = i / chunks, c = (i - row * chunks) * 8;
    const uint4 v = *reinterpret_cast<const uint4*>(x + row * sm + c);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      m = max(m, (w[e] & 0x7fffu) << 16);
      m = max(m, w[e] & 0x7fff0000u);
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, o, 64));
  __shared__ uint32_t red[kLpThreads / 64];
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kLpThreads / 64; ++w) m = max(m, red[w]);
    atomicMax(reinterpret_cast<unsigned int*>(amax), m);
  }
}

int launch_rows(const char* what, int64_t M, int64_t K) {
  OUDJAT_REQUIRE(M >= 0 && K >= 0, OUDJAT_ERR_INVALID_ARGUMENT, "%s: negative size", what);
  OUDJAT_REQUIRE(K % 8 == 0, OUDJAT_ERR_UNSUPPORTED_SHAPE, "%s: the row length %lld must be a multiple of 8", what,
                 (long long)K);
  OUDJAT_REQUIRE(M * (K / 8) < ((int64_t)1 << 40), OUDJAT_ERR_TOO_LARGE, "%s: too large", what);
  return OUDJAT_OK;
}

}  // namespace
}  // namespace oudjat

using namespace oudjat;

extern "C" int oudjat_fp8_quantize_dequantize(const uint16_t* x, int64_t M, int64_t K, int64_t stride_m,
                                              const float* scale, int mode, uint16_t* out, int64_t out_stride,
                                              oudjat_stream_t stream) {
  int st = launch_rows("fp8_quantize_dequantize", M, K);
  if (st != OUDJAT_OK) return st;
  OUDJAT_REQUIRE(mode == 0 || mode == 1, OUDJAT_ERR_INVALID_ARGUMENT, "fp8_quantize_dequantize: mode %d", mode);
  if (M == 0 || K == 0) return OUDJAT_OK;
  OUDJAT_REQUIRE(x && scale && out, OUDJAT_ERR_INVALID_ARGUMENT, "fp8_quantize_dequantize: null pointer");
  OUDJAT_REQUIRE(aligned(x, 16) && aligned(out, 16) && stride_m % 8 == 0 && out_stride % 8 == 0, OUDJAT_ERR_UNSUPPORTED_LAYOUT,
                 "fp8_quantize_dequantize: 16-byte aligned rows required");
  const int64_t n = M * (K / 8);
  fp8_qdq_kernel<<<(unsigned)cdiv(n, kLpThreads), kLpThreads, 0, as_stream(stream)>>>(x, M, K, stride_m, scale, mode,
                                                                                      out, out_stride);
  return check_launch("fp8_quantize_dequantize");
}

extern "C" int oudjat_fp8_quantize(const uint16_t* x, int64_t M, int64_t K, int64_t stride_m, const float* scale,
                                   int mode, uint8_t* out, int64_t out_stride, oudjat_stream_t stream) {
  int st = launch_rows("fp8_quantize", M, K);
  if (st != OUDJAT_OK) return st;
  OUDJAT_REQUIRE(mode == 0 || mode == 1, OUDJAT_ERR_INVALID_ARGUMENT, "fp8_quantize: mode %d", mode);
  if (M == 0 || K == 0) return OUDJAT_OK;
  OUDJAT_REQUIRE(x && scale && out, OUDJAT_ERR_INVALID_ARGUMENT, "fp8_quantize: null pointer");
  OUDJAT_REQUIRE(aligned(x, 16) && aligned(out, 8) && stride_m % 8 == 0 && out_stride % 8 == 0,
                 OUDJAT_ERR_UNSUPPORTED_LAYOUT, "fp8_quantize: 16-byte aligned input rows, 8-byte aligned output rows");
  const int64_t n = M * (K / 8);
  fp8_quantize_kernel<<<(unsigned)cdiv(n, kLpThreads), kLpThreads, 0, as_stream(stream)>>>(x, M, K, stride_m, scale,
                                                                                           mode, out, out_stride);
  return check_launch("fp8_quantize");
}

extern "C" int oudjat_scale_bias_rows(const uint16_t* x, int64_t M, int64_t N, int64_t x_stride, float scale,
                                      const uint16_t* bias, const uint16_t* gamma, uint16_t* out, int64_t out_stride,
                                      oudjat_stream_t stream) {
  int st = launch_rows("scale_bias_rows", M, N);
  if (st != OUDJAT_OK) return st;
  if (M == 0 || N == 0) return OUDJAT_OK;
  OUDJAT_REQUIRE(x && out, OUDJAT_ERR_INVALID_ARGUMENT, "scale_bias_rows: null pointer");
  OUDJAT_REQUIRE(aligned(x, 16) && aligned(out, 16) && (!bias || aligned(bias, 16)) && (!gamma || aligned(gamma, 16)) &&
                     x_stride % 8 == 0 && out_stride % 8 == 0,
                 OUDJAT_ERR_UNSUPPORTED_LAYOUT, "scale_bias_rows: 16-byte aligned rows required");
  const int64_t n = M * (N / 8);
  scale_bias_kernel<<<(unsigned)cdiv(n, kLpThreads), kLpThreads, 0, as_stream(stream)>>>(x, M, N, x_stride, scale,
                                                                                         bias, gamma, out, out_stride);
  return check_launch("scale_bias_rows");
}

static int swiglu_launch(const uint16_t* x1, float s1, const uint16_t* b1, const uint16_t* x2, float s2,
                         const uint16_t* b2, int64_t M, int64_t N, const float* xh_ts, uint16_t* out,
                         oudjat_stream_t stream, const char* what) {
  int st = launch_rows(what, M, N);
  if (st != OUDJAT_OK) return st;
  if (M == 0 || N == 0) return OUDJAT_OK;
  OUDJAT_REQUIRE(x1 && x2 && out && ((b1 == nullptr) == (b2 == nullptr)), OUDJAT_ERR_INVALID_ARGUMENT,
                 "%s: null pointer (both biases or neither)", what);
  OUDJAT_REQUIRE(aligned(x1, 16) && aligned(x2, 16) && aligned(out, 16) && (!b1 || (aligned(b1, 16) && aligned(b2, 16))),
                 OUDJAT_ERR_UNSUPPORTED_LAYOUT, "%s: 16-byte aligned rows required", what);
  const int64_t n = M * (N / 8);
  const unsigned grid = (unsigned)cdiv(n, kLpThreads);
  if (xh_ts) {
    OUDJAT_REQUIRE(N % 16 == 0, OUDJAT_ERR_UNSUPPORTED_SHAPE, "%s: NVFP4 output needs N %% 16 == 0", what);
    swiglu_scaled_kernel<true><<<grid, kLpThreads, 0, as_stream(stream)>>>(x1, s1, b1, x2, s2, b2, M, N, out, xh_ts);
  } else {
    swiglu_scaled_kernel<false><<<grid, kLpThreads, 0, as_stream(stream)>>>(x1, s1, b1, x2, s2, b2, M, N, out, nullptr);
  }
  return check_launch(what);
}

extern "C" int oudjat_swiglu_scaled(const uint16_t* x1, float s1, const uint16_t* b1, const uint16_t* x2, float s2,
                                    const uint16_t* b2, int64_t M, int64_t N, uint16_t* out, oudjat_stream_t stream) {
  return swiglu_launch(x1, s1, b1, x2, s2, b2, M, N, nullptr, out, stream, "swiglu_scaled");
}

extern "C" int oudjat_swiglu_scaled_nvfp4(const uint16_t* x1, float s1, const uint16_t* b1, const uint16_t* x2,
                                          float s2, const uint16_t* b2, int64_t M, int64_t N,
                                          const float* tensor_scale, uint16_t* xhat, oudjat_stream_t stream) {
  OUDJAT_REQUIRE(tensor_scale || M == 0 || N == 0, OUDJAT_ERR_INVALID_ARGUMENT, "swiglu_scaled_nvfp4: null tensor scale");
  return swiglu_launch(x1, s1, b1, x2, s2, b2, M, N, tensor_scale, xhat, stream, "swiglu_scaled_nvfp4");
}

extern "C" int oudjat_amax_update(const uint16_t* x, int64_t M, int64_t K, int64_t stride_m, float* amax,
                                  oudjat_stream_t stream) {
  int st = launch_rows("amax_update", M, K);
  if (st != OUDJAT_OK) return st;
  if (M == 0 || K == 0) return OUDJAT_OK;
  OUDJAT_REQUIRE(x && amax, OUDJAT_ERR_INVALID_ARGUMENT, "amax_update: null pointer");
  OUDJAT_REQUIRE(aligned(x, 16) && stride_m % 8 == 0 && aligned(amax, 4), OUDJAT_ERR_UNSUPPORTED_LAYOUT,
                 "amax_update: 16-byte aligned rows required");
  const int64_t n = M * (K / 8);
  const int64_t blocks = cdiv(n, kLpThreads) < 2048 ? cdiv(n, kLpThreads) : 2048;
  amax_kernel<<<(unsigned)blocks, kLpThreads, 0, as_stream(stream)>>>(x, M, K, stride_m, amax);
  return check_launch("amax_update");
}
