// Dense server score of the approximate pass: the mean attention probability each key receives, over
// heads and all queries (patch_attn_prob / patch_attn_prob_layermean).
//
// Two launches, nothing of size N x N is materialised:
//   stats:  for every (image, head, query) the softmax max m and sum l over all keys (two passes over
//           the keys, so that every term exp(s - m) uses the final max, as a row softmax does);
//   colsum: for every (image, 32-key block) the column sums of the probabilities over all queries and
//           heads. Four waves split the query blocks; their partial sums meet in LDS in a fixed order.
//
// Rounding modes (the two paths of attention.py:241-253 and triton_kernels/attention_pscore.py):
//   kDense: s = bf16(bf16(q.k) * scale), p = bf16(exp(s - m) / l) (torch softmax of a bf16 tensor),
//           head mean hm = bf16(sum_h p * fl(1/H)), score = bf16(sum_q hm * fl(1/N));
//   kLse:   s = (q.k) * scale in fp32, lse = m + log(l), p = exp2(s * log2e - lse * log2e) in fp32,
//           score = bf16(sum_{q,h} p * fl(1/(H N))) -- the fused kernel's key-side sum from the row
//           log-sum-exp.
// q.k is one v_mfma_f32_32x32x16_bf16 chain (fp32 accumulation). Stats use S^T = K . Q^T so a query's
// scores sit in one lane pair (lanes l, l ^ 32); colsum uses S = Q . K^T so a key's column sits in one
// lane pair and the sum over queries is a register sum plus one exchange.
#include <cmath>

#include "common.hpp"

namespace oudjat {

static constexpr int kPaWaves = 4;
static constexpr int kPaThreads = kPaWaves * 64;
enum { kDense = 0, kLse = 1 };

// A 16-byte operand fragment of row `row` (< rows, else zeros) at head-dim offset `d0`.
__device__ __forceinline__ bf16x8_t frag16(const uint16_t* base, int64_t row_stride, int row, int rows, int d0) {
  uint4 v = make_uint4(0, 0, 0, 0);
  if (row < rows) v = *reinterpret_cast<const uint4*>(base + (int64_t)row * row_stride + d0);
  return as_bf16x8(v);
}

template <int DH, int MODE>
__global__ __launch_bounds__(kPaThreads) void pattn_stats_kernel(const uint16_t* __restrict__ q, int64_t qrs,
                                                                 const uint16_t* __restrict__ kv, int64_t kvb,
                                                                 int64_t kvn, int64_t kvh, int N, int H, float scale,
                                                                 float* __restrict__ m_out,
                                                                 float* __restrict__ l_out) {
  constexpr int KS = DH / 16;
  const int b = blockIdx.z, h = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l32 = lane & 31, g = lane >> 5;
  const int q0 = (blockIdx.x * kPaWaves + wave) * 32;
  if (q0 >= N) return;  // no barriers below
  const uint16_t* qb = q + (int64_t)b * N * qrs + (int64_t)h * DH;
  const uint16_t* kb = kv + (int64_t)b * kvb + (int64_t)h * kvh;
  bf16x8_t qf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) qf[ks] = frag16(qb, qrs, q0 + l32, N, ks * 16 + 8 * g);

  auto tile = [&](int k0, f32x16_t& acc) {
    bf16x8_t kf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) kf[ks] = frag16(kb, kvn, k0 + l32, N, ks * 16 + 8 * g);
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[ks], qf[ks], acc, 0, 0, 0);
  };
  auto score = [&](float a) -> float {
    return MODE == kDense ? round_bf16(round_bf16(a) * scale) : a * scale;
  };

  float m = -INFINITY;
  for (int k0 = 0; k0 < N; k0 += 32) {
    f32x16_t acc;
    tile(k0, acc);
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int key = k0 + 8 * (v >> 2) + 4 * g + (v & 3);
      if (key < N) m = fmaxf(m, score(acc[v]));
    }
  }
  m = fmaxf(m, __shfl_xor(m, 32, 64));
  float l = 0.0f;
  for (int k0 = 0; k0 < N; k0 += 32) {
    f32x16_t acc;
    tile(k0, acc);
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int key = k0 + 8 * (v >> 2) + 4 * g + (v & 3);
      if (key < N) l += expf(score(acc[v]) - m);
    }
  }
  l += __shfl_xor(l, 32, 64);
  const int qi = q0 + l32;
  if (g == 0 && qi < N) {
    const int64_t o = ((int64_t)b * H + h) * N + qi;
    m_out[o] = MODE == kDense ? m : m + logf(l);  // kLse keeps the row log-sum-exp in m_out
    l_out[o] = l;
  }
}

template <int DH, int MODE>
__global__ __launch_bounds__(kPaThreads) void pattn_colsum_kernel(const uint16_t* __restrict__ q, int64_t qrs,
                                                                  const uint16_t* __restrict__ kv, int64_t kvb,
                                                                  int64_t kvn, int64_t kvh, int N, int H, float scale,
                                                                  const float* __restrict__ m_in,
                                                                  const float* __restrict__ l_in,
                                                                  uint16_t* __restrict__ out, int64_t osb) {
  constexpr int KS = DH / 16;
  constexpr float kLog2e = 1.4426950408889634f;
  __shared__ float part[kPaWaves][32];
  const int b = blockIdx.y;
  const int k0 = blockIdx.x * 32;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l32 = lane & 31, g = lane >> 5;
  const int nqb = (N + 31) / 32;
  const float inv_h = 1.0f / (float)H;
  float col = 0.0f;
  for (int qblk = wave; qblk < nqb; qblk += kPaWaves) {
    const int q0 = qblk * 32;
    float hs[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) hs[v] = 0.0f;
    for (int h = 0; h < H; ++h) {
      const uint16_t* qb = q + (int64_t)b * N * qrs + (int64_t)h * DH;
      const uint16_t* kb = kv + (int64_t)b * kvb + (int64_t)h * kvh;
      f32x16_t acc;
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(frag16(qb, qrs, q0 + l32, N, ks * 16 + 8 * g),
                                                      frag16(kb, kvn, k0 + l32, N, ks * 16 + 8 * g), acc, 0, 0, 0);
      const float* mrow = m_in + ((int64_t)b * H + h) * N;
      const float* lrow = l_in + ((int64_t)b * H + h) * N;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int qi = q0 + 8 * (v >> 2) + 4 * g + (v & 3);
        if (qi < N) {
          if (MODE == kDense) {
            const float s = round_bf16(round_bf16(acc[v]) * scale);
            hs[v] += round_bf16(expf(s - mrow[qi]) / lrow[qi]);
          } else {
            col += exp2f(acc[v] * (scale * kLog2e) - mrow[qi] * kLog2e);
          }
        }
      }
    }
    if (MODE == kDense) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int qi = q0 + 8 * (v >> 2) + 4 * g + (v & 3);
        if (qi < N) col += round_bf16(hs[v] * inv_h);
      }
    }
  }
  col += __shfl_xor(col, 32, 64);
  if (g == 0) part[wave][l32] = col;
  __syncthreads();
  if (wave == 0 && g == 0) {
    float t = part[0][l32];
#pragma unroll
    for (int w = 1; w < kPaWaves; ++w) t += part[w][l32];
    const float factor = MODE == kDense ? 1.0f / (float)N : 1.0f / (float)((int64_t)H * N);
    const int key = k0 + l32;
    if (key < N) out[(int64_t)b * osb + key] = (uint16_t)f32_to_bf16(t * factor);
  }
}

template <int DH, int MODE>
void launch_pattn(const uint16_t* q, int64_t qrs, const uint16_t* kv, int64_t kvb, int64_t kvn, int64_t kvh, int B,
                  int N, int H, float scale, float* ws, uint16_t* out, int64_t osb, hipStream_t st) {
  float* m = ws;
  float* l = ws + (int64_t)B * H * N;
  const dim3 g1((unsigned)cdiv(cdiv(N, 32), kPaWaves), (unsigned)H, (unsigned)B);
  pattn_stats_kernel<DH, MODE><<<g1, kPaThreads, 0, st>>>(q, qrs, kv, kvb, kvn, kvh, N, H, scale, m, l);
  const dim3 g2((unsigned)cdiv(N, 32), (unsigned)B);
  pattn_colsum_kernel<DH, MODE><<<g2, kPaThreads, 0, st>>>(q, qrs, kv, kvb, kvn, kvh, N, H, scale, m, l, out, osb);
}

}  // namespace oudjat

using namespace oudjat;

extern "C" int oudjat_patch_attention_prob(const uint16_t* q, int64_t q_row_stride, int64_t B, int64_t N, int64_t H,
                                           int64_t Dh, const uint16_t* kv, int64_t kv_stride_b, int64_t kv_stride_n,
                                           int64_t kv_stride_h, float scale, int mode, float* workspace,
                                           uint16_t* out, int64_t out_stride_b, oudjat_stream_t stream) {
  OUDJAT_REQUIRE(B >= 0 && N >= 0 && H > 0, OUDJAT_ERR_INVALID_ARGUMENT, "patch_attention_prob: bad size");
  OUDJAT_REQUIRE(mode == kDense || mode == kLse, OUDJAT_ERR_INVALID_ARGUMENT, "patch_attention_prob: mode %d", mode);
  OUDJAT_REQUIRE(Dh == 64 || Dh == 128, OUDJAT_ERR_UNSUPPORTED_SHAPE, "patch_attention_prob: Dh=%lld (64 or 128)",
                 (long long)Dh);
  if (B == 0 || N == 0) return OUDJAT_OK;
  OUDJAT_REQUIRE(q && kv && workspace && out, OUDJAT_ERR_INVALID_ARGUMENT, "patch_attention_prob: null pointer");
  OUDJAT_REQUIRE(q_row_stride >= H * Dh && kv_stride_h >= Dh && out_stride_b >= N, OUDJAT_ERR_UNSUPPORTED_LAYOUT,
                 "patch_attention_prob: strides");
  OUDJAT_REQUIRE(aligned(q, 16) && aligned(kv, 16) && q_row_stride % 8 == 0 && kv_stride_b % 8 == 0 &&
                     kv_stride_n % 8 == 0 && kv_stride_h % 8 == 0,
                 OUDJAT_ERR_UNSUPPORTED_LAYOUT, "patch_attention_prob: 16-byte aligned rows required");
  OUDJAT_REQUIRE(N < (1 << 24) && H < 65536 && B < 65536, OUDJAT_ERR_TOO_LARGE, "patch_attention_prob: too large");
  const hipStream_t st = as_stream(stream);
  const int b = (int)B, n = (int)N, h = (int)H;
  if (Dh == 64) {
    if (mode == kDense) launch_pattn<64, kDense>(q, q_row_stride, kv, kv_stride_b, kv_stride_n, kv_stride_h, b, n, h, scale, workspace, out, out_stride_b, st);
    else launch_pattn<64, kLse>(q, q_row_stride, kv, kv_stride_b, kv_stride_n, kv_stride_h, b, n, h, scale, workspace, out, out_stride_b, st);
  } else {
    if (mode == kDense) launch_pattn<128, kDense>(q, q_row_stride, kv, kv_stride_b, kv_stride_n, kv_stride_h, b, n, h, scale, workspace, out, out_stride_b, st);
    else launch_pattn<128, kLse>(q, q_row_stride, kv, kv_stride_b, kv_stride_n, kv_stride_h, b, n, h, scale, workspace, out, out_stride_b, st);
  }
  return check_launch("patch_attention_prob");
}
