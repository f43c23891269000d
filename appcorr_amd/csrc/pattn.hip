// Dense server score of the approximate pass: the mean attention probability each key receives, over
// heads and all queries (patch_attn_prob / patch_attn_prob_layermean).
//
// Nothing of size N x N is materialised:
//   stats:  for every (image, head, query) the softmax max m and sum l over all keys (two passes over
//           the keys, so that every term exp(s - m) uses the final max, as a row softmax does);
//   colsum: dense mode, for every (image, 32-key block) the column sums of the probabilities over all
//           queries and heads; four waves split the query blocks, their partial sums meet in LDS in a
//           fixed order. Log-sum-exp mode: one pass per (256-key block, head group, image) from the row
//           LSE (the stats launch's, or the attention's own), then the head groups added in order.
//
// Rounding modes (the two paths of attention.py:241-253 and triton_kernels/attention_pscore.py):
//   kDense: s = bf16(bf16(q.k) * scale), p = bf16(exp(s - m) / l) (torch softmax of a bf16 tensor),
//           head mean hm = bf16(sum_h p * fl(1/H)), score = bf16(sum_q hm * fl(1/N));
//   kLse:   s = (q.k) in fp32, lse = m + log(l), p = exp2(s * (scale log2e) - lse * log2e) in fp32,
//           score = bf16(sum_{q,h} p * fl(1/(H N))) -- the fused kernel's key-side sum from the row
//           log-sum-exp.
// q.k is one v_mfma_f32_32x32x16_bf16 chain (fp32 accumulation). Stats use S^T = K . Q^T so a query's
// scores sit in one lane pair (lanes l, l ^ 32); colsum uses S = Q . K^T so a key's column sits in one
// lane pair and the sum over queries is a register sum plus one exchange.
#include <algorithm>
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

// Dense mode: workgroup = (32-key block, image); the head sum of each (query, key) is rounded before the
// query sum, so the loop runs heads inside query blocks.
template <int DH>
__global__ __launch_bounds__(kPaThreads) void pattn_colsum_kernel(const uint16_t* __restrict__ q, int64_t qrs,
                                                                  const uint16_t* __restrict__ kv, int64_t kvb,
                                                                  int64_t kvn, int64_t kvh, int N, int H, float scale,
                                                                  const float* __restrict__ m_in,
                                                                  const float* __restrict__ l_in,
                                                                  uint16_t* __restrict__ out, int64_t osb) {
  constexpr int KS = DH / 16;
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
          const float s = round_bf16(round_bf16(acc[v]) * scale);
          hs[v] += round_bf16(expf(s - mrow[qi]) / lrow[qi]);
        }
      }
    }
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int qi = q0 + 8 * (v >> 2) + 4 * g + (v & 3);
      if (qi < N) col += round_bf16(hs[v] * inv_h);
    }
  }
  col += __shfl_xor(col, 32, 64);
  if (g == 0) part[wave][l32] = col;
  __syncthreads();
  if (wave == 0 && g == 0) {
    float t = part[0][l32];
#pragma unroll
    for (int w = 1; w < kPaWaves; ++w) t += part[w][l32];
    const float factor = 1.0f / (float)N;
    const int key = k0 + l32;
    if (key < N) out[(int64_t)b * osb + key] = (uint16_t)f32_to_bf16(t * factor);
  }
}

// Key-side score from the row log-sum-exp (mode kLse), one pass over the scores. Workgroup = (block
// of 256 keys, group of `hpg` heads, image), 8 waves of 32 keys each. For every (head, 32-query block)
// the query tile (32 x DH bf16, 16-byte chunks XOR-swizzled by row so that 16 consecutive rows read at
// one chunk cover all banks) and its 32 row LSEs (times log2 e; +inf past N) are staged once in LDS
// for all waves, double-buffered through registers; each wave keeps its keys' K fragments of the
// current head in registers, forms S = Q . K^T on v_mfma_f32_32x32x16_bf16 (a key's column in one
// lane pair) and adds exp2(s * scale log2 e - lse log2 e) over its queries in fp32 registers. Keys and
// queries past N read as zeros; their terms never reach a stored column. Partial column sums per head
// group -> part[b][group][n]; pattn_lse_reduce_kernel adds the groups in order.
static constexpr int kLseWaves = 8;
static constexpr int kLseKeys = 32 * kLseWaves;

template <int DH>
__global__ __launch_bounds__(kLseWaves * 64) void pattn_colsum_lse_kernel(
    const uint16_t* __restrict__ q, int64_t qrs, const uint16_t* __restrict__ kv, int64_t kvb, int64_t kvn,
    int64_t kvh, int N, int H, int hpg, float scale_log2, const float* __restrict__ lse, float* __restrict__ part) {
  constexpr int KS = DH / 16;          // 16-deep MFMA steps
  constexpr int CPR = DH / 8;          // 16-byte chunks per query row
  constexpr int CHUNKS = 32 * CPR;     // chunks per query tile
  constexpr int NT = kLseWaves * 64;
  constexpr int IT = (CHUNKS + NT - 1) / NT;
  constexpr float kLog2e = 1.4426950408889634f;
  __shared__ __align__(16) unsigned char qs[2][32 * DH * 2];
  __shared__ __align__(16) float ls[2][32];
  const int b = blockIdx.z, grp = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, g = lane >> 5;
  const int key = blockIdx.x * kLseKeys + wave * 32 + l32;
  const int nqb = (N + 31) / 32;
  const int h0 = grp * hpg;
  const int nh = min(H - h0, hpg);
  const int steps = nh * nqb;
  const uint16_t* qimg = q + (int64_t)b * N * qrs;
  const float* limg = lse + (int64_t)b * H * N;

  uint4 rq[IT];
  float rl = INFINITY;
  auto load = [&](int st) {
    const int h = h0 + st / nqb, q0 = (st % nqb) * 32;
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int c = tid + i * NT;
      rq[i] = make_uint4(0, 0, 0, 0);
      if (c < CHUNKS) {
        const int r = c / CPR, ch = c - r * CPR;
        if (q0 + r < N) rq[i] = *reinterpret_cast<const uint4*>(qimg + (int64_t)(q0 + r) * qrs + (int64_t)h * DH + ch * 8);
      }
    }
    if (tid < 32) rl = q0 + tid < N ? limg[(int64_t)h * N + q0 + tid] * kLog2e : INFINITY;
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int c = tid + i * NT;
      if (c < CHUNKS) {
        const int r = c / CPR, ch = c - r * CPR;
        *reinterpret_cast<uint4*>(&qs[buf][r * DH * 2 + ((ch ^ (r & (CPR - 1))) << 4)]) = rq[i];
      }
    }
    if (tid < 32) ls[buf][tid] = rl;
  };

  bf16x8_t kf[KS];
  auto load_k = [&](int h) {
    const uint16_t* kb = kv + (int64_t)b * kvb + (int64_t)h * kvh;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      uint4 v = make_uint4(0, 0, 0, 0);
      if (key < N) v = *reinterpret_cast<const uint4*>(kb + (int64_t)key * kvn + ks * 16 + 8 * g);
      kf[ks] = as_bf16x8(v);
    }
  };

  float col = 0.0f;
  if (steps > 0) {
    load(0);
    store(0);
  }
  __syncthreads();
  for (int st = 0; st < steps; ++st) {
    const int buf = st & 1;
    if (st % nqb == 0) load_k(h0 + st / nqb);
    if (st + 1 < steps) load(st + 1);
    const unsigned char* qt = qs[buf];
    f32x16_t acc;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int ch = 2 * ks + g;
      const bf16x8_t qf = as_bf16x8(*reinterpret_cast<const uint4*>(qt + l32 * DH * 2 + ((ch ^ (l32 & (CPR - 1))) << 4)));
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qf, kf[ks], acc, 0, 0, 0);
    }
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const float4 l4 = *reinterpret_cast<const float4*>(&ls[buf][8 * a + 4 * g]);
      col += __builtin_amdgcn_exp2f(fmaf(acc[4 * a + 0], scale_log2, -l4.x));
      col += __builtin_amdgcn_exp2f(fmaf(acc[4 * a + 1], scale_log2, -l4.y));
      col += __builtin_amdgcn_exp2f(fmaf(acc[4 * a + 2], scale_log2, -l4.z));
      col += __builtin_amdgcn_exp2f(fmaf(acc[4 * a + 3], scale_log2, -l4.w));
    }
    if (st + 1 < steps) store(buf ^ 1);
    __syncthreads();
  }
  col += __shfl_xor(col, 32, 64);
  if (g == 0 && key < N) part[((int64_t)b * gridDim.y + grp) * N + key] = col;
}

// out[b, n] = bf16(fl(sum_group part[b][group][n]) * factor), groups added in order.
__global__ void pattn_lse_reduce_kernel(const float* __restrict__ part, int B, int N, int groups, float factor,
                                        uint16_t* __restrict__ out, int64_t osb) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)B * N) return;
  const int b = (int)(i / N), n = (int)(i - (int64_t)b * N);
  const float* p = part + (int64_t)b * groups * N + n;
  float t = 0.0f;
  for (int gi = 0; gi < groups; ++gi) t += p[(int64_t)gi * N];
  out[(int64_t)b * osb + n] = (uint16_t)f32_to_bf16(t * factor);
}

// Heads per group of the one-pass LSE kernel: enough groups that the grid holds about 512 workgroups.
static int lse_heads_per_group(int B, int N, int H) {
  const int kblocks = (N + kLseKeys - 1) / kLseKeys;
  const int want = (int)std::min<int64_t>(H, std::max<int64_t>(1, cdiv(512, (int64_t)kblocks * B)));
  return (H + want - 1) / want;
}

// The one-pass key-side score from lse [B, H, N] (natural log) into out, through part (B * H * N fp32
// at most: B * groups * N used).
template <int DH>
void launch_colsum_lse(const uint16_t* q, int64_t qrs, const uint16_t* kv, int64_t kvb, int64_t kvn, int64_t kvh,
                       int B, int N, int H, float scale, const float* lse, float* part, uint16_t* out, int64_t osb,
                       hipStream_t st) {
  constexpr float kLog2e = 1.4426950408889634f;
  const int hpg = lse_heads_per_group(B, N, H);
  const int groups = (H + hpg - 1) / hpg;
  const dim3 g1((unsigned)cdiv(N, kLseKeys), (unsigned)groups, (unsigned)B);
  pattn_colsum_lse_kernel<DH><<<g1, kLseWaves * 64, 0, st>>>(q, qrs, kv, kvb, kvn, kvh, N, H, hpg, scale * kLog2e,
                                                              lse, part);
  const int64_t n = (int64_t)B * N;
  pattn_lse_reduce_kernel<<<(unsigned)cdiv(n, 256), 256, 0, st>>>(part, B, N, groups,
                                                                  1.0f / (float)((int64_t)H * N), out, osb);
}

template <int DH, int MODE>
void launch_pattn(const uint16_t* q, int64_t qrs, const uint16_t* kv, int64_t kvb, int64_t kvn, int64_t kvh, int B,
                  int N, int H, float scale, float* ws, uint16_t* out, int64_t osb, hipStream_t st) {
  float* m = ws;
  float* l = ws + (int64_t)B * H * N;
  const dim3 g1((unsigned)cdiv(cdiv(N, 32), kPaWaves), (unsigned)H, (unsigned)B);
  pattn_stats_kernel<DH, MODE><<<g1, kPaThreads, 0, st>>>(q, qrs, kv, kvb, kvn, kvh, N, H, scale, m, l);
  if constexpr (MODE == kLse) {
    // m holds the row log-sum-exp; l (no longer read) takes the partial column sums.
    launch_colsum_lse<DH>(q, qrs, kv, kvb, kvn, kvh, B, N, H, scale, m, l, out, osb, st);
  } else {
    const dim3 g2((unsigned)cdiv(N, 32), (unsigned)B);
    pattn_colsum_kernel<DH><<<g2, kPaThreads, 0, st>>>(q, qrs, kv, kvb, kvn, kvh, N, H, scale, m, l, out, osb);
  }
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

extern "C" int oudjat_patch_attention_prob_lse(const uint16_t* q, int64_t q_row_stride, int64_t B, int64_t N,
                                               int64_t H, int64_t Dh, const uint16_t* kv, int64_t kv_stride_b,
                                               int64_t kv_stride_n, int64_t kv_stride_h, float scale, const float* lse,
                                               float* workspace, uint16_t* out, int64_t out_stride_b,
                                               oudjat_stream_t stream) {
  OUDJAT_REQUIRE(B >= 0 && N >= 0 && H > 0, OUDJAT_ERR_INVALID_ARGUMENT, "patch_attention_prob_lse: bad size");
  OUDJAT_REQUIRE(Dh == 64 || Dh == 128, OUDJAT_ERR_UNSUPPORTED_SHAPE, "patch_attention_prob_lse: Dh=%lld (64 or 128)",
                 (long long)Dh);
  if (B == 0 || N == 0) return OUDJAT_OK;
  OUDJAT_REQUIRE(q && kv && lse && workspace && out, OUDJAT_ERR_INVALID_ARGUMENT,
                 "patch_attention_prob_lse: null pointer");
  OUDJAT_REQUIRE(q_row_stride >= H * Dh && kv_stride_h >= Dh && out_stride_b >= N, OUDJAT_ERR_UNSUPPORTED_LAYOUT,
                 "patch_attention_prob_lse: strides");
  OUDJAT_REQUIRE(aligned(q, 16) && aligned(kv, 16) && aligned(lse, 4) && aligned(workspace, 4) &&
                     q_row_stride % 8 == 0 && kv_stride_b % 8 == 0 && kv_stride_n % 8 == 0 && kv_stride_h % 8 == 0,
                 OUDJAT_ERR_UNSUPPORTED_LAYOUT, "patch_attention_prob_lse: 16-byte aligned rows required");
  OUDJAT_REQUIRE(N < (1 << 24) && H < 65536 && B < 65536, OUDJAT_ERR_TOO_LARGE, "patch_attention_prob_lse: too large");
  const hipStream_t st = as_stream(stream);
  const int b = (int)B, n = (int)N, h = (int)H;
  if (Dh == 64)
    launch_colsum_lse<64>(q, q_row_stride, kv, kv_stride_b, kv_stride_n, kv_stride_h, b, n, h, scale, lse, workspace,
                          out, out_stride_b, st);
  else
    launch_colsum_lse<128>(q, q_row_stride, kv, kv_stride_b, kv_stride_n, kv_stride_h, b, n, h, scale, lse, workspace,
                           out, out_stride_b, st);
  return check_launch("patch_attention_prob_lse");
}
