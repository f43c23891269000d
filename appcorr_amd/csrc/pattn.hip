// Dense server score of the approximate pass: the mean attention probability each key receives, over
// heads and all queries (patch_attn_prob / patch_attn_prob_layermean).
//
// Nothing of size N x N is materialised:
//   stats:  for every (image, head, query) the softmax max m and sum l over all keys (two passes over
//           the keys, so that every term exp(s - m) uses the final max, as a row softmax does);
//   colsum: dense mode, for every (image, 128-query block, 128-key block) the column sums over its
//           queries of the head-mean probabilities, then the query blocks added in order; log-sum-exp
//           mode, one pass per (256-key block, head group, image) from the row LSE (the stats launch's,
//           or the attention's own), then the head groups added in order.
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

enum { kDense = 0, kLse = 1 };

// A 16-byte operand fragment of row `row` (< rows, else zeros) at head-dim offset `d0`.
__device__ __forceinline__ bf16x8_t frag16(const uint16_t* base, int64_t row_stride, int row, int rows, int d0) {
  uint4 v = make_uint4(0, 0, 0, 0);
  if (row < rows) v = *reinterpret_cast<const uint4*>(base + (int64_t)row * row_stride + d0);
  return as_bf16x8(v);
}

// Two values rounded to bf16 (nearest even) and back to fp32 with one hardware convert.
__device__ __forceinline__ void round2_bf16(float& a, float& b) {
  typedef float f32x2v_t __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2v_t __attribute__((ext_vector_type(2)));
  const uint32_t p = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2v_t){a, b}, bf16x2v_t));
  a = __uint_as_float(p << 16);
  b = __uint_as_float(p & 0xffff0000u);
}

// The scores of one 32 x 32 MFMA block in place: dense s = bf16(bf16(q.k) * scale), log-sum-exp mode
// s = (q.k) * scale.
template <int MODE>
__device__ __forceinline__ void block_scores(f32x16_t& acc, float scale) {
#pragma unroll
  for (int v = 0; v < 16; v += 2) {
    float a = acc[v], c = acc[v + 1];
    if (MODE == kDense) {
      round2_bf16(a, c);
      a *= scale;
      c *= scale;
      round2_bf16(a, c);
    } else {
      a *= scale;
      c *= scale;
    }
    acc[v] = a;
    acc[v + 1] = c;
  }
}

// Row statistics: workgroup = (256 queries = 8 waves x 32, head, image). Key tiles of 64 (two 32-key
// MFMA blocks) are staged once in LDS for all waves, double-buffered through registers (16-byte chunks
// XOR-swizzled by row); S^T = K . Q^T puts a query's scores in one lane pair (lanes l, l ^ 32). Two
// passes over the keys, the max and then the sum of exp(s - max) with the final max, as a row softmax
// computes them. Waves whose queries lie past N still stage tiles and meet every barrier.
static constexpr int kStWaves = 8;
static constexpr int kStKeys = 64;

template <int DH, int MODE>
__global__ __launch_bounds__(kStWaves * 64) void pattn_stats_kernel(const uint16_t* __restrict__ q, int64_t qrs,
                                                                    const uint16_t* __restrict__ kv, int64_t kvb,
                                                                    int64_t kvn, int64_t kvh, int N, int H,
                                                                    float scale, float* __restrict__ m_out,
                                                                    float* __restrict__ l_out) {
  constexpr int KS = DH / 16;
  constexpr int CPR = DH / 8;
  constexpr int CHUNKS = kStKeys * CPR;
  constexpr int NT = kStWaves * 64;
  constexpr int IT = CHUNKS / NT;
  static_assert(CHUNKS % NT == 0, "whole chunks per thread");
  __shared__ __align__(16) unsigned char kt[2][kStKeys * DH * 2];
  const int b = blockIdx.z, h = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, g = lane >> 5;
  const int q0 = (blockIdx.x * kStWaves + wave) * 32;
  const bool active = q0 < N;
  const uint16_t* qb = q + (int64_t)b * N * qrs + (int64_t)h * DH;
  const uint16_t* kb = kv + (int64_t)b * kvb + (int64_t)h * kvh;
  bf16x8_t qf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) qf[ks] = frag16(qb, qrs, q0 + l32, N, ks * 16 + 8 * g);
  const int ntiles = (N + kStKeys - 1) / kStKeys;

  uint4 rk[IT];
  auto load = [&](int t) {
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int c = tid + i * NT;
      const int r = c / CPR, ch = c - r * CPR;
      const int key = t * kStKeys + r;
      rk[i] = make_uint4(0, 0, 0, 0);
      if (key < N) rk[i] = *reinterpret_cast<const uint4*>(kb + (int64_t)key * kvn + ch * 8);
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int c = tid + i * NT;
      const int r = c / CPR, ch = c - r * CPR;
      *reinterpret_cast<uint4*>(&kt[buf][r * DH * 2 + ((ch ^ (r & (CPR - 1))) << 4)]) = rk[i];
    }
  };
  auto scores = [&](int buf, f32x16_t (&acc)[2]) {
#pragma unroll
    for (int kb2 = 0; kb2 < 2; ++kb2) {
      const int r = kb2 * 32 + l32;
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[kb2][v] = 0.0f;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int ch = 2 * ks + g;
        const bf16x8_t kf =
            as_bf16x8(*reinterpret_cast<const uint4*>(&kt[buf][r * DH * 2 + ((ch ^ (r & (CPR - 1))) << 4)]));
        acc[kb2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[ks], acc[kb2], 0, 0, 0);
      }
      block_scores<MODE>(acc[kb2], scale);
    }
  };
  // Keys past N exist only in the last tile: there the scores of those keys become -inf.
  auto mask_tail = [&](int t, f32x16_t (&acc)[2]) {
    if ((t + 1) * kStKeys > N) {
#pragma unroll
      for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
        for (int v = 0; v < 16; ++v)
          if (t * kStKeys + kb2 * 32 + 8 * (v >> 2) + 4 * g + (v & 3) >= N) acc[kb2][v] = -INFINITY;
    }
  };

  float m = -INFINITY;
  load(0);
  store(0);
  __syncthreads();
  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    if (t + 1 < ntiles) load(t + 1);
    if (active) {
      f32x16_t acc[2];
      scores(buf, acc);
      mask_tail(t, acc);
#pragma unroll
      for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
        for (int v = 0; v < 16; ++v) m = fmaxf(m, acc[kb2][v]);
    }
    if (t + 1 < ntiles) store(buf ^ 1);
    __syncthreads();
  }
  m = fmaxf(m, __shfl_xor(m, 32, 64));
  float l = 0.0f;
  load(0);
  store(0);
  __syncthreads();
  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    if (t + 1 < ntiles) load(t + 1);
    if (active) {
      f32x16_t acc[2];
      scores(buf, acc);
      mask_tail(t, acc);
#pragma unroll
      for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
        for (int v = 0; v < 16; ++v) l += expf(acc[kb2][v] - m);
    }
    if (t + 1 < ntiles) store(buf ^ 1);
    __syncthreads();
  }
  l += __shfl_xor(l, 32, 64);
  const int qi = q0 + l32;
  if (active && g == 0 && qi < N) {
    const int64_t o = ((int64_t)b * H + h) * N + qi;
    m_out[o] = MODE == kDense ? m : m + logf(l);  // kLse keeps the row log-sum-exp in m_out
    l_out[o] = l;
  }
}

// Dense key-side score: workgroup = (128-query block, 128-key block, image), 8 waves; wave w takes
// queries 32 (w % 4) .. + 31 and keys 64 (w / 4) .. + 63 of the tile (two 32-key MFMA blocks, S = Q . K^T
// so a key's column sits in one lane pair). For every head the Q and K tiles (128 x DH each, swizzled
// 16-byte chunks) and the 128 queries' row max and sum are staged once in LDS, double-buffered through
// registers; p = bf16(exp(s - m) / l) (the quotient by one correction step from the reciprocal,
// q0 = e r, q = fma(fma(-q0, l, e), r, q0), the correctly rounded quotient for normal results) is
// summed over heads per (query, key) in registers. After the last head each (query, key) takes
// bf16(sum * fl(1/H)); the tile's column sums over its queries (four query waves added in order in
// LDS) go to part[b][query block][key], and pattn_dense_reduce_kernel adds the query blocks in order.
static constexpr int kDnTile = 128;

template <int DH>
__global__ __launch_bounds__(512) void pattn_colsum_kernel(const uint16_t* __restrict__ q, int64_t qrs,
                                                           const uint16_t* __restrict__ kv, int64_t kvb, int64_t kvn,
                                                           int64_t kvh, int N, int H, float scale,
                                                           const float* __restrict__ m_in,
                                                           const float* __restrict__ l_in,
                                                           float* __restrict__ part) {
  constexpr int KS = DH / 16;
  constexpr int CPR = DH / 8;
  constexpr int ROWB = DH * 2;
  constexpr int TILEB = kDnTile * ROWB;
  constexpr int CHUNKS = 2 * kDnTile * CPR;  // Q and K chunks of one head
  constexpr int NT = 512;
  constexpr int IT = CHUNKS / NT;
  static_assert(CHUNKS % NT == 0, "whole chunks per thread");
  __shared__ __align__(16) unsigned char tiles[2][2 * TILEB];
  __shared__ __align__(16) float st[2][3][kDnTile];  // row max, row sum, 1 / row sum
  __shared__ float colp[4][kDnTile];
  const int b = blockIdx.z;
  const int qt0 = blockIdx.y * kDnTile, kt0 = blockIdx.x * kDnTile;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, g = lane >> 5;
  const int wq = 32 * (wave & 3), wk = 64 * (wave >> 2);
  const uint16_t* qimg = q + (int64_t)b * N * qrs;
  const uint16_t* kimg = kv + (int64_t)b * kvb;

  uint4 rq[IT];
  float rs = 0.0f;
  auto load = [&](int h) {
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int c = tid + i * NT;
      const int isk = c >= kDnTile * CPR;
      const int cc = c - isk * kDnTile * CPR;
      const int r = cc / CPR, ch = cc - r * CPR;
      rq[i] = make_uint4(0, 0, 0, 0);
      if (isk) {
        if (kt0 + r < N)
          rq[i] = *reinterpret_cast<const uint4*>(kimg + (int64_t)(kt0 + r) * kvn + (int64_t)h * kvh + ch * 8);
      } else if (qt0 + r < N) {
        rq[i] = *reinterpret_cast<const uint4*>(qimg + (int64_t)(qt0 + r) * qrs + (int64_t)h * DH + ch * 8);
      }
    }
    if (tid < 2 * kDnTile) {
      const int r = tid & (kDnTile - 1);
      const float* src = tid < kDnTile ? m_in : l_in;
      rs = qt0 + r < N ? src[((int64_t)b * H + h) * N + qt0 + r] : (tid < kDnTile ? 0.0f : 1.0f);
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int c = tid + i * NT;
      const int isk = c >= kDnTile * CPR;
      const int cc = c - isk * kDnTile * CPR;
      const int r = cc / CPR, ch = cc - r * CPR;
      *reinterpret_cast<uint4*>(&tiles[buf][isk * TILEB + r * ROWB + ((ch ^ (r & (CPR - 1))) << 4)]) = rq[i];
    }
    if (tid < kDnTile) {
      st[buf][0][tid] = rs;
    } else if (tid < 2 * kDnTile) {
      st[buf][1][tid - kDnTile] = rs;
      st[buf][2][tid - kDnTile] = 1.0f / rs;
    }
  };

  float hs[2][16];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int v = 0; v < 16; ++v) hs[j][v] = 0.0f;

  load(0);
  store(0);
  __syncthreads();
  for (int h = 0; h < H; ++h) {
    const int buf = h & 1;
    if (h + 1 < H) load(h + 1);
    const unsigned char* qs = tiles[buf];
    const unsigned char* ks = tiles[buf] + TILEB;
    f32x16_t acc[2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[j][v] = 0.0f;
#pragma unroll
    for (int kstep = 0; kstep < KS; ++kstep) {
      const int ch = 2 * kstep + g;
      const int rq_ = wq + l32;
      const bf16x8_t qf = as_bf16x8(*reinterpret_cast<const uint4*>(qs + rq_ * ROWB + ((ch ^ (rq_ & (CPR - 1))) << 4)));
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int rk_ = wk + 32 * j + l32;
        const bf16x8_t kf =
            as_bf16x8(*reinterpret_cast<const uint4*>(ks + rk_ * ROWB + ((ch ^ (rk_ & (CPR - 1))) << 4)));
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qf, kf, acc[j], 0, 0, 0);
      }
    }
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const int r0 = wq + 8 * a + 4 * g;
      const float4 m4 = *reinterpret_cast<const float4*>(&st[buf][0][r0]);
      const float4 l4 = *reinterpret_cast<const float4*>(&st[buf][1][r0]);
      const float4 i4 = *reinterpret_cast<const float4*>(&st[buf][2][r0]);
      const float mm[4] = {m4.x, m4.y, m4.z, m4.w};
      const float ll[4] = {l4.x, l4.y, l4.z, l4.w};
      const float ii[4] = {i4.x, i4.y, i4.z, i4.w};
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        float sv[4];
#pragma unroll
        for (int e = 0; e < 4; e += 2) {
          float x0 = acc[j][4 * a + e], x1 = acc[j][4 * a + e + 1];
          round2_bf16(x0, x1);
          x0 *= scale;
          x1 *= scale;
          round2_bf16(x0, x1);
          sv[e] = x0;
          sv[e + 1] = x1;
        }
        float pv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float ex = expf(sv[e] - mm[e]);
          const float q0 = ex * ii[e];
          pv[e] = fmaf(fmaf(-q0, ll[e], ex), ii[e], q0);
        }
        round2_bf16(pv[0], pv[1]);
        round2_bf16(pv[2], pv[3]);
#pragma unroll
        for (int e = 0; e < 4; ++e) hs[j][4 * a + e] += pv[e];
      }
    }
    if (h + 1 < H) store(buf ^ 1);
    __syncthreads();
  }
  // bf16 head means of the valid queries, summed over this wave's queries per key.
  const float inv_h = 1.0f / (float)H;
  float col[2] = {0.0f, 0.0f};
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int qi = qt0 + wq + 8 * (v >> 2) + 4 * g + (v & 3);
      if (qi < N) col[j] += round_bf16(hs[j][v] * inv_h);
    }
#pragma unroll
  for (int j = 0; j < 2; ++j) col[j] += __shfl_xor(col[j], 32, 64);
  if (g == 0) {
    colp[wave & 3][wk + l32] = col[0];
    colp[wave & 3][wk + 32 + l32] = col[1];
  }
  __syncthreads();
  if (tid < kDnTile && kt0 + tid < N) {
    const float t = ((colp[0][tid] + colp[1][tid]) + colp[2][tid]) + colp[3][tid];
    part[((int64_t)b * gridDim.y + blockIdx.y) * N + kt0 + tid] = t;
  }
}

// out[b, n] = bf16(fl(sum_qb part[b][qb][n]) * fl(1/N)), query blocks added in order.
__global__ void pattn_dense_reduce_kernel(const float* __restrict__ part, int B, int N, int nqb,
                                          uint16_t* __restrict__ out, int64_t osb) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)B * N) return;
  const int b = (int)(i / N), n = (int)(i - (int64_t)b * N);
  const float* p = part + (int64_t)b * nqb * N + n;
  float t = 0.0f;
  for (int qb = 0; qb < nqb; ++qb) t += p[(int64_t)qb * N];
  out[(int64_t)b * osb + n] = (uint16_t)f32_to_bf16(t * (1.0f / (float)N));
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
  const dim3 g1((unsigned)cdiv(N, 32 * kStWaves), (unsigned)H, (unsigned)B);
  pattn_stats_kernel<DH, MODE><<<g1, kStWaves * 64, 0, st>>>(q, qrs, kv, kvb, kvn, kvh, N, H, scale, m, l);
  if constexpr (MODE == kLse) {
    // m holds the row log-sum-exp; l (no longer read) takes the partial column sums.
    launch_colsum_lse<DH>(q, qrs, kv, kvb, kvn, kvh, B, N, H, scale, m, l, out, osb, st);
  } else {
    // Partial column sums per 128-query block after the statistics.
    float* part = ws + 2 * (int64_t)B * H * N;
    const int nqb = (int)cdiv(N, kDnTile);
    const dim3 g2((unsigned)cdiv(N, kDnTile), (unsigned)nqb, (unsigned)B);
    pattn_colsum_kernel<DH><<<g2, 512, 0, st>>>(q, qrs, kv, kvb, kvn, kvh, N, H, scale, m, l, part);
    const int64_t n = (int64_t)B * N;
    pattn_dense_reduce_kernel<<<(unsigned)cdiv(n, 256), 256, 0, st>>>(part, B, N, nqb, out, osb);
  }
}

}  // namespace oudjat

using namespace oudjat;

extern "C" int64_t oudjat_patch_attention_prob_workspace_elems(int64_t B, int64_t N, int64_t H, int mode) {
  if (B <= 0 || N <= 0 || H <= 0) return 0;
  // row statistics (max or log-sum-exp, sum), then the dense mode's per-query-block column sums (the
  // log-sum-exp mode's per-head-group sums reuse the second array)
  return 2 * B * H * N + (mode == kDense ? B * cdiv(N, kDnTile) * N : 0);
}

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
