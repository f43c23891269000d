// LayerNorm over selected rows, rotate-half RoPE on the active rows, and the fused post-QKV step
// (RoPE + in-place K/V cache rewrite + packed query write).
#include <type_traits>

#include "nvfp4.hpp"

namespace oudjat {

static constexpr int kNormThreads = 256;
static constexpr int kNormRowsPerWg = kNormThreads / 64;

// Waves per LayerNorm row (see layernorm_row): 1 up to C = 1024; 2 up to 2048 and 4 up to 8192 when
// the row's 16-byte chunks split into that many equal, even parts (an NVFP4 block of 16 elements is
// two chunks and must stay in one wave); 1 otherwise. A workgroup holds kNormRowsPerWg / parts rows.
static int row_parts(int64_t C) {
  const int64_t chunks = C / 8;
  if (C <= 1024) return 1;
  const int n = C <= 2048 ? 2 : 4;
  return chunks % (2 * n) == 0 ? n : 1;
}

// LayerNorm of one row held by one wave: lane l holds chunks l + 64 j (j < CH, 8 values each, as
// fp32 from bf16). Statistics are fp32: mean, then the biased variance around it. Shared by the
// standalone kernel and the fused residual kernel so both give the same bits.
// xh_ts (NULL: plain LayerNorm): the row written is instead the NVFP4 operand x_hat of the bf16
// LayerNorm output with tensor scale *xh_ts -- what nvfp4_quantize_dequantize gives on the output
// (a 16-element block is the chunk pair of lanes l, l ^ 1). The LayerNorm values themselves are the
// same either way.
//
// Rows wider than 1024 are split over NWR = 2 or 4 waves of one workgroup (row_parts): each wave holds
// an equal, even number of the row's chunks (`chunks` and the w / bias / out_row pointers are then
// its part's), the two row sums combine the waves' sums in wave order through `red` (LDS,
// 2 * kNormRowsPerWg floats: NWR per row slot `slot` for each sum), and a row past the end (`live` false) still takes part in
// the workgroup barriers but stores nothing. NWR = 1 is the one-wave row above.
template <int NWR>
__device__ __forceinline__ float row_parts_sum(float s, float* red, int slot, int part, int lane) {
  if constexpr (NWR == 1) {
    return s;
  } else {
    if (lane == 0) red[slot * NWR + part] = s;
    __syncthreads();
    float t = red[slot * NWR];
#pragma unroll
    for (int i = 1; i < NWR; ++i) t += red[slot * NWR + i];
    return t;
  }
}

template <int CH, int NWR = 1>
__device__ __forceinline__ void layernorm_row(const float (&v)[CH][8], int lane, int chunks, int C,
                                              const uint16_t* __restrict__ w, const uint16_t* __restrict__ bias,
                                              float eps, uint16_t* __restrict__ out_row,
                                              const float* __restrict__ xh_ts = nullptr, float* red = nullptr,
                                              int slot = 0, int part = 0, bool live = true) {
  float sum = 0.0f;
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    const int c = lane + 64 * j;
    if (c < chunks) {
#pragma unroll
      for (int e = 0; e < 8; ++e) sum += v[j][e];
    }
  }
  const float mean = row_parts_sum<NWR>(wave_sum(sum), red, slot, part, lane) / (float)C;
  float sq = 0.0f;
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    const int c = lane + 64 * j;
    if (c < chunks) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float dlt = v[j][e] - mean;
        sq = fmaf(dlt, dlt, sq);
      }
    }
  }
  // (a second set of slots: no barrier needed between the two sums)
  const float var = row_parts_sum<NWR>(wave_sum(sq), red + kNormRowsPerWg, slot, part, lane) / (float)C;
  const float rstd = 1.0f / sqrtf(var + eps);
  const uint4* wv = reinterpret_cast<const uint4*>(w);
  const uint4* bv = reinterpret_cast<const uint4*>(bias);
  uint4* ov = reinterpret_cast<uint4*>(out_row);
  if (xh_ts == nullptr) {
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int c = lane + 64 * j;
      if (c < chunks) {
        float fw[8], fb[8], y[8];
        unpack8(wv[c], fw);
        unpack8(bv[c], fb);
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = fmaf(fw[e], (v[j][e] - mean) * rstd, fb[e]);
        if (live) ov[c] = pack8(y);
      }
    }
    return;
  }
  const float ts = *xh_ts;
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    const int c = lane + 64 * j;
    float y[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    if (c < chunks) {
      float fw[8], fb[8];
      unpack8(wv[c], fw);
      unpack8(bv[c], fb);
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = fmaf(fw[e], (v[j][e] - mean) * rstd, fb[e]);
      unpack8(pack8(y), y);  // the bf16 LayerNorm output the quantizer reads
    }
    float h[8];
    nvfp4_xhat8_pair(y, ts, h);  // every lane takes part (the block maximum is a lane-pair exchange)
    if (live && c < chunks) ov[c] = pack8(h);
  }
}

// One wave per row (NWR waves for rows wider than 1024: layernorm_row); each lane keeps its CH 16-byte
// chunks (8 bf16 each) in registers, so the row is read from HBM exactly once.
// PF: the launch also reads one 32-bit word of every 128-byte line of the region [pf, pf + 128 pf_lines)
// (a lane per line, the lines dealt over all waves of the grid, issued beside the row loads), so that
// the region sits in the last-level cache when the kernels after this one read it: the weights of a
// linear that follows, whose first-touch misses would otherwise go to HBM. The words are folded into
// a register that an empty asm statement consumes (nothing is stored); the output is the same bits.
template <int CH, int NWR, bool PF = false>
__global__ __launch_bounds__(kNormThreads) void layernorm_kernel(const uint16_t* __restrict__ x, int64_t rows, int C,
                                                               int64_t xs, const uint16_t* __restrict__ w,
                                                               const uint16_t* __restrict__ bias, float eps,
                                                               uint16_t* __restrict__ out, int64_t os,
                                                               const float* __restrict__ xh_ts,
                                                               const uint32_t* __restrict__ pf = nullptr,
                                                               int64_t pf_lines = 0) {
  __shared__ float red[2 * kNormRowsPerWg];
  const int wave = threadIdx.x >> 6, slot = wave / NWR, part = wave % NWR;
  const int64_t row = (int64_t)blockIdx.x * (kNormRowsPerWg / NWR) + slot;
  if (NWR == 1 && !PF && row >= rows) return;
  const bool live = row < rows;
  const int lane = threadIdx.x & 63;
  const int chunks = (C >> 3) / NWR;  // this wave's part of the row
  const int c0 = part * chunks * 8;   // its first column
  // Every load of the lane is issued before the first use (one memory round trip per wave).
  uint4 raw[CH];
#pragma unroll
  for (int j = 0; j < CH; ++j) raw[j] = make_uint4(0u, 0u, 0u, 0u);
  if (live) {
    const uint4* xv = reinterpret_cast<const uint4*>(x + row * xs + c0);
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int c = lane + 64 * j;
      if (c < chunks) raw[j] = xv[c];
    }
  }
  uint32_t touched = 0;
  const int64_t l0 = (int64_t)blockIdx.x * kNormThreads + threadIdx.x;
  if (PF && l0 < pf_lines) touched = pf[l0 * 32];
  if (NWR > 1 || live) {
    float v[CH][8];
#pragma unroll
    for (int j = 0; j < CH; ++j) unpack8(raw[j], v[j]);
    layernorm_row<CH, NWR>(v, lane, chunks, C, w + c0, bias + c0, eps, out + (live ? row : 0) * os + c0, xh_ts, red,
                           slot, part, live);
  }
  if constexpr (PF) {
    // Regions of more lines than the grid has lanes: the rest after the row's work.
    const int64_t lanes = (int64_t)gridDim.x * kNormThreads;
    for (int64_t l = l0 + lanes; l < pf_lines; l += lanes) touched ^= pf[l * 32];
    asm volatile("" ::"v"(touched));
  }
}

// The gather of a packed run's selected rows fused with the first block's LayerNorm: packed row i is
// x[batch_idx[i], token_idx[i]], copied byte for byte to x_out, and its LayerNorm (or the NVFP4 operand
// of it) goes to ln_out with layernorm_kernel's arithmetic (the same bits).
template <int CH, int NWR>
__global__ __launch_bounds__(kNormThreads) void gather_ln_kernel(const uint16_t* __restrict__ x, int64_t sb,
                                                                int64_t sn, const int64_t* __restrict__ bidx,
                                                                const int64_t* __restrict__ tidx, int64_t rows, int C,
                                                                const uint16_t* __restrict__ w,
                                                                const uint16_t* __restrict__ bias, float eps,
                                                                uint16_t* __restrict__ x_out,
                                                                uint16_t* __restrict__ ln_out,
                                                                const float* __restrict__ xh_ts) {
  __shared__ float red[2 * kNormRowsPerWg];
  const int wave = threadIdx.x >> 6, slot = wave / NWR, part = wave % NWR;
  const int64_t row = (int64_t)blockIdx.x * (kNormRowsPerWg / NWR) + slot;
  if (NWR == 1 && row >= rows) return;
  const bool live = row < rows;
  const int lane = threadIdx.x & 63;
  const int chunks = (C >> 3) / NWR;
  const int c0 = part * chunks * 8;
  const int64_t r = live ? row : 0;
  uint4 raw[CH];
#pragma unroll
  for (int j = 0; j < CH; ++j) raw[j] = make_uint4(0u, 0u, 0u, 0u);
  uint4* ov = reinterpret_cast<uint4*>(x_out + r * C + c0);
  if (live) {
    const uint4* xv = reinterpret_cast<const uint4*>(x + bidx[row] * sb + tidx[row] * sn + c0);
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int c = lane + 64 * j;
      if (c < chunks) raw[j] = xv[c];
    }
  }
  float v[CH][8];
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    const int c = lane + 64 * j;
    if (live && c < chunks) ov[c] = raw[j];
    unpack8(raw[j], v[j]);
  }
  layernorm_row<CH, NWR>(v, lane, chunks, C, w + c0, bias + c0, eps, ln_out + r * C + c0, xh_ts, red, slot, part,
                         live);
}

// The residual step of a correction block on packed selected rows fused with the next block's
// LayerNorm: x_new = bf16(x_attn + mlp), blocks_out_sum[b_i, t_i] = bf16(bf16(x_attn - x_act) + mlp)
// and ln_out = LayerNorm(x_new) (of the bf16 x_new, exactly as the standalone kernel computes it).
template <int CH, int NWR>
__global__ __launch_bounds__(kNormThreads) void packed_residual_ln_kernel(
    const uint16_t* __restrict__ xa, const uint16_t* __restrict__ xt, const uint16_t* __restrict__ mlp, int64_t rows,
    int C, const int64_t* __restrict__ bi, const int64_t* __restrict__ ti, uint16_t* __restrict__ bos, int64_t bsb,
    int64_t bsn, uint16_t* __restrict__ xn, const uint16_t* __restrict__ w, const uint16_t* __restrict__ bias,
    float eps, uint16_t* __restrict__ ln_out, const float* __restrict__ xh_ts) {
  __shared__ float red[2 * kNormRowsPerWg];
  const int wave = threadIdx.x >> 6, slot = wave / NWR, part = wave % NWR;
  const int64_t row = (int64_t)blockIdx.x * (kNormRowsPerWg / NWR) + slot;
  if (NWR == 1 && row >= rows) return;
  const bool live = row < rows;
  const int lane = threadIdx.x & 63;
  const int chunks = (C >> 3) / NWR;
  const int c0 = part * chunks * 8;
  const int64_t r = live ? row : 0;
  const uint4* av = reinterpret_cast<const uint4*>(xa + r * C + c0);
  const uint4* tv = reinterpret_cast<const uint4*>(xt + r * C + c0);
  const uint4* mv = reinterpret_cast<const uint4*>(mlp + r * C + c0);
  uint4* ov = reinterpret_cast<uint4*>(xn + r * C + c0);
  uint4* bv = reinterpret_cast<uint4*>(bos + (live ? bi[row] * bsb + ti[row] * bsn : 0) + c0);
  uint4 ra[CH], rt[CH], rm[CH];  // every load of the lane in flight before the first use
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    const int c = lane + 64 * j;
    if (live && c < chunks) {
      ra[j] = av[c];
      rt[j] = tv[c];
      rm[j] = mv[c];
    } else {
      ra[j] = rt[j] = rm[j] = make_uint4(0u, 0u, 0u, 0u);
    }
  }
  float v[CH][8];
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    const int c = lane + 64 * j;
    float fa[8], ft[8], fm[8], fo[8], fb[8];
    unpack8(ra[j], fa);
    unpack8(rt[j], ft);
    unpack8(rm[j], fm);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      fo[e] = ft[e] + fm[e];
      fb[e] = round_bf16(ft[e] - fa[e]) + fm[e];
    }
    const uint4 o = pack8(fo);
    if (live && c < chunks) {
      ov[c] = o;
      bv[c] = pack8(fb);
    }
    unpack8(o, v[j]);
  }
  layernorm_row<CH, NWR>(v, lane, chunks, C, w + c0, bias + c0, eps, ln_out + r * C + c0, xh_ts, red, slot, part,
                         live);
}

// The split-K reduce of a LayerScale projection (fc2 / w3) fused with the packed residual step and
// the next block's LayerNorm: mlp = bf16(bf16(sum_s P[s] * acc_scale + b) * gamma), the slices summed
// in order from slice 0 (splitk_reduce_kernel's arithmetic), then exactly packed_residual_ln_kernel
// (x_new, the blocks_out_sum row, and LayerNorm(x_new) when w is given). One wave per row.
template <int CH, int NWR>
__global__ __launch_bounds__(kNormThreads) void splitk_ls_residual_ln_kernel(
    const float* __restrict__ P, int S, const uint16_t* __restrict__ fb, const uint16_t* __restrict__ fg,
    float acc_scale, const uint16_t* __restrict__ xa, const uint16_t* __restrict__ xt, int64_t rows, int C,
    const int64_t* __restrict__ bi, const int64_t* __restrict__ ti, uint16_t* __restrict__ bos, int64_t bsb,
    int64_t bsn, uint16_t* __restrict__ xn, const uint16_t* __restrict__ w, const uint16_t* __restrict__ bias,
    float eps, uint16_t* __restrict__ ln_out) {
  __shared__ float red[2 * kNormRowsPerWg];
  const int wave = threadIdx.x >> 6, slot = wave / NWR, part = wave % NWR;
  const int64_t row = (int64_t)blockIdx.x * (kNormRowsPerWg / NWR) + slot;
  if (NWR == 1 && row >= rows) return;
  const bool live = row < rows;
  const int lane = threadIdx.x & 63;
  const int chunks = (C >> 3) / NWR;
  const int c0 = part * chunks * 8;
  const int64_t r = live ? row : 0;
  const int64_t slice = rows * (int64_t)C;
  const uint4* av = reinterpret_cast<const uint4*>(xa + r * C + c0);
  const uint4* tv = reinterpret_cast<const uint4*>(xt + r * C + c0);
  uint4* ov = reinterpret_cast<uint4*>(xn + r * C + c0);
  uint4* bv = reinterpret_cast<uint4*>(bos + (live ? bi[row] * bsb + ti[row] * bsn : 0) + c0);
  float v[CH][8];
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    const int c = lane + 64 * j;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[j][e] = 0.0f;
    if (live && c < chunks) {
      const float* p = P + r * C + c0 + 8 * c;
      float4 a0 = *reinterpret_cast<const float4*>(p), a1 = *reinterpret_cast<const float4*>(p + 4);
      for (int sl = 1; sl < S; ++sl) {
        const float4 b0 = *reinterpret_cast<const float4*>(p + sl * slice);
        const float4 b1 = *reinterpret_cast<const float4*>(p + sl * slice + 4);
        a0.x += b0.x; a0.y += b0.y; a0.z += b0.z; a0.w += b0.w;
        a1.x += b1.x; a1.y += b1.y; a1.z += b1.z; a1.w += b1.w;
      }
      const float acc[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
      float fbias[8], g[8], xm[8], fa[8], ft[8], fm[8], fo[8], fbo[8];
      if (fb) {
        unpack8(reinterpret_cast<const uint4*>(fb + c0)[c], fbias);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) fbias[e] = 0.0f;
      }
      unpack8(reinterpret_cast<const uint4*>(fg + c0)[c], g);
#pragma unroll
      for (int e = 0; e < 8; ++e) xm[e] = round_bf16(__builtin_fmaf(acc[e], acc_scale, fbias[e])) * g[e];
      unpack8(pack8(xm), fm);  // the bf16 mlp row, as the unfused step reads it back
      unpack8(av[c], fa);
      unpack8(tv[c], ft);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        fo[e] = ft[e] + fm[e];
        fbo[e] = round_bf16(ft[e] - fa[e]) + fm[e];
      }
      const uint4 o = pack8(fo);
      ov[c] = o;
      bv[c] = pack8(fbo);
      unpack8(o, v[j]);
    }
  }
  if (w) layernorm_row<CH, NWR>(v, lane, chunks, C, w + c0, bias + c0, eps, ln_out + r * C + c0, nullptr, red, slot,
                                part, live);
}

// Thread = (row, head, chunk of 8 in the left half). Rows with patch_mask == 0 are left untouched.
__global__ __launch_bounds__(256) void rope_active_inplace_kernel(
    uint16_t* q, int64_t qst, int64_t qsh, uint16_t* k, int64_t kst, int64_t ksh, const float* __restrict__ sin_t,
    const float* __restrict__ cos_t, int64_t tst, const uint8_t* __restrict__ pm, const int64_t* __restrict__ ridx,
    int64_t n, int H, int Dh) {
  const int half = Dh >> 1;
  const int cph = half >> 3;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per_row = (int64_t)H * cph;
  const int64_t row = gid / per_row;
  if (row >= n) return;
  if (!pm[row]) return;
  const int rem = (int)(gid - row * per_row);
  const int h = rem / cph;
  const int c = rem - h * cph;
  const int64_t tr = ridx[row];
  const int d0 = c * 8;
  float cl[8], cr[8], sl[8], sr[8];
  load8f(cos_t + tr * tst + d0, cl);
  load8f(cos_t + tr * tst + d0 + half, cr);
  load8f(sin_t + tr * tst + d0, sl);
  load8f(sin_t + tr * tst + d0 + half, sr);
  uint16_t* ptrs[2] = {q + row * qst + h * qsh, k + row * kst + h * ksh};
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    uint4* lp = reinterpret_cast<uint4*>(ptrs[m] + d0);
    uint4* rp = reinterpret_cast<uint4*>(ptrs[m] + d0 + half);
    float l[8], r[8];
    unpack8(*lp, l);
    unpack8(*rp, r);
    rope8(l, r, cl, cr, sl, sr);
    *lp = pack8(l);
    *rp = pack8(r);
  }
}

// Post-QKV step: qkv [M, 3, H, Dh] -> RoPE(q), RoPE(k) on patch rows; q -> q_out [M, H, Dh];
// k, v -> kv[b, t, 0 | 1, h, :] (the [2, H, Dh] part of a cache row is contiguous).
// SCALED: qkv holds the raw product of an NVFP4 qkv linear, and every value is first taken through its
// scale-and-bias epilogue, bf16(raw * s + bias[col]) (bf16(raw * s) without a bias), exactly as
// scale_bias_kernel writes it; RoPE and the writes then proceed on those values.
template <bool SCALED>
__global__ __launch_bounds__(256) void qkv_rope_kv_scatter_kernel(
    const uint16_t* __restrict__ qkv, int64_t M, int H, int Dh, const float* __restrict__ sin_t,
    const float* __restrict__ cos_t, int64_t tst, const uint8_t* __restrict__ pm, const int64_t* __restrict__ ridx,
    const int64_t* __restrict__ bi, const int64_t* __restrict__ ti, uint16_t* __restrict__ kv, int64_t kvb,
    int64_t kvn, uint16_t* __restrict__ qo, float sc, const uint16_t* __restrict__ sbias) {
  const int half = Dh >> 1;
  const int cph = half >> 3;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per_row = (int64_t)H * cph;
  const int64_t row = gid / per_row;
  if (row >= M) return;
  const int rem = (int)(gid - row * per_row);
  const int h = rem / cph;
  const int c = rem - h * cph;
  const int d0 = c * 8;
  const int64_t HD = (int64_t)H * Dh;
  const uint16_t* src = qkv + row * 3 * HD + (int64_t)h * Dh;
  uint4 q_l = *reinterpret_cast<const uint4*>(src + d0);
  uint4 q_r = *reinterpret_cast<const uint4*>(src + d0 + half);
  uint4 k_l = *reinterpret_cast<const uint4*>(src + HD + d0);
  uint4 k_r = *reinterpret_cast<const uint4*>(src + HD + d0 + half);
  uint4 v_l = *reinterpret_cast<const uint4*>(src + 2 * HD + d0);
  uint4 v_r = *reinterpret_cast<const uint4*>(src + 2 * HD + d0 + half);
  if constexpr (SCALED) {
    auto sb8 = [&](uint4 u, int64_t col) __attribute__((always_inline)) {
      float f[8], b[8];
      unpack8(u, f);
      if (sbias) {
        unpack8(*reinterpret_cast<const uint4*>(sbias + col), b);
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = __builtin_fmaf(f[e], sc, b[e]);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = f[e] * sc;
      }
      return pack8(f);
    };
    const int64_t c0 = (int64_t)h * Dh + d0;
    q_l = sb8(q_l, c0);
    q_r = sb8(q_r, c0 + half);
    k_l = sb8(k_l, HD + c0);
    k_r = sb8(k_r, HD + c0 + half);
    v_l = sb8(v_l, 2 * HD + c0);
    v_r = sb8(v_r, 2 * HD + c0 + half);
  }
  if (pm[row]) {
    const int64_t tr = ridx[row];
    float cl[8], cr[8], sl[8], sr[8];
    load8f(cos_t + tr * tst + d0, cl);
    load8f(cos_t + tr * tst + d0 + half, cr);
    load8f(sin_t + tr * tst + d0, sl);
    load8f(sin_t + tr * tst + d0 + half, sr);
    float l[8], r[8];
    unpack8(q_l, l);
    unpack8(q_r, r);
    rope8(l, r, cl, cr, sl, sr);
    q_l = pack8(l);
    q_r = pack8(r);
    unpack8(k_l, l);
    unpack8(k_r, r);
    rope8(l, r, cl, cr, sl, sr);
    k_l = pack8(l);
    k_r = pack8(r);
  }
  uint16_t* qd = qo + row * HD + (int64_t)h * Dh;
  *reinterpret_cast<uint4*>(qd + d0) = q_l;
  *reinterpret_cast<uint4*>(qd + d0 + half) = q_r;
  uint16_t* kd = kv + bi[row] * kvb + ti[row] * kvn + (int64_t)h * Dh;
  *reinterpret_cast<uint4*>(kd + d0) = k_l;
  *reinterpret_cast<uint4*>(kd + d0 + half) = k_r;
  *reinterpret_cast<uint4*>(kd + HD + d0) = v_l;
  *reinterpret_cast<uint4*>(kd + HD + d0 + half) = v_r;
}

}  // namespace oudjat

using namespace oudjat;

// Calls f(CH, NWR) (integral constants) with the instance of a LayerNorm-family kernel for row width C:
// NWR = row_parts(C) waves per row and CH 16-byte chunks per lane (the wave's part over 64 lanes).
template <typename F>
static void row_dispatch(int64_t C, F&& f) {
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I4 = std::integral_constant<int, 4>;
  using I8 = std::integral_constant<int, 8>;
  using I16 = std::integral_constant<int, 16>;
  const int parts = row_parts(C);
  if (parts == 4) {
    if (C <= 4096) f(I2{}, I4{});
    else f(I4{}, I4{});
  } else if (parts == 2) {
    f(I2{}, I2{});
  } else if (C <= 512) {
    f(I1{}, I1{});
  } else if (C <= 1024) {
    f(I2{}, I1{});
  } else if (C <= 2048) {
    f(I4{}, I1{});
  } else if (C <= 4096) {
    f(I8{}, I1{});
  } else {
    f(I16{}, I1{});
  }
}

static int layernorm_launch(const uint16_t* x, int64_t rows, int64_t C, int64_t xs, const uint16_t* w,
                            const uint16_t* b, float eps, const float* xh_ts, uint16_t* out, int64_t os,
                            oudjat_stream_t stream, const char* what, const void* pf = nullptr,
                            int64_t pf_bytes = 0) {
  OUDJAT_REQUIRE(rows >= 0 && C > 0, OUDJAT_ERR_INVALID_ARGUMENT, "%s: bad size", what);
  OUDJAT_REQUIRE(pf_bytes >= 0 && (pf_bytes == 0 || pf), OUDJAT_ERR_INVALID_ARGUMENT,
                 "%s: prefetch region of %lld bytes without a pointer", what, (long long)pf_bytes);
  OUDJAT_REQUIRE(pf_bytes == 0 || aligned(pf, 4), OUDJAT_ERR_UNSUPPORTED_LAYOUT,
                 "%s: prefetch region must be 4-byte aligned", what);
  if (rows == 0) return OUDJAT_OK;
  OUDJAT_REQUIRE(x && w && b && out, OUDJAT_ERR_INVALID_ARGUMENT, "%s: null pointer", what);
  OUDJAT_REQUIRE(C % 8 == 0 && xs % 8 == 0 && os % 8 == 0 && aligned(x, 16) && aligned(out, 16) && aligned(w, 16) &&
                     aligned(b, 16),
                 OUDJAT_ERR_UNSUPPORTED_LAYOUT, "%s: 16-byte aligned rows with C %% 8 == 0 required", what);
  OUDJAT_REQUIRE(!xh_ts || C % 16 == 0, OUDJAT_ERR_UNSUPPORTED_SHAPE, "%s: NVFP4 output needs C %% 16 == 0", what);
  OUDJAT_REQUIRE(C <= 8192, OUDJAT_ERR_TOO_LARGE, "%s: C=%lld > 8192", what, (long long)C);
  const unsigned grid = (unsigned)cdiv(rows, kNormRowsPerWg / row_parts(C));
  hipStream_t st = as_stream(stream);
  const int64_t pf_lines = pf_bytes / 128;  // whole lines; a partial last line is left to the reader
  const uint32_t* p = static_cast<const uint32_t*>(pf);
  auto go = [&](auto pf_c) {
    row_dispatch(C, [&](auto ch, auto nwr) {
      layernorm_kernel<decltype(ch)::value, decltype(nwr)::value, decltype(pf_c)::value>
          <<<grid, kNormThreads, 0, st>>>(x, rows, (int)C, xs, w, b, eps, out, os, xh_ts, p, pf_lines);
    });
  };
  if (pf_lines > 0) go(std::true_type{});
  else go(std::false_type{});
  return check_launch(what);
}

extern "C" int oudjat_layernorm_rows(const uint16_t* x, int64_t rows, int64_t C, int64_t xs, const uint16_t* w,
                                     const uint16_t* b, float eps, uint16_t* out, int64_t os, oudjat_stream_t stream) {
  return layernorm_launch(x, rows, C, xs, w, b, eps, nullptr, out, os, stream, "layernorm_rows");
}

extern "C" int oudjat_layernorm_rows_prefetch(const uint16_t* x, int64_t rows, int64_t C, int64_t xs,
                                              const uint16_t* w, const uint16_t* b, float eps, uint16_t* out,
                                              int64_t os, const void* prefetch, int64_t prefetch_bytes,
                                              oudjat_stream_t stream) {
  return layernorm_launch(x, rows, C, xs, w, b, eps, nullptr, out, os, stream, "layernorm_rows_prefetch", prefetch,
                          prefetch_bytes);
}

extern "C" int oudjat_layernorm_rows_nvfp4(const uint16_t* x, int64_t rows, int64_t C, int64_t xs, const uint16_t* w,
                                           const uint16_t* b, float eps, const float* tensor_scale, uint16_t* xhat,
                                           int64_t xhat_stride, oudjat_stream_t stream) {
  OUDJAT_REQUIRE(tensor_scale || rows == 0, OUDJAT_ERR_INVALID_ARGUMENT, "layernorm_rows_nvfp4: null tensor scale");
  return layernorm_launch(x, rows, C, xs, w, b, eps, tensor_scale, xhat, xhat_stride, stream, "layernorm_rows_nvfp4");
}

extern "C" int oudjat_gather_rows_ln(const uint16_t* x, int64_t stride_b, int64_t stride_n, int64_t C,
                                     const int64_t* batch_idx, const int64_t* token_idx, int64_t rows,
                                     const uint16_t* w, const uint16_t* b, float eps, const float* tensor_scale,
                                     uint16_t* x_out, uint16_t* ln_out, oudjat_stream_t stream) {
  const char* what = "gather_rows_ln";
  OUDJAT_REQUIRE(rows >= 0 && C > 0, OUDJAT_ERR_INVALID_ARGUMENT, "%s: bad size", what);
  if (rows == 0) return OUDJAT_OK;
  OUDJAT_REQUIRE(x && batch_idx && token_idx && w && b && x_out && ln_out, OUDJAT_ERR_INVALID_ARGUMENT,
                 "%s: null pointer", what);
  OUDJAT_REQUIRE(C % 8 == 0 && stride_b % 8 == 0 && stride_n % 8 == 0 && aligned(x, 16) && aligned(x_out, 16) &&
                     aligned(ln_out, 16) && aligned(w, 16) && aligned(b, 16) && aligned(batch_idx, 8) &&
                     aligned(token_idx, 8),
                 OUDJAT_ERR_UNSUPPORTED_LAYOUT, "%s: 16-byte aligned rows with C %% 8 == 0 required", what);
  OUDJAT_REQUIRE(!tensor_scale || C % 16 == 0, OUDJAT_ERR_UNSUPPORTED_SHAPE, "%s: NVFP4 output needs C %% 16 == 0",
                 what);
  OUDJAT_REQUIRE(C <= 8192, OUDJAT_ERR_TOO_LARGE, "%s: C=%lld > 8192", what, (long long)C);
  const unsigned grid = (unsigned)cdiv(rows, kNormRowsPerWg / row_parts(C));
  hipStream_t st = as_stream(stream);
  row_dispatch(C, [&](auto ch, auto nwr) {
    gather_ln_kernel<decltype(ch)::value, decltype(nwr)::value><<<grid, kNormThreads, 0, st>>>(
        x, stride_b, stride_n, batch_idx, token_idx, rows, (int)C, w, b, eps, x_out, ln_out, tensor_scale);
  });
  return check_launch(what);
}

extern "C" int oudjat_rope_active_inplace(uint16_t* q, int64_t qst, int64_t qsh, uint16_t* k, int64_t kst, int64_t ksh,
                                          const float* sin_t, const float* cos_t, int64_t tst, const uint8_t* pm,
                                          const int64_t* ridx, int64_t n, int64_t H, int64_t Dh,
                                          oudjat_stream_t stream) {
  OUDJAT_REQUIRE(n >= 0 && H >= 0 && Dh >= 0, OUDJAT_ERR_INVALID_ARGUMENT, "rope_active_inplace: negative size");
  if (n == 0 || H == 0 || Dh == 0) return OUDJAT_OK;
  OUDJAT_REQUIRE(q && k && sin_t && cos_t && pm && ridx, OUDJAT_ERR_INVALID_ARGUMENT, "rope_active_inplace: null pointer");
  OUDJAT_REQUIRE(Dh % 16 == 0, OUDJAT_ERR_UNSUPPORTED_SHAPE, "rope_active_inplace: Dh=%lld must be a multiple of 16",
                 (long long)Dh);
  OUDJAT_REQUIRE(qst % 8 == 0 && qsh % 8 == 0 && kst % 8 == 0 && ksh % 8 == 0 && tst % 8 == 0 && aligned(q, 16) &&
                     aligned(k, 16) && aligned(sin_t, 16) && aligned(cos_t, 16),
                 OUDJAT_ERR_UNSUPPORTED_LAYOUT, "rope_active_inplace: 16-byte aligned rows/heads required");
  const int64_t threads = n * H * (Dh / 16);
  rope_active_inplace_kernel<<<(unsigned)cdiv(threads, 256), 256, 0, as_stream(stream)>>>(
      q, qst, qsh, k, kst, ksh, sin_t, cos_t, tst, pm, ridx, n, (int)H, (int)Dh);
  return check_launch("rope_active_inplace");
}

static int qkv_rope_kv_scatter_launch(const uint16_t* qkv, int64_t M, int64_t H, int64_t Dh, const float* sin_t,
                                      const float* cos_t, int64_t tst, const uint8_t* pm, const int64_t* ridx,
                                      const int64_t* bi, const int64_t* ti, uint16_t* kv, int64_t kvb, int64_t kvn,
                                      uint16_t* qo, bool scaled, float sc, const uint16_t* sbias,
                                      oudjat_stream_t stream, const char* what) {
  OUDJAT_REQUIRE(M >= 0 && H > 0 && Dh > 0, OUDJAT_ERR_INVALID_ARGUMENT, "%s: bad size", what);
  if (M == 0) return OUDJAT_OK;
  OUDJAT_REQUIRE(qkv && sin_t && cos_t && pm && ridx && bi && ti && kv && qo, OUDJAT_ERR_INVALID_ARGUMENT,
                 "%s: null pointer", what);
  OUDJAT_REQUIRE(Dh % 16 == 0, OUDJAT_ERR_UNSUPPORTED_SHAPE, "%s: Dh=%lld must be a multiple of 16", what,
                 (long long)Dh);
  OUDJAT_REQUIRE(kvb % 8 == 0 && kvn % 8 == 0 && tst % 8 == 0 && aligned(qkv, 16) && aligned(kv, 16) &&
                     aligned(qo, 16) && aligned(sin_t, 16) && aligned(cos_t, 16) && (!sbias || aligned(sbias, 16)),
                 OUDJAT_ERR_UNSUPPORTED_LAYOUT, "%s: 16-byte aligned rows required", what);
  const int64_t threads = M * H * (Dh / 16);
  const unsigned grid = (unsigned)cdiv(threads, 256);
  if (scaled)
    qkv_rope_kv_scatter_kernel<true><<<grid, 256, 0, as_stream(stream)>>>(qkv, M, (int)H, (int)Dh, sin_t, cos_t, tst,
                                                                           pm, ridx, bi, ti, kv, kvb, kvn, qo, sc,
                                                                           sbias);
  else
    qkv_rope_kv_scatter_kernel<false><<<grid, 256, 0, as_stream(stream)>>>(qkv, M, (int)H, (int)Dh, sin_t, cos_t, tst,
                                                                            pm, ridx, bi, ti, kv, kvb, kvn, qo, 1.0f,
                                                                            nullptr);
  return check_launch(what);
}

extern "C" int oudjat_qkv_rope_kv_scatter(const uint16_t* qkv, int64_t M, int64_t H, int64_t Dh, const float* sin_t,
                                          const float* cos_t, int64_t tst, const uint8_t* pm, const int64_t* ridx,
                                          const int64_t* bi, const int64_t* ti, uint16_t* kv, int64_t kvb,
                                          int64_t kvn, uint16_t* qo, oudjat_stream_t stream) {
  return qkv_rope_kv_scatter_launch(qkv, M, H, Dh, sin_t, cos_t, tst, pm, ridx, bi, ti, kv, kvb, kvn, qo, false, 1.0f,
                                    nullptr, stream, "qkv_rope_kv_scatter");
}

extern "C" int oudjat_qkv_rope_kv_scatter_scaled(const uint16_t* qkv_raw, int64_t M, int64_t H, int64_t Dh,
                                                 float scale, const uint16_t* bias, const float* sin_t,
                                                 const float* cos_t, int64_t tst, const uint8_t* pm,
                                                 const int64_t* ridx, const int64_t* bi, const int64_t* ti,
                                                 uint16_t* kv, int64_t kvb, int64_t kvn, uint16_t* qo,
                                                 oudjat_stream_t stream) {
  return qkv_rope_kv_scatter_launch(qkv_raw, M, H, Dh, sin_t, cos_t, tst, pm, ridx, bi, ti, kv, kvb, kvn, qo, true,
                                    scale, bias, stream, "qkv_rope_kv_scatter_scaled");
}

static int packed_residual_ln_launch(const uint16_t* x_act, const uint16_t* x_attn, const uint16_t* mlp,
                                     int64_t rows, int64_t C, const int64_t* batch_idx, const int64_t* token_idx,
                                     uint16_t* bos, int64_t bos_stride_b, int64_t bos_stride_n, uint16_t* x_new,
                                     const uint16_t* ln_w, const uint16_t* ln_b, float eps, const float* xh_ts,
                                     uint16_t* ln_out, oudjat_stream_t stream, const char* what) {
  OUDJAT_REQUIRE(rows >= 0 && C > 0, OUDJAT_ERR_INVALID_ARGUMENT, "%s: bad size", what);
  if (rows == 0) return OUDJAT_OK;
  OUDJAT_REQUIRE(x_act && x_attn && mlp && batch_idx && token_idx && bos && x_new && ln_w && ln_b && ln_out,
                 OUDJAT_ERR_INVALID_ARGUMENT, "%s: null pointer", what);
  OUDJAT_REQUIRE(C % 8 == 0 && aligned(x_act, 16) && aligned(x_attn, 16) && aligned(mlp, 16) && aligned(bos, 16) &&
                     aligned(x_new, 16) && aligned(ln_w, 16) && aligned(ln_b, 16) && aligned(ln_out, 16) &&
                     bos_stride_b % 8 == 0 && bos_stride_n % 8 == 0,
                 OUDJAT_ERR_UNSUPPORTED_LAYOUT, "%s: 16-byte aligned rows, C %% 8 == 0", what);
  OUDJAT_REQUIRE(!xh_ts || C % 16 == 0, OUDJAT_ERR_UNSUPPORTED_SHAPE, "%s: NVFP4 output needs C %% 16 == 0", what);
  OUDJAT_REQUIRE(C <= 8192, OUDJAT_ERR_TOO_LARGE, "%s: C=%lld > 8192", what, (long long)C);
  const unsigned grid = (unsigned)cdiv(rows, kNormRowsPerWg / row_parts(C));
  hipStream_t st = as_stream(stream);
  row_dispatch(C, [&](auto ch, auto nwr) {
    packed_residual_ln_kernel<decltype(ch)::value, decltype(nwr)::value><<<grid, kNormThreads, 0, st>>>(
        x_act, x_attn, mlp, rows, (int)C, batch_idx, token_idx, bos, bos_stride_b, bos_stride_n, x_new, ln_w, ln_b,
        eps, ln_out, xh_ts);
  });
  return check_launch(what);
}

extern "C" int oudjat_packed_residual_persist_ln(const uint16_t* x_act, const uint16_t* x_attn, const uint16_t* mlp,
                                                 int64_t rows, int64_t C, const int64_t* batch_idx,
                                                 const int64_t* token_idx, uint16_t* bos, int64_t bos_stride_b,
                                                 int64_t bos_stride_n, uint16_t* x_new, const uint16_t* ln_w,
                                                 const uint16_t* ln_b, float eps, uint16_t* ln_out,
                                                 oudjat_stream_t stream) {
  return packed_residual_ln_launch(x_act, x_attn, mlp, rows, C, batch_idx, token_idx, bos, bos_stride_b, bos_stride_n,
                                   x_new, ln_w, ln_b, eps, nullptr, ln_out, stream, "packed_residual_persist_ln");
}

extern "C" int oudjat_packed_residual_persist_ln_nvfp4(const uint16_t* x_act, const uint16_t* x_attn,
                                                       const uint16_t* mlp, int64_t rows, int64_t C,
                                                       const int64_t* batch_idx, const int64_t* token_idx,
                                                       uint16_t* bos, int64_t bos_stride_b, int64_t bos_stride_n,
                                                       uint16_t* x_new, const uint16_t* ln_w, const uint16_t* ln_b,
                                                       float eps, const float* tensor_scale, uint16_t* xhat,
                                                       oudjat_stream_t stream) {
  OUDJAT_REQUIRE(tensor_scale || rows == 0, OUDJAT_ERR_INVALID_ARGUMENT,
                 "packed_residual_persist_ln_nvfp4: null tensor scale");
  return packed_residual_ln_launch(x_act, x_attn, mlp, rows, C, batch_idx, token_idx, bos, bos_stride_b, bos_stride_n,
                                   x_new, ln_w, ln_b, eps, tensor_scale, xhat, stream,
                                   "packed_residual_persist_ln_nvfp4");
}

extern "C" int oudjat_splitk_ls_packed_residual(const float* partials, int64_t slices, const uint16_t* fc_bias,
                                                const uint16_t* ls_gamma, float acc_scale, const uint16_t* x_act,
                                                const uint16_t* x_attn, int64_t rows, int64_t C,
                                                const int64_t* batch_idx, const int64_t* token_idx, uint16_t* bos,
                                                int64_t bos_stride_b, int64_t bos_stride_n, uint16_t* x_new,
                                                const uint16_t* ln_w, const uint16_t* ln_b, float eps,
                                                uint16_t* ln_out, oudjat_stream_t stream) {
  OUDJAT_REQUIRE(rows >= 0 && C > 0 && slices >= 1, OUDJAT_ERR_INVALID_ARGUMENT, "splitk_ls_packed_residual: bad size");
  if (rows == 0) return OUDJAT_OK;
  OUDJAT_REQUIRE(partials && ls_gamma && x_act && x_attn && batch_idx && token_idx && bos && x_new &&
                     (ln_w == nullptr) == (ln_b == nullptr) && (ln_w == nullptr) == (ln_out == nullptr),
                 OUDJAT_ERR_INVALID_ARGUMENT, "splitk_ls_packed_residual: null pointer (LayerNorm w, b, out together)");
  OUDJAT_REQUIRE(C % 8 == 0 && aligned(partials, 16) && aligned(ls_gamma, 16) && (!fc_bias || aligned(fc_bias, 16)) &&
                     aligned(x_act, 16) && aligned(x_attn, 16) && aligned(bos, 16) && aligned(x_new, 16) &&
                     (!ln_w || (aligned(ln_w, 16) && aligned(ln_b, 16) && aligned(ln_out, 16))) &&
                     bos_stride_b % 8 == 0 && bos_stride_n % 8 == 0,
                 OUDJAT_ERR_UNSUPPORTED_LAYOUT, "splitk_ls_packed_residual: 16-byte aligned rows, C %% 8 == 0");
  OUDJAT_REQUIRE(C <= 8192 && slices < 65536, OUDJAT_ERR_TOO_LARGE, "splitk_ls_packed_residual: C=%lld > 8192",
                 (long long)C);
  const unsigned grid = (unsigned)cdiv(rows, kNormRowsPerWg / row_parts(C));
  hipStream_t st = as_stream(stream);
  row_dispatch(C, [&](auto ch, auto nwr) {
    splitk_ls_residual_ln_kernel<decltype(ch)::value, decltype(nwr)::value><<<grid, kNormThreads, 0, st>>>(
        partials, (int)slices, fc_bias, ls_gamma, acc_scale, x_act, x_attn, rows, (int)C, batch_idx, token_idx, bos,
        bos_stride_b, bos_stride_n, x_new, ln_w, ln_b, eps, ln_out);
  });
  return check_launch("splitk_ls_packed_residual");
}
