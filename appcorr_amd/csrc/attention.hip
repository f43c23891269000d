// Sparse-query attention against the full K/V cache.
//
// Queries: the T selected rows of each image (packed [B*T, H, Dh]); keys/values: all N cached rows of
// the same image, read in place from the [B, N, 2, H, Dh] cache (K after RoPE, V raw), no mask.
//
// Workgroup = (64-query tile, head, image); 4 waves, each owning 16 query rows. Keys stream through
// LDS in tiles of 64: K row-major (its rows are the B operand of Q.K^T as-is) and V transposed in LDS
// (so 8 consecutive keys of one head dim are a 16-byte read, the B operand layout of P.V). Both
// products run on v_mfma_f32_16x16x32_bf16 with fp32 accumulators; softmax is the online (running
// max / running sum) form in fp32 with exp2, so the N keys are visited once.
#include "common.hpp"

namespace oudjat {

static constexpr int kAttnThreads = 256;
static constexpr int kKeyTile = 64;
static constexpr int kQTile = 64;

__device__ __forceinline__ float max16(float v) {
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float sum16(float v) {
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) v += __shfl_xor(v, o, 64);
  return v;
}

template <int DH>
__global__ __launch_bounds__(kAttnThreads) void sq_attention_kernel(
    const uint16_t* __restrict__ q, int64_t qrs, int T, const uint16_t* __restrict__ kv, int64_t kvb, int64_t kvn,
    int64_t kvkv, int64_t kvh, int N, float scale_log2, uint16_t* __restrict__ out, int64_t ors) {
  constexpr int KROW = DH + 8;
  constexpr int VROW = kKeyTile + 8;
  constexpr int PROW = kKeyTile + 8;
  constexpr int QK_STEPS = DH / 32;   // K=32 steps over the head dim
  constexpr int OB = DH / 16;         // 16-wide output blocks over the head dim
  constexpr int CPK = DH / 8;         // 16-byte chunks per key row
  __shared__ uint16_t Ks[kKeyTile * KROW];
  __shared__ uint16_t Vt[DH * VROW];
  __shared__ uint16_t Ps[4][16 * PROW];

  const int b = blockIdx.z, h = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int q0 = blockIdx.x * kQTile + wave * 16;
  const int l16 = lane & 15, g16 = lane >> 4;

  bf16x8_t qf[QK_STEPS];
  {
    const int qr = q0 + l16;
#pragma unroll
    for (int ks = 0; ks < QK_STEPS; ++ks) {
      uint4 v = make_uint4(0, 0, 0, 0);
      if (qr < T) v = *reinterpret_cast<const uint4*>(q + ((int64_t)b * T + qr) * qrs + (int64_t)h * DH + ks * 32 + g16 * 8);
      qf[ks] = as_bf16x8(v);
    }
  }

  f32x4_t o[OB];
#pragma unroll
  for (int d = 0; d < OB; ++d) o[d] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  float mrow[4], lrow[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    mrow[v] = -INFINITY;
    lrow[v] = 0.0f;
  }

  const uint16_t* kbase = kv + (int64_t)b * kvb + (int64_t)h * kvh;
  const uint16_t* vbase = kbase + kvkv;
  uint16_t* Pw = Ps[wave];

  for (int n0 = 0; n0 < N; n0 += kKeyTile) {
    for (int c = tid; c < kKeyTile * CPK; c += kAttnThreads) {
      const int key = c / CPK, dc = (c - key * CPK) * 8;
      const int n = n0 + key;
      uint4 kk = make_uint4(0, 0, 0, 0), vv = make_uint4(0, 0, 0, 0);
      if (n < N) {
        kk = *reinterpret_cast<const uint4*>(kbase + (int64_t)n * kvn + dc);
        vv = *reinterpret_cast<const uint4*>(vbase + (int64_t)n * kvn + dc);
      }
      *reinterpret_cast<uint4*>(&Ks[key * KROW + dc]) = kk;
      const uint32_t w[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        Vt[(dc + 2 * e) * VROW + key] = (uint16_t)(w[e] & 0xffffu);
        Vt[(dc + 2 * e + 1) * VROW + key] = (uint16_t)(w[e] >> 16);
      }
    }
    __syncthreads();

    // S = Q . K^T for four 16-key blocks: s[kb][v] = S[row 4*g16+v][key kb*16 + l16]
    f32x4_t s[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      s[kb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int ks = 0; ks < QK_STEPS; ++ks) {
        const bf16x8_t kf = as_bf16x8(*reinterpret_cast<const uint4*>(&Ks[(kb * 16 + l16) * KROW + ks * 32 + g16 * 8]));
        s[kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qf[ks], kf, s[kb], 0, 0, 0);
      }
      if (n0 + kb * 16 + l16 >= N) s[kb] = f32x4_t{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    }

#pragma unroll
    for (int v = 0; v < 4; ++v) {
      float mx = fmaxf(fmaxf(s[0][v], s[1][v]), fmaxf(s[2][v], s[3][v]));
      mx = max16(mx);
      const float mnew = fmaxf(mrow[v], mx);
      const float alpha = exp2f((mrow[v] - mnew) * scale_log2);
      float rs = 0.0f;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        const float p = exp2f((s[kb][v] - mnew) * scale_log2);
        rs += p;
        Pw[(4 * g16 + v) * PROW + kb * 16 + l16] = (uint16_t)f32_to_bf16(p);
      }
      rs = sum16(rs);
      lrow[v] = lrow[v] * alpha + rs;
      mrow[v] = mnew;
#pragma unroll
      for (int d = 0; d < OB; ++d) o[d][v] *= alpha;
    }
    __syncthreads();

    // O += P . V over the 64 keys (two K=32 steps).
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const bf16x8_t pf = as_bf16x8(*reinterpret_cast<const uint4*>(&Pw[l16 * PROW + ks * 32 + g16 * 8]));
#pragma unroll
      for (int d = 0; d < OB; ++d) {
        const bf16x8_t vf = as_bf16x8(*reinterpret_cast<const uint4*>(&Vt[(d * 16 + l16) * VROW + ks * 32 + g16 * 8]));
        o[d] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pf, vf, o[d], 0, 0, 0);
      }
    }
    __syncthreads();
  }

#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int qr = q0 + 4 * g16 + v;
    if (qr >= T) continue;
    const float inv = 1.0f / lrow[v];
    uint16_t* orow = out + ((int64_t)b * T + qr) * ors + (int64_t)h * DH;
#pragma unroll
    for (int d = 0; d < OB; ++d) orow[d * 16 + l16] = (uint16_t)f32_to_bf16(o[d][v] * inv);
  }
}

}  // namespace oudjat

using namespace oudjat;

extern "C" int oudjat_sparse_query_attention(const uint16_t* q, int64_t qrs, int64_t B, int64_t T, int64_t H,
                                             int64_t Dh, const uint16_t* kv, int64_t kvb, int64_t kvn, int64_t kvkv,
                                             int64_t kvh, int64_t N, float scale, uint16_t* out, int64_t ors,
                                             oudjat_stream_t stream) {
  OUDJAT_REQUIRE(B >= 0 && T >= 0 && H >= 0 && N >= 0, OUDJAT_ERR_INVALID_ARGUMENT,
                 "sparse_query_attention: negative size");
  if (B == 0 || T == 0 || H == 0) return OUDJAT_OK;
  OUDJAT_REQUIRE(q && kv && out, OUDJAT_ERR_INVALID_ARGUMENT, "sparse_query_attention: null pointer");
  OUDJAT_REQUIRE(N > 0, OUDJAT_ERR_UNSUPPORTED_SHAPE, "sparse_query_attention: no keys");
  OUDJAT_REQUIRE(Dh == 64 || Dh == 128, OUDJAT_ERR_UNSUPPORTED_SHAPE, "sparse_query_attention: Dh=%lld (64 or 128)",
                 (long long)Dh);
  OUDJAT_REQUIRE(qrs % 8 == 0 && kvb % 8 == 0 && kvn % 8 == 0 && kvkv % 8 == 0 && kvh % 8 == 0 && aligned(q, 16) &&
                     aligned(kv, 16),
                 OUDJAT_ERR_UNSUPPORTED_LAYOUT, "sparse_query_attention: 16-byte aligned q and kv rows required");
  OUDJAT_REQUIRE(B <= 65535 && H <= 65535, OUDJAT_ERR_TOO_LARGE, "sparse_query_attention: grid too large");
  OUDJAT_REQUIRE(N < ((int64_t)1 << 31) && T < ((int64_t)1 << 31), OUDJAT_ERR_TOO_LARGE,
                 "sparse_query_attention: N or T too large");
  const float scale_log2 = scale * 1.4426950408889634f;
  dim3 grid((unsigned)cdiv(T, kQTile), (unsigned)H, (unsigned)B);
  hipStream_t st = as_stream(stream);
  if (Dh == 64)
    sq_attention_kernel<64><<<grid, kAttnThreads, 0, st>>>(q, qrs, (int)T, kv, kvb, kvn, kvkv, kvh, (int)N,
                                                           scale_log2, out, ors);
  else
    sq_attention_kernel<128><<<grid, kAttnThreads, 0, st>>>(q, qrs, (int)T, kv, kvb, kvn, kvkv, kvh, (int)N,
                                                            scale_log2, out, ors);
  return check_launch("sparse_query_attention");
}
