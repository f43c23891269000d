// Selected-row GEMMs: C[M, N] = epilogue(A[M, K] . W[N, K]^T), bf16 in, fp32 accumulate on MFMA.
//
// Both operands are K-contiguous (activations [M, K] row-major, nn.Linear weights [N, K]), which is
// the natural operand layout of v_mfma_f32_32x32x16_bf16: each lane feeds 8 consecutive K values of
// one row of A and one row of W, i.e. one 16-byte LDS read per operand per MFMA.
//
// Workgroup tile BM x BN x 64 with 4 waves in a 2 x 2 arrangement; each wave owns a
// (BM/2) x (BN/2) sub-tile made of 32x32 MFMA blocks. K tiles are double-buffered in LDS with a
// register prefetch of the next tile, so one barrier per K step separates the LDS producer and
// consumer. LDS rows are padded by 16 bytes so the 16-byte fragment reads of 8 consecutive rows hit
// disjoint banks.
//
// The epilogues fold in the elementwise work the reference runs as separate kernels after each
// Linear: bias, exact-erf GELU (fc1), LayerScale (fc2) and LayerScale + residual (proj), with a bf16
// rounding at every point where the reference materialises a bf16 tensor.
#include "common.hpp"

namespace oudjat {

static constexpr int kBK = 64;
static constexpr int kLdsPad = 8;  // bf16 elements of padding per LDS row
static constexpr int kGemmThreads = 256;

struct EpiArgs {
  const uint16_t* bias;
  const uint16_t* gamma;
  const uint16_t* resid;
  int64_t ldr;
};

template <int EPI>
__device__ __forceinline__ float epilogue(float acc, int64_t row, int64_t col, const EpiArgs& ea) {
  float v = acc;
  if (ea.bias) v += bf16_to_f32(ea.bias[col]);
  v = round_bf16(v);
  if (EPI == OUDJAT_EPI_BIAS_GELU) {
    v = v * 0.5f * (1.0f + erff(v * 0.70710678118654752440f));
  } else if (EPI == OUDJAT_EPI_BIAS_LS_RESID) {
    v = fmaf(v, bf16_to_f32(ea.gamma[col]), bf16_to_f32(ea.resid[row * ea.ldr + col]));
  } else if (EPI == OUDJAT_EPI_BIAS_LS) {
    v = v * bf16_to_f32(ea.gamma[col]);
  } else if (EPI == OUDJAT_EPI_BIAS_SILU_MUL) {
    v = round_bf16(v / (1.0f + expf(-v))) * bf16_to_f32(ea.resid[row * ea.ldr + col]);
  }
  return v;
}

template <int BM, int BN, int EPI>
__global__ __launch_bounds__(kGemmThreads) void gemm_bf16_kernel(const uint16_t* __restrict__ A, int64_t M, int64_t K,
                                                                 int64_t lda, const uint16_t* __restrict__ W,
                                                                 int64_t N, int64_t ldw, EpiArgs ea,
                                                                 uint16_t* __restrict__ C, int64_t ldc) {
  constexpr int LDS_ROW = kBK + kLdsPad;
  constexpr int WM = BM / 2, WN = BN / 2;     // wave tile
  constexpr int FM = WM / 32, FN = WN / 32;   // 32x32 MFMA blocks per wave
  constexpr int A_CHUNKS = BM * kBK / 8 / kGemmThreads;  // 16-byte chunks per thread
  constexpr int B_CHUNKS = BN * kBK / 8 / kGemmThreads;
  static_assert(A_CHUNKS * kGemmThreads * 8 == BM * kBK, "A tile must split evenly");
  static_assert(B_CHUNKS * kGemmThreads * 8 == BN * kBK, "B tile must split evenly");

  __shared__ uint16_t As[2][BM * LDS_ROW];
  __shared__ uint16_t Bs[2][BN * LDS_ROW];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm0 = (wave >> 1) * WM;
  const int wn0 = (wave & 1) * WN;
  const int64_t m0 = (int64_t)blockIdx.y * BM;
  const int64_t n0 = (int64_t)blockIdx.x * BN;

  uint4 ra[A_CHUNKS], rb[B_CHUNKS];

  auto load_tile = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) {
      const int c = tid + i * kGemmThreads;
      const int r = c >> 3, cc = (c & 7) * 8;
      const int64_t gr = m0 + r;
      ra[i] = gr < M ? *reinterpret_cast<const uint4*>(A + gr * lda + k0 + cc) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < B_CHUNKS; ++i) {
      const int c = tid + i * kGemmThreads;
      const int r = c >> 3, cc = (c & 7) * 8;
      const int64_t gr = n0 + r;
      rb[i] = gr < N ? *reinterpret_cast<const uint4*>(W + gr * ldw + k0 + cc) : make_uint4(0, 0, 0, 0);
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) {
      const int c = tid + i * kGemmThreads;
      const int r = c >> 3, cc = (c & 7) * 8;
      *reinterpret_cast<uint4*>(&As[buf][r * LDS_ROW + cc]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_CHUNKS; ++i) {
      const int c = tid + i * kGemmThreads;
      const int r = c >> 3, cc = (c & 7) * 8;
      *reinterpret_cast<uint4*>(&Bs[buf][r * LDS_ROW + cc]) = rb[i];
    }
  };

  f32x16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  const int KT = (int)(K / kBK);
  load_tile(0);
  store_tile(0);
  __syncthreads();

  const int frow = lane & 31;         // row of the fragment within a 32-block
  const int fk = (lane >> 5) * 8;     // K offset of the fragment within a 16-wide step

  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < KT) load_tile((int64_t)(kt + 1) * kBK);
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      bf16x8_t fa[FM], fb[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        fa[i] = as_bf16x8(*reinterpret_cast<const uint4*>(&As[cur][(wm0 + i * 32 + frow) * LDS_ROW + ks * 16 + fk]));
#pragma unroll
      for (int j = 0; j < FN; ++j)
        fb[j] = as_bf16x8(*reinterpret_cast<const uint4*>(&Bs[cur][(wn0 + j * 32 + frow) * LDS_ROW + ks * 16 + fk]));
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < KT) store_tile(cur ^ 1);
    __syncthreads();
  }

  // Output layout of a 32x32 block: lane l, register v -> row 8*(v/4) + 4*(l/32) + v%4, col l%32.
#pragma unroll
  for (int i = 0; i < FM; ++i) {
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int64_t col = n0 + wn0 + j * 32 + (lane & 31);
      if (col >= N) continue;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t row = m0 + wm0 + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        if (row < M) C[row * ldc + col] = (uint16_t)f32_to_bf16(epilogue<EPI>(acc[i][j][v], row, col, ea));
      }
    }
  }
}

template <int BM, int BN>
static void launch_gemm(int epi, const uint16_t* A, int64_t M, int64_t K, int64_t lda, const uint16_t* W, int64_t N,
                        int64_t ldw, const EpiArgs& ea, uint16_t* C, int64_t ldc, hipStream_t st) {
  dim3 grid((unsigned)cdiv(N, BN), (unsigned)cdiv(M, BM));
  switch (epi) {
    case OUDJAT_EPI_BIAS:
      gemm_bf16_kernel<BM, BN, OUDJAT_EPI_BIAS><<<grid, kGemmThreads, 0, st>>>(A, M, K, lda, W, N, ldw, ea, C, ldc);
      break;
    case OUDJAT_EPI_BIAS_GELU:
      gemm_bf16_kernel<BM, BN, OUDJAT_EPI_BIAS_GELU><<<grid, kGemmThreads, 0, st>>>(A, M, K, lda, W, N, ldw, ea, C,
                                                                                   ldc);
      break;
    case OUDJAT_EPI_BIAS_LS_RESID:
      gemm_bf16_kernel<BM, BN, OUDJAT_EPI_BIAS_LS_RESID><<<grid, kGemmThreads, 0, st>>>(A, M, K, lda, W, N, ldw, ea,
                                                                                       C, ldc);
      break;
    case OUDJAT_EPI_BIAS_LS:
      gemm_bf16_kernel<BM, BN, OUDJAT_EPI_BIAS_LS><<<grid, kGemmThreads, 0, st>>>(A, M, K, lda, W, N, ldw, ea, C, ldc);
      break;
    default:
      gemm_bf16_kernel<BM, BN, OUDJAT_EPI_BIAS_SILU_MUL><<<grid, kGemmThreads, 0, st>>>(A, M, K, lda, W, N, ldw, ea,
                                                                                       C, ldc);
      break;
  }
}

}  // namespace oudjat

using namespace oudjat;

extern "C" int oudjat_linear_bf16(const uint16_t* A, int64_t M, int64_t K, int64_t lda, const uint16_t* W, int64_t N,
                                  int64_t ldw, const uint16_t* bias, int epi, const uint16_t* gamma,
                                  const uint16_t* resid, int64_t ldr, uint16_t* C, int64_t ldc,
                                  oudjat_stream_t stream) {
  OUDJAT_REQUIRE(M >= 0 && N >= 0 && K >= 0, OUDJAT_ERR_INVALID_ARGUMENT, "linear_bf16: negative size");
  OUDJAT_REQUIRE(epi >= OUDJAT_EPI_BIAS && epi <= OUDJAT_EPI_BIAS_SILU_MUL, OUDJAT_ERR_INVALID_ARGUMENT,
                 "linear_bf16: bad epilogue %d", epi);
  if (M == 0 || N == 0) return OUDJAT_OK;
  OUDJAT_REQUIRE(A && W && C, OUDJAT_ERR_INVALID_ARGUMENT, "linear_bf16: null pointer");
  OUDJAT_REQUIRE((epi != OUDJAT_EPI_BIAS_LS && epi != OUDJAT_EPI_BIAS_LS_RESID) || gamma, OUDJAT_ERR_INVALID_ARGUMENT,
                 "linear_bf16: epilogue needs gamma");
  OUDJAT_REQUIRE((epi != OUDJAT_EPI_BIAS_LS_RESID && epi != OUDJAT_EPI_BIAS_SILU_MUL) || resid,
                 OUDJAT_ERR_INVALID_ARGUMENT,
                 "linear_bf16: epilogue needs resid");
  OUDJAT_REQUIRE(K > 0 && K % kBK == 0, OUDJAT_ERR_UNSUPPORTED_SHAPE, "linear_bf16: K=%lld must be a multiple of %d",
                 (long long)K, kBK);
  OUDJAT_REQUIRE(N % 64 == 0, OUDJAT_ERR_UNSUPPORTED_SHAPE, "linear_bf16: N=%lld must be a multiple of 64",
                 (long long)N);
  OUDJAT_REQUIRE(lda % 8 == 0 && ldw % 8 == 0 && lda >= K && ldw >= K && ldc >= N && aligned(A, 16) && aligned(W, 16),
                 OUDJAT_ERR_UNSUPPORTED_LAYOUT, "linear_bf16: operands must be 16-byte aligned, ld %% 8 == 0");
  EpiArgs ea{bias, gamma, resid, ldr};
  hipStream_t st = as_stream(stream);
  if (N % 128 == 0) launch_gemm<128, 128>(epi, A, M, K, lda, W, N, ldw, ea, C, ldc, st);
  else launch_gemm<128, 64>(epi, A, M, K, lda, W, N, ldw, ea, C, ldc, st);
  return check_launch("linear_bf16");
}
