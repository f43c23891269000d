// Selected-row GEMMs: C[M, N] = epilogue(A[M, K] . W[N, K]^T), bf16 in, fp32 accumulate on MFMA.
//
// Both operands are K-contiguous (activations [M, K] row-major, nn.Linear weights [N, K]), the
// natural operand layout of v_mfma_f32_32x32x16_bf16: each lane feeds 8 consecutive K values of one
// row of A and one row of W, i.e. one 16-byte LDS read per operand per MFMA.
//
// Kernel family (template): workgroup tile BM x BN x 64, WGM x WGN waves, each wave owning a
// (BM/WGM) x (BN/WGN) sub-tile of 32x32 MFMA blocks whose accumulators live in AGPRs.
//   * LDS holds two K tiles (double buffer). Rows are 128 bytes with the 16-byte chunks
//     XOR-swizzled by (row & 7), so both the 16-byte stores of a row and the 16-byte fragment reads
//     of 8 consecutive rows touch disjoint banks without padding.
//   * Global loads run PF tiles ahead through registers (PF = 1 or 2), so a K step's loads have one
//     or two K steps of MFMA work to hide their latency.
//   * Rows of A beyond M are clamped to M-1 instead of predicated: they only feed output rows that
//     are never stored.
//   * Workgroups are renumbered so that consecutive tiles land on the same XCD (dispatch places
//     workgroup i on XCD i % 8): each XCD sweeps a contiguous band of the tile grid and reuses the
//     A rows and W columns of that band from its own L2.
//
// The epilogues fold in the elementwise work the reference runs as separate kernels after each
// Linear: bias, exact-erf GELU (fc1), LayerScale (fc2), LayerScale + residual (proj) and the SwiGLU
// gate, with a bf16 rounding at every point where the reference materialises a bf16 tensor.
#include <stdlib.h>

#include <type_traits>

#include "common.hpp"

namespace oudjat {

static constexpr int kBK = 64;
static constexpr int kNumXcd = 8;

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

// The part of the epilogue after the first rounding point v = bf16(acc + bias).
template <int EPI>
__device__ __forceinline__ float epilogue_post(float v, int64_t row, int64_t col, const EpiArgs& ea) {
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

// Byte offset of 16-byte chunk `c` (K elements 8c .. 8c+7) of LDS row `r`.
__device__ __forceinline__ int swz(int r, int c) { return r * 128 + ((c ^ (r & 7)) << 4); }

template <int BM, int BN, int WGM, int WGN, int PF, int EPI>
__global__ __launch_bounds__(WGM * WGN * 64) void gemm_bf16_kernel(const uint16_t* __restrict__ A, int M, int K,
                                                                   int64_t lda, const uint16_t* __restrict__ W, int N,
                                                                   int64_t ldw, EpiArgs ea, uint16_t* __restrict__ C,
                                                                   int64_t ldc, int group_m) {
  constexpr int NT = WGM * WGN * 64;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int FM = WM / 32, FN = WN / 32;
  constexpr int A_CH = BM * 8 / NT;  // 16-byte chunks per thread per K tile (8 chunks per 64-wide row)
  constexpr int B_CH = BN * 8 / NT;
  static_assert(A_CH * NT == BM * 8 && B_CH * NT == BN * 8, "tile must split evenly over the threads");
  static_assert(FM >= 1 && FN >= 1 && WM % 32 == 0 && WN % 32 == 0, "wave tile must be 32x32 blocks");

  extern __shared__ __align__(16) unsigned char smem[];
  unsigned char* As = smem;                       // [2][BM * 128]
  unsigned char* Bs = smem + 2 * BM * 128;        // [2][BN * 128]

  // XCD-aware tile order. Workgroup `bid` runs on XCD x = bid % 8 as that XCD's (bid / 8)-th
  // workgroup; XCD x receives q + (x < r) workgroups (q = tiles / 8, r = tiles % 8), so giving it the
  // contiguous band of tiles starting at x*q + min(x, r) is a bijection onto [0, tiles).
  // Within the band, tiles run in groups of `group_m` tile-rows, row index fastest, so the ~64
  // workgroups an XCD holds at once cover a group_m x (64 / group_m) block of tiles whose A rows and
  // W columns fit its L2 together.
  const int tiles_n = (N + BN - 1) / BN;
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles = gridDim.x;
  const int bid = blockIdx.x;
  const int xcd = bid % kNumXcd;
  const int q = tiles / kNumXcd, r = tiles % kNumXcd;
  const int tile = xcd * q + min(xcd, r) + bid / kNumXcd;
  const int per_group = group_m * tiles_n;
  const int grp = tile / per_group;
  const int first_m = grp * group_m;
  const int gsize = min(tiles_m - first_m, group_m);
  const int in_grp = tile - grp * per_group;
  const int tm = first_m + in_grp % gsize, tn = in_grp / gsize;
  const int m0 = tm * BM, n0 = tn * BN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm0 = (wave / WGN) * WM;
  const int wn0 = (wave % WGN) * WN;

  // Per-thread global source rows / chunks (fixed across K tiles).
  const uint16_t* a_src[A_CH];
  const uint16_t* b_src[B_CH];
  int a_lds[A_CH], b_lds[B_CH];
#pragma unroll
  for (int i = 0; i < A_CH; ++i) {
    const int c = tid + i * NT, r = c >> 3, cc = c & 7;
    const int gr = min(m0 + r, M - 1);
    a_src[i] = A + (int64_t)gr * lda + cc * 8;
    a_lds[i] = swz(r, cc);
  }
#pragma unroll
  for (int i = 0; i < B_CH; ++i) {
    const int c = tid + i * NT, r = c >> 3, cc = c & 7;
    const int gr = min(n0 + r, N - 1);
    b_src[i] = W + (int64_t)gr * ldw + cc * 8;
    b_lds[i] = swz(r, cc);
  }

  // Staging registers (clang vector types, so they stay in VGPRs), one set per prefetch slot.
  u32x4_t ra0[A_CH], rb0[B_CH], ra1[PF == 2 ? A_CH : 1], rb1[PF == 2 ? B_CH : 1];
  auto load = [&](auto S, int kt) __attribute__((always_inline)) {
    constexpr int slot = decltype(S)::value;
    u32x4_t* ra = slot == 0 ? ra0 : ra1;
    u32x4_t* rb = slot == 0 ? rb0 : rb1;
    const int k0 = kt * kBK;
#pragma unroll
    for (int i = 0; i < A_CH; ++i) ra[i] = *reinterpret_cast<const u32x4_t*>(a_src[i] + k0);
#pragma unroll
    for (int i = 0; i < B_CH; ++i) rb[i] = *reinterpret_cast<const u32x4_t*>(b_src[i] + k0);
  };
  auto store = [&](auto S, int buf) __attribute__((always_inline)) {
    constexpr int slot = decltype(S)::value;
    const u32x4_t* ra = slot == 0 ? ra0 : ra1;
    const u32x4_t* rb = slot == 0 ? rb0 : rb1;
    unsigned char* a = As + buf * BM * 128;
    unsigned char* b = Bs + buf * BN * 128;
#pragma unroll
    for (int i = 0; i < A_CH; ++i) *reinterpret_cast<u32x4_t*>(a + a_lds[i]) = ra[i];
#pragma unroll
    for (int i = 0; i < B_CH; ++i) *reinterpret_cast<u32x4_t*>(b + b_lds[i]) = rb[i];
  };

  f32x16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  const int KT = K / kBK;
  const int frow = lane & 31;   // fragment row within a 32-row block
  const int fchunk = lane >> 5; // fragment K chunk (0/1) within a 16-wide K step

  auto compute = [&](int buf) __attribute__((always_inline)) {
    const unsigned char* a = As + buf * BM * 128;
    const unsigned char* b = Bs + buf * BN * 128;
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      bf16x8_t fa[FM], fb[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        fa[i] = as_bf16x8(*reinterpret_cast<const uint4*>(a + swz(wm0 + i * 32 + frow, ks * 2 + fchunk)));
#pragma unroll
      for (int j = 0; j < FN; ++j)
        fb[j] = as_bf16x8(*reinterpret_cast<const uint4*>(b + swz(wn0 + j * 32 + frow, ks * 2 + fchunk)));
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
  };
  // One K step. Register slots are compile-time constants (LS: slot the loads PF tiles ahead go to,
  // SS: slot holding tile kt+1), so the staging arrays stay in registers.
  auto step = [&](int kt, auto LS, auto SS) __attribute__((always_inline)) {
    if (kt + PF < KT) load(LS, kt + PF);
    compute(kt & 1);
    if (kt + 1 < KT) store(SS, (kt & 1) ^ 1);
    __syncthreads();
  };

  load(std::integral_constant<int, 0>{}, 0);
  if (PF == 2 && KT > 1) load(std::integral_constant<int, PF - 1>{}, 1);
  store(std::integral_constant<int, 0>{}, 0);
  __syncthreads();
  if (PF == 2) {
    // slot (t & 1) holds tile t
    for (int kt = 0; kt < KT; kt += 2) {
      step(kt, std::integral_constant<int, 0>{}, std::integral_constant<int, PF - 1>{});
      if (kt + 1 < KT) step(kt + 1, std::integral_constant<int, PF - 1>{}, std::integral_constant<int, 0>{});
    }
  } else {
    for (int kt = 0; kt < KT; ++kt) step(kt, std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{});
  }

  // Output layout of a 32x32 block: lane l, register v -> row 8*(v/4) + 4*(l/32) + v%4, col l%32.
#pragma unroll
  for (int i = 0; i < FM; ++i) {
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int col = n0 + wn0 + j * 32 + (lane & 31);
      if (col >= N) continue;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = m0 + wm0 + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        if (row < M) C[(int64_t)row * ldc + col] = (uint16_t)f32_to_bf16(epilogue<EPI>(acc[i][j][v], row, col, ea));
      }
    }
  }
}

// ------------------------------------------------------------------------------------------------
// Direct-to-LDS variant. global_load_lds_dwordx4 writes lane l's 16 bytes to LDS at
// M0 + 16*l, i.e. one wave instruction fills 8 consecutive 128-byte LDS rows. Lane l therefore
// fetches row (l / 8) of its 8-row group at the K chunk that the swizzle places in slot l % 8:
// chunk (l % 8) ^ (l / 8). No staging VGPRs, so a 256x256 tile with 128x128 per wave fits with
// every accumulator in AGPRs; each K step gives a wave FM*FN*4 MFMAs (64 for 128x128, ~2k cycles)
// to cover the next step's loads.
// ------------------------------------------------------------------------------------------------

typedef __attribute__((address_space(3))) void* lds_ptr_t;

__device__ __forceinline__ void wait_vm_all() { __builtin_amdgcn_s_waitcnt(0); }

template <int BM, int BN, int WGM, int WGN, int EPI>
__global__ __launch_bounds__(WGM * WGN * 64) void gemm_bf16_dma_kernel(const uint16_t* __restrict__ A, int M, int K,
                                                                       int64_t lda, const uint16_t* __restrict__ W,
                                                                       int N, int64_t ldw, EpiArgs ea,
                                                                       uint16_t* __restrict__ C, int64_t ldc,
                                                                       int group_m) {
  constexpr int NW = WGM * WGN;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int FM = WM / 32, FN = WN / 32;
  constexpr int AG = BM / 8 / NW;  // 8-row groups of A loaded per wave per K step
  constexpr int BG = BN / 8 / NW;
  constexpr int STAGE = (BM + BN) * 128;
  static_assert(AG * NW * 8 == BM && BG * NW * 8 == BN, "rows must split into 8-row groups per wave");

  extern __shared__ __align__(16) unsigned char smem[];

  const int tiles_n = (N + BN - 1) / BN;
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles = gridDim.x;
  const int bid = blockIdx.x;
  const int xcd = bid % kNumXcd;
  const int q = tiles / kNumXcd, r = tiles % kNumXcd;
  const int tile = xcd * q + min(xcd, r) + bid / kNumXcd;
  const int per_group = group_m * tiles_n;
  const int grp = tile / per_group;
  const int first_m = grp * group_m;
  const int gsize = min(tiles_m - first_m, group_m);
  const int in_grp = tile - grp * per_group;
  const int tm = first_m + in_grp % gsize, tn = in_grp / gsize;
  const int m0 = tm * BM, n0 = tn * BN;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm0 = (wave / WGN) * WM;
  const int wn0 = (wave % WGN) * WN;
  const int lrow = lane >> 3;                 // row within an 8-row group
  const int lchunk = (lane & 7) ^ lrow;       // global K chunk this lane fetches

  const uint16_t* a_src[AG];
  const uint16_t* b_src[BG];
#pragma unroll
  for (int i = 0; i < AG; ++i) {
    const int row = (wave * AG + i) * 8 + lrow;
    a_src[i] = A + (int64_t)min(m0 + row, M - 1) * lda + lchunk * 8;
  }
#pragma unroll
  for (int i = 0; i < BG; ++i) {
    const int row = (wave * BG + i) * 8 + lrow;
    b_src[i] = W + (int64_t)min(n0 + row, N - 1) * ldw + lchunk * 8;
  }
  auto issue = [&](int stage, int kt) __attribute__((always_inline)) {
    unsigned char* base = smem + stage * STAGE;
    const int k0 = kt * kBK;
#pragma unroll
    for (int i = 0; i < AG; ++i)
      __builtin_amdgcn_global_load_lds((const void*)(a_src[i] + k0), (lds_ptr_t)(base + (wave * AG + i) * 1024), 16,
                                       0, 0);
#pragma unroll
    for (int i = 0; i < BG; ++i)
      __builtin_amdgcn_global_load_lds((const void*)(b_src[i] + k0),
                                       (lds_ptr_t)(base + BM * 128 + (wave * BG + i) * 1024), 16, 0, 0);
  };

  f32x16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  const int KT = K / kBK;
  const int frow = lane & 31;
  const int fchunk = lane >> 5;
  issue(0, 0);
  for (int kt = 0; kt < KT; ++kt) {
    wait_vm_all();      // this wave's loads of step kt have landed
    __syncthreads();    // ... and every wave's; every wave is also done reading step kt-1's stage
    if (kt + 1 < KT) issue((kt + 1) & 1, kt + 1);
    const unsigned char* a = smem + (kt & 1) * STAGE;
    const unsigned char* b = a + BM * 128;
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      bf16x8_t fa[FM], fb[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        fa[i] = as_bf16x8(*reinterpret_cast<const uint4*>(a + swz(wm0 + i * 32 + frow, ks * 2 + fchunk)));
#pragma unroll
      for (int j = 0; j < FN; ++j)
        fb[j] = as_bf16x8(*reinterpret_cast<const uint4*>(b + swz(wn0 + j * 32 + frow, ks * 2 + fchunk)));
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
  }

  // Epilogue, phase 1: bf16(acc + bias) into LDS (the K stages are free once every wave is past the
  // last MFMA). Output layout of a 32x32 block: lane l, register v -> row 8*(v/4) + 4*(l/32) + v%4,
  // col l%32. Rows are padded by 16 bytes so lanes 0-31 and 32-63 (rows r, r+4) use different banks.
  constexpr int LDT = BN + 8;
  uint16_t* ct = reinterpret_cast<uint16_t*>(smem);
  __syncthreads();
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int cl = wn0 + j * 32 + (lane & 31);
    const float bias = ea.bias ? bf16_to_f32(ea.bias[min(n0 + cl, N - 1)]) : 0.0f;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int rl = wm0 + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        ct[rl * LDT + cl] = (uint16_t)f32_to_bf16(acc[i][j][v] + bias);
      }
    }
  }
  __syncthreads();
  // Phase 2: 8 consecutive columns per lane, the rest of the epilogue, 16-byte stores.
  constexpr int CPR = BN / 8;
  for (int c = threadIdx.x; c < BM * CPR; c += NW * 64) {
    const int rl = c / CPR, cl = (c - rl * CPR) * 8;
    const int row = m0 + rl, col = n0 + cl;
    if (row >= M || col >= N) continue;
    float v[8];
    unpack8(*reinterpret_cast<const uint4*>(ct + rl * LDT + cl), v);
    if (EPI != OUDJAT_EPI_BIAS) {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = epilogue_post<EPI>(v[e], row, col + e, ea);
    }
    *reinterpret_cast<uint4*>(C + (int64_t)row * ldc + col) = pack8(v);
  }
}

// ------------------------------------------------------------------------------------------------
// Configurations and dispatch
// ------------------------------------------------------------------------------------------------

typedef void (*gemm_fn)(const uint16_t*, int, int, int64_t, const uint16_t*, int, int64_t, EpiArgs, uint16_t*,
                        int64_t, int);

struct GemmCfg {
  int bm, bn, wgm, wgn, pf;
  gemm_fn fn[5];
};

#define OUDJAT_GEMM_CFG(BM, BN, WGM, WGN, PF)                                                             \
  {BM, BN, WGM, WGN, PF,                                                                                 \
   {gemm_bf16_kernel<BM, BN, WGM, WGN, PF, 0>, gemm_bf16_kernel<BM, BN, WGM, WGN, PF, 1>,                 \
    gemm_bf16_kernel<BM, BN, WGM, WGN, PF, 2>, gemm_bf16_kernel<BM, BN, WGM, WGN, PF, 3>,                 \
    gemm_bf16_kernel<BM, BN, WGM, WGN, PF, 4>}}

#define OUDJAT_GEMM_DMA_CFG(BM, BN, WGM, WGN)                                                             \
  {BM, BN, WGM, WGN, 0,                                                                                  \
   {gemm_bf16_dma_kernel<BM, BN, WGM, WGN, 0>, gemm_bf16_dma_kernel<BM, BN, WGM, WGN, 1>,                 \
    gemm_bf16_dma_kernel<BM, BN, WGM, WGN, 2>, gemm_bf16_dma_kernel<BM, BN, WGM, WGN, 3>,                 \
    gemm_bf16_dma_kernel<BM, BN, WGM, WGN, 4>}}

static const GemmCfg kCfgs[] = {
    OUDJAT_GEMM_CFG(128, 128, 2, 2, 1),  // 0
    OUDJAT_GEMM_CFG(128, 128, 2, 2, 2),  // 1
    OUDJAT_GEMM_CFG(256, 128, 2, 2, 1),  // 2
    OUDJAT_GEMM_CFG(256, 128, 2, 2, 2),  // 3
    OUDJAT_GEMM_CFG(128, 256, 2, 2, 2),  // 4
    OUDJAT_GEMM_CFG(256, 256, 2, 4, 2),  // 5
    OUDJAT_GEMM_CFG(256, 128, 4, 2, 2),  // 6
    OUDJAT_GEMM_CFG(128, 128, 2, 2, 2),  // 7 (placeholder slot)
    OUDJAT_GEMM_CFG(128, 64, 2, 2, 2),   // 8 (N % 128 != 0)
    OUDJAT_GEMM_DMA_CFG(256, 256, 2, 2),  // 9
    OUDJAT_GEMM_DMA_CFG(256, 128, 2, 2),  // 10
    OUDJAT_GEMM_DMA_CFG(128, 128, 2, 2),  // 11
    OUDJAT_GEMM_DMA_CFG(128, 256, 2, 2),  // 12
    OUDJAT_GEMM_DMA_CFG(256, 256, 4, 2),  // 13
    OUDJAT_GEMM_DMA_CFG(256, 256, 2, 4),  // 14
};
static constexpr int kNumCfgs = sizeof(kCfgs) / sizeof(kCfgs[0]);

static int env_int(const char* name, int dflt) {
  const char* e = getenv(name);
  return e ? atoi(e) : dflt;
}

static int choose_cfg(int64_t M, int64_t N, int64_t K) {
  static const int forced = env_int("OUDJAT_GEMM_CFG", -1);
  if (forced >= 0 && forced < kNumCfgs && N % kCfgs[forced].bn == 0) return forced;
  if (N % 128 != 0) return 8;
  (void)K;
  // 256x256 tiles (8 waves, direct-to-LDS) when their grid nearly fills the 256 CUs in one round;
  // otherwise 128x128 direct-to-LDS tiles (two workgroups per CU, finer-grained load balance).
  const int64_t tiles256 = cdiv(M, 256) * cdiv(N, 256);
  if (N % 256 == 0 && tiles256 >= 192 && tiles256 <= 256) return 14;
  return 11;
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
                 OUDJAT_ERR_INVALID_ARGUMENT, "linear_bf16: epilogue needs resid");
  OUDJAT_REQUIRE(K > 0 && K % kBK == 0, OUDJAT_ERR_UNSUPPORTED_SHAPE, "linear_bf16: K=%lld must be a multiple of %d",
                 (long long)K, kBK);
  OUDJAT_REQUIRE(N % 64 == 0, OUDJAT_ERR_UNSUPPORTED_SHAPE, "linear_bf16: N=%lld must be a multiple of 64",
                 (long long)N);
  OUDJAT_REQUIRE(lda % 8 == 0 && ldw % 8 == 0 && lda >= K && ldw >= K && ldc >= N && aligned(A, 16) && aligned(W, 16),
                 OUDJAT_ERR_UNSUPPORTED_LAYOUT, "linear_bf16: operands must be 16-byte aligned, ld %% 8 == 0");
  OUDJAT_REQUIRE(M < ((int64_t)1 << 31) && N < ((int64_t)1 << 31) && K < ((int64_t)1 << 31), OUDJAT_ERR_TOO_LARGE,
                 "linear_bf16: dimensions must fit in int32");
  const GemmCfg& cfg = kCfgs[choose_cfg(M, N, K)];
  const int64_t tiles = cdiv(M, cfg.bm) * cdiv(N, cfg.bn);
  OUDJAT_REQUIRE(tiles < ((int64_t)1 << 31), OUDJAT_ERR_TOO_LARGE, "linear_bf16: too many tiles");
  // K stages, or (direct-to-LDS kernels) the bf16 output tile of the epilogue if that is larger.
  size_t lds = (size_t)2 * (cfg.bm + cfg.bn) * 128;
  if (cfg.pf == 0) lds = lds > (size_t)cfg.bm * (cfg.bn + 8) * 2 ? lds : (size_t)cfg.bm * (cfg.bn + 8) * 2;
  const gemm_fn fn = cfg.fn[epi];
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return set_error(OUDJAT_ERR_HIP, "linear_bf16: hipFuncSetAttribute: %s", hipGetErrorString(e));
  }
  EpiArgs ea{bias, gamma, resid, ldr};
  const int threads = cfg.wgm * cfg.wgn * 64;
  static const int group_m = env_int("OUDJAT_GEMM_GROUP_M", 8);
  hipLaunchKernelGGL(fn, dim3((unsigned)tiles), dim3(threads), lds, as_stream(stream), A, (int)M, (int)K, lda, W,
                     (int)N, ldw, ea, C, ldc, group_m > 0 ? group_m : 1);
  return check_launch("linear_bf16");
}
