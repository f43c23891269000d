// Selected-row GEMMs: C[M, N] = epilogue(A[M, K] . W[N, K]^T), bf16 in, fp32 accumulate on MFMA.
//
// Both operands are K-contiguous (activations [M, K] row-major, nn.Linear weights [N, K]), the
// natural operand layout of v_mfma_f32_32x32x16_bf16: each lane feeds 8 consecutive K values of one
// row of A and one row of W, i.e. one 16-byte LDS read per operand per MFMA.
//
// Kernel families (templates over the workgroup tile BM x BN and the WGM x WGN wave grid):
//   * gemm_bf16_pp_kernel: 288-row tiles (M = B (5 + k) = 4176 = 14.5 x 288 at the headline shape)
//     with 8 waves in two groups that alternate between MFMA-only and LDS-read phases; fc1 and the
//     fused QKV projection.
//   * gemm_bf16_r16_kernel: 144- and 288-row tiles on 16x16x32 MFMAs with optional split K inside
//     the workgroup; the N = C projections.
//   * gemm_bf16_pipe_kernel: direct-to-LDS loads (global_load_lds, no staging registers), K tiles of
//     32 in four LDS stages issued three tiles ahead, fragments read one K tile ahead of their
//     MFMAs. 256 x 256 tiles with 8 waves; used when one round of tiles fills the GPU.
//   * gemm_bf16_dma_kernel: direct-to-LDS loads, K tiles of 64, two stages. 128 x 128 tiles with 4
//     waves, two workgroups per CU; used for the other grids.
//   * gemm_bf16_kernel: register-staged loads with 16-byte-aligned fallbacks (any N % 64 == 0, any
//     output alignment).
// Common to all:
//   * LDS rows of 16-byte chunks XOR-swizzled so that the 16-byte fragment reads of 16 consecutive
//     rows cover all 64 LDS banks (measured: zero bank-conflict cycles).
//   * Rows of A beyond M are clamped to M-1 instead of predicated: they only feed output rows that
//     are never stored.
//   * Workgroups are renumbered so that consecutive tiles land on the same XCD (dispatch places
//     workgroup i on XCD i % 8): each XCD sweeps a contiguous band of the tile grid and reuses the
//     A rows and W columns of that band from its own L2.
//
// The epilogues fold in the elementwise work the reference runs as separate kernels after each
// Linear: bias, exact-erf GELU (fc1), LayerScale (fc2), LayerScale + residual (proj) and the SwiGLU
// gate, with a bf16 rounding at every point where the reference materialises a bf16 tensor.
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <type_traits>

#include "nvfp4.hpp"
#include "common.hpp"

namespace oudjat {

static constexpr int kBK = 64;
static constexpr int kNumXcd = 8;
static constexpr int kNumCus = 256;  // MI355X: 8 XCDs of 32 CUs

// Epilogue kind beyond the public ones: QKV projection followed by RoPE on q and k of patch rows,
// q written packed and k, v written into the K/V cache rows (used by oudjat_linear_qkv_rope_kv).
static constexpr int kEpiQkv = 5;
// Split-K partial: the 16-row-block kernel over one K slice (blockIdx.y) writes its fp32 accumulator
// tile to slice blockIdx.y of a [S, M, N] workspace; splitk_reduce_kernel sums the slices in order
// and applies the epilogue.
static constexpr int kEpiPartial = 6;
// SwiGLU of two NVFP4 linears in w2's epilogue (oudjat_linear_swiglu_nvfp4): the tile holds x2 =
// bf16(acc) (raw rounding, scale 1, no bias); phase 2 reads x1 (w1's bf16 output) as the residual row,
// forms swiglu_scaled8 and writes the NVFP4 operand x_hat of its bf16 value (w3's input).
static constexpr int kEpiSwigluXh = 7;
static constexpr int kNumEpi = 8;

struct QkvArgs {
  int H, Dh;
  const float* sin_t;
  const float* cos_t;
  int64_t tst;
  const uint8_t* pm;
  const int64_t* ridx;
  const int64_t* bi;
  const int64_t* ti;
  uint16_t* kv;
  int64_t kvb, kvn;
  uint16_t* q_out;
};

// The first rounding point of every epilogue is v = bf16(acc * acc_scale + bias) (one fp32 rounding:
// with acc_scale = 1 exactly bf16(acc + bias)); acc_scale carries the per-tensor factors of an FP8
// GEMM, which apply to the fp32 accumulator before its rounding.
struct EpiArgs {
  const uint16_t* bias;
  const uint16_t* gamma;
  const uint16_t* resid;
  int64_t ldr;
  QkvArgs qkv;
  float acc_scale;
  // NVFP4 linears (OUDJAT_EPI_RAW_BF16): the accumulator is rounded to bf16 before the scale and the
  // bias, v = bf16(bf16(acc) * raw_scale + raw_bias) -- the reference's _scaled_mm writes its bf16
  // output and scales it afterwards (fp4_fast_linear.py:221-283). The first rounding point then runs
  // with acc_scale = 1 and no bias (it gives bf16(acc) exactly) and raw_scale_bias8 follows it.
  int raw_round;
  float raw_scale;
  const uint16_t* raw_bias;
  // kEpiSwigluXh: w1's scale and bias (x1 = resid rows), w2's scale and bias, w3's NVFP4 tensor scale.
  float s1, s2;
  const uint16_t* b1;
  const uint16_t* b2;
  const float* xh_ts;
  // Cache warming (direct-to-LDS 16-row and ping-pong kernels, unsplit launches): workgroups
  // blockIdx.x >= work_tiles compute no tile; they read one dword of every 128-byte line of
  // warm[0 .. warm_lines * 32) (the weight of a later launch) and exit. work_tiles = 0: every
  // workgroup computes a tile.
  const uint32_t* warm;
  int64_t warm_lines;
  int work_tiles;
};

// A warming workgroup's share of the lines (part of parts), eight loads in flight per lane; the
// loaded words are consumed by an empty asm so that the loads stay.
__device__ __forceinline__ void warm_lines(const uint32_t* __restrict__ p, int64_t lines, int part, int parts) {
  const int64_t stride = (int64_t)parts * blockDim.x;
  int64_t l = (int64_t)part * blockDim.x + threadIdx.x;
  uint32_t acc = 0;
  for (; l + 7 * stride < lines; l += 8 * stride) {
    uint32_t v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = p[(l + u * stride) * 32];
#pragma unroll
    for (int u = 0; u < 8; ++u) acc ^= v[u];
  }
  for (; l < lines; l += stride) acc ^= p[l * 32];
  asm volatile("" ::"v"(acc));
}

// OUDJAT_EPI_RAW_BF16 on 8 consecutive bf16 values of columns col .. col + 7 (already bf16(acc)):
// bf16(v * raw_scale + raw_bias), or bf16(v * raw_scale) without a bias (scale_bias's arithmetic).
__device__ __forceinline__ uint4 raw_scale_bias8(uint4 o, int64_t col, const EpiArgs& ea) {
  float v[8], b[8];
  unpack8(o, v);
  if (ea.raw_bias) {
    unpack8(*reinterpret_cast<const uint4*>(ea.raw_bias + col), b);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = __builtin_fmaf(v[e], ea.raw_scale, b[e]);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = v[e] * ea.raw_scale;
  }
  return pack8(v);
}

// Two fp32 -> packed bf16 pair (low half = a) with the hardware round-to-nearest-even convert.
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t cvt_pk_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, bf16x2_t));
}

// GELU of a bf16 input as a table. The input of the GELU epilogue is already a bf16 value
// v = bf16(acc + bias), so the result bf16(0.5 v erfc(-v / sqrt 2)) is a function of 16 bits:
//   * |v| in [2^-16, 16) (magnitude bits 0x3780 .. 0x417f, both signs): 5120-entry table, filled
//     on the host from the double-precision erfc, rounded to fp32 and then RNE to bf16;
//   * |v| < 2^-16: 0.5 v exactly (the next term, v^2 / sqrt(2 pi), is below 2^-17 relative and
//     cannot move the rounding); bf16 subnormals and zeros give a signed zero;
//   * v >= 16: v;  v <= -16: -0.0 (the product underflows);  NaN: NaN;  -inf: NaN (as -inf * 0).
static constexpr int kGeluLut = 5120;
static constexpr uint32_t kGeluLo = 0x3780u, kGeluSpan = 0x0a00u;
__device__ uint16_t g_gelu_lut[kGeluLut];

__device__ __forceinline__ uint32_t gelu_bf16_bits(uint32_t b, const uint16_t* lut) {
  const uint32_t a = b & 0x7fffu;
  const uint32_t d = a - kGeluLo;  // unsigned: wraps for a < kGeluLo
  const uint32_t t = lut[min(d, kGeluSpan - 1u) + (b >> 15) * kGeluSpan];
  if (__builtin_expect(d < kGeluSpan, 1)) return t;
  if (a < kGeluLo) return a >= 0x0100u ? b - 0x80u : (b & 0x8000u);
  if ((b >> 15) == 0u) return b;
  return a == 0x7f80u ? 0x7fc0u : (a > 0x7f80u ? b : 0x8000u);
}

// Two bf16 GELUs per 32-bit word through the table, without branches in the common case: the
// packed 16-bit index (sign * span + clamped magnitude offset) is computed for both halves at once
// and both table entries are read unconditionally; `ok` is false when either half lies outside the
// table range, and the caller then redoes that word with gelu_bf16_bits.
typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t gelu_pair_bits(uint32_t w, const uint16_t* lut, bool& ok) {
  const u16x2_t v = __builtin_bit_cast(u16x2_t, w);
  const u16x2_t mag = v & (u16x2_t)(0x7fff);
  const u16x2_t d = mag - (u16x2_t)(kGeluLo);                           // wraps below the range
  const u16x2_t dc = __builtin_elementwise_min(d, (u16x2_t)(kGeluSpan - 1));
  const u16x2_t idx = (v >> (u16x2_t)(15)) * (u16x2_t)(kGeluSpan) + dc;  // < 2 * kGeluSpan
  ok = __builtin_bit_cast(uint32_t, dc) == __builtin_bit_cast(uint32_t, d);
  const uint32_t lo = lut[idx.x], hi = lut[idx.y];
  return lo | (hi << 16);
}

template <int EPI>
__device__ __forceinline__ float epilogue(float acc, int64_t row, int64_t col, const EpiArgs& ea) {
  float v = round_bf16(__builtin_fmaf(acc, ea.acc_scale, ea.bias ? bf16_to_f32(ea.bias[col]) : -0.0f));
  if (ea.raw_round)
    v = round_bf16(ea.raw_bias ? __builtin_fmaf(v, ea.raw_scale, bf16_to_f32(ea.raw_bias[col])) : v * ea.raw_scale);
  if (EPI == OUDJAT_EPI_BIAS_GELU) {
    v = __uint_as_float(gelu_bf16_bits(__float_as_uint(v) >> 16, g_gelu_lut) << 16);
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
    v = __uint_as_float(gelu_bf16_bits(__float_as_uint(v) >> 16, g_gelu_lut) << 16);
  } else if (EPI == OUDJAT_EPI_BIAS_LS_RESID) {
    v = fmaf(v, bf16_to_f32(ea.gamma[col]), bf16_to_f32(ea.resid[row * ea.ldr + col]));
  } else if (EPI == OUDJAT_EPI_BIAS_LS) {
    v = v * bf16_to_f32(ea.gamma[col]);
  } else if (EPI == OUDJAT_EPI_BIAS_SILU_MUL) {
    v = round_bf16(v / (1.0f + expf(-v))) * bf16_to_f32(ea.resid[row * ea.ldr + col]);
  }
  return v;
}

// Byte offset of 16-byte chunk `c` (K elements 8c .. 8c+7) of 128-byte LDS row `r`. The XOR with
// (r >> 1) & 7 spreads 16 consecutive rows read at one chunk over all 64 LDS banks (two rows share a
// 256-byte bank line, so rows r and r + 1 differ in line half and rows 2q apart in slot).
__device__ __forceinline__ int swz(int r, int c) { return r * 128 + ((c ^ ((r >> 1) & 7)) << 4); }


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

// Tile epilogue shared by the direct-to-LDS kernels. The MFMAs take W as their first operand, so
// block (i, j) holds the transposed product: lane l, register v -> row wm0 + 32 i + l % 32, column
// wn0 + 32 j + 8 (v / 4) + 4 (l / 32) + v % 4, i.e. every lane owns runs of 4 consecutive columns
// of one row. Phase 1: bf16(acc + bias) into LDS with 8-byte writes. Phase 2: the rest of the
// epilogue on 8 consecutive columns per lane, 16-byte global stores. Needs N % BN == 0, 16-byte
// aligned C / gamma / resid rows and an 8-byte aligned bias; the caller has passed a barrier
// after the last LDS read of the main loop.
// Phase 2 of the tile epilogue, shared by every kernel family: the bf16(acc + bias) tile sits in LDS
// (row pitch BN + 8 elements) and all NT threads finish the epilogue on 8 consecutive columns each.
template <int BM, int BN, int NT, int EPI>
__device__ __forceinline__ void store_tile_phase2(unsigned char* smem, const uint16_t* lut, int m0, int n0, int M,
                                                  const EpiArgs& ea, uint16_t* __restrict__ C, int64_t ldc) {
  constexpr int LDT = BN + 8;
  constexpr int NW = NT / 64;
  const uint16_t* ct = reinterpret_cast<const uint16_t*>(smem);
  if constexpr (EPI == kEpiQkv) {
    // One work item = (row, 8-wide chunk c of a head's left half); the item handles that chunk and
    // its partner c + Dh/2 in every head of the tile (Dh | BN), so the row's metadata and its four
    // RoPE table chunks (cos / sin at c and c + Dh/2) are loaded once for all of them: RoPE on q and
    // k of patch rows, then q packed or k / v into the cache row. Metadata of all of a thread's items
    // first, then their table chunks (one round trip each), then the heads.
    const QkvArgs& qa = ea.qkv;
    const int Dh = qa.Dh, HD = qa.H * Dh, half = Dh >> 1;
    const int cph = half >> 3;                               // chunks per half head (4 at Dh = 64)
    const int lg_cph = __builtin_ctz((unsigned)cph);
    const int nh = BN / Dh;                                  // heads in the tile
    const int n_items = BM * cph;
    constexpr int ITEMS = (BM * 8 + NW * 64 - 1) / (NW * 64);  // cph <= 8 (Dh <= 128)
    const bool tile_qk = n0 < 2 * HD;                        // some head of the tile is q or k
    bool rope[ITEMS];
    int64_t trow[ITEMS], rowq[ITEMS], kvrow[ITEMS];
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
      const int p = threadIdx.x + it * NW * 64;
      const int pc = p < n_items ? p : n_items - 1;
      const int rl = pc >> lg_cph, cc = pc & (cph - 1);
      const int row = min(m0 + rl, M - 1);
      const bool pm = qa.pm[row];
      const int64_t ri = qa.ridx[row], bi = qa.bi[row], ti = qa.ti[row];
      rope[it] = pm && tile_qk;
      trow[it] = (rope[it] ? ri * qa.tst : 0) + cc * 8;
      rowq[it] = (int64_t)row * HD;
      kvrow[it] = bi * qa.kvb + ti * qa.kvn;
    }
    float cl8[ITEMS][8], cr8[ITEMS][8], sl8[ITEMS][8], sr8[ITEMS][8];
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
      if (tile_qk && threadIdx.x + it * NW * 64 < n_items) {
        load8f(qa.cos_t + trow[it], cl8[it]);
        load8f(qa.cos_t + trow[it] + half, cr8[it]);
        load8f(qa.sin_t + trow[it], sl8[it]);
        load8f(qa.sin_t + trow[it] + half, sr8[it]);
      }
    }
#pragma unroll
    for (int it = 0; it < ITEMS; ++it) {
      const int p = threadIdx.x + it * NW * 64;
      const int rl = p >> lg_cph, cc = p & (cph - 1);
      if (p >= n_items || m0 + rl >= M) continue;
#pragma unroll
      for (int j = 0; j < BN / 16; ++j) {  // Dh >= 16
        if (j >= nh) break;
        const int c0 = j * Dh + cc * 8;
        const int colg = n0 + c0;
        const int which = colg >= 2 * HD ? 2 : (colg >= HD ? 1 : 0);
        const int hcol = colg - which * HD;  // column within q, k or v
        uint4 lo = *reinterpret_cast<const uint4*>(ct + rl * LDT + c0);
        uint4 hi = *reinterpret_cast<const uint4*>(ct + rl * LDT + c0 + half);
        if (ea.raw_round) {
          lo = raw_scale_bias8(lo, colg, ea);
          hi = raw_scale_bias8(hi, colg + half, ea);
        }
        if (which < 2 && rope[it]) {
          float l[8], rr[8];
          unpack8(lo, l);
          unpack8(hi, rr);
          rope8(l, rr, cl8[it], cr8[it], sl8[it], sr8[it]);
          lo = pack8(l);
          hi = pack8(rr);
        }
        uint16_t* d = which == 0 ? qa.q_out + rowq[it] + hcol : qa.kv + kvrow[it] + (which - 1) * HD + hcol;
        *reinterpret_cast<uint4*>(d) = lo;
        *reinterpret_cast<uint4*>(d + half) = hi;
      }
    }
    return;
  }
  constexpr int CPR = BN / 8;
  if constexpr (EPI == OUDJAT_EPI_BIAS_GELU) {
    // Fully unrolled: all LDS reads of a thread's chunks first (their latencies overlap), then
    // per chunk the table lookups and its store.
    // Chunks of rows at or past M are never stored: they are set to bf16 1.0 (inside the table
    // range) instead of read, so that their values (bf16(bias) on the zero-loaded rows, exactly zero
    // with zero biases, below the table range) cannot send the wave to the per-element path.
    constexpr int ITERS = (BM * CPR + NT - 1) / NT;
    uint4 o[ITERS];
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      const int c = threadIdx.x + it * NT;
      const int cc = c < BM * CPR ? c : BM * CPR - 1;
      const int rl = cc / CPR, cl = (cc - rl * CPR) * 8;
      o[it] = (c < BM * CPR && m0 + rl < M) ? *reinterpret_cast<const uint4*>(ct + rl * LDT + cl)
                                             : make_uint4(0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u);
    }
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      uint32_t* w = reinterpret_cast<uint32_t*>(&o[it]);
      bool ok0, ok1, ok2, ok3;
      const uint32_t g0 = gelu_pair_bits(w[0], lut, ok0), g1 = gelu_pair_bits(w[1], lut, ok1);
      const uint32_t g2 = gelu_pair_bits(w[2], lut, ok2), g3 = gelu_pair_bits(w[3], lut, ok3);
      const bool ok = ok0 && ok1 && ok2 && ok3;
      if (__builtin_expect(__builtin_amdgcn_ballot_w64(!ok) != 0, 0)) {
        if (!ok) {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            w[e] = gelu_bf16_bits(w[e] & 0xffffu, lut) | (gelu_bf16_bits(w[e] >> 16, lut) << 16);
        } else {
          w[0] = g0; w[1] = g1; w[2] = g2; w[3] = g3;
        }
      } else {
        w[0] = g0; w[1] = g1; w[2] = g2; w[3] = g3;
      }
      // Stored as soon as it is ready: the stores drain while the next chunks' lookups run.
      const int c = threadIdx.x + it * NT;
      const int rl = c / CPR, cl = (c - rl * CPR) * 8;
      const int row = m0 + rl;
      if (c < BM * CPR && row < M) *reinterpret_cast<uint4*>(C + (int64_t)row * ldc + n0 + cl) = o[it];
    }
    return;
  }
  if constexpr ((EPI == OUDJAT_EPI_BIAS_LS_RESID || EPI == OUDJAT_EPI_BIAS_SILU_MUL) && BN < 384) {
    // The epilogues that read a row segment (the residual or the gate) take their chunks in batches
    // of EB: every LDS read and global load (gamma, the row segment) of a batch is issued before
    // the first is used, so a batch costs one memory round trip instead of one per chunk; the
    // arithmetic is the per-chunk loop's below. (The 384-wide tiles keep that loop: their kernel has
    // no registers to spare for the batch.)
    constexpr int ITERS = (BM * CPR + NT - 1) / NT;
    constexpr int EB = 4;
#pragma unroll
    for (int b0 = 0; b0 < ITERS; b0 += EB) {
      uint4 o[EB], gv[EB], rv[EB];
      bool live[EB];
#pragma unroll
      for (int u = 0; u < EB; ++u) {
        const int c = threadIdx.x + (b0 + u) * NT;
        const int rl = c / CPR, cl = (c - rl * CPR) * 8;
        live[u] = b0 + u < ITERS && c < BM * CPR && m0 + rl < M;
        if (live[u]) {
          o[u] = *reinterpret_cast<const uint4*>(ct + rl * LDT + cl);
          if constexpr (EPI == OUDJAT_EPI_BIAS_LS_RESID) gv[u] = *reinterpret_cast<const uint4*>(ea.gamma + n0 + cl);
          rv[u] = *reinterpret_cast<const uint4*>(ea.resid + (int64_t)(m0 + rl) * ea.ldr + n0 + cl);
        }
      }
#pragma unroll
      for (int u = 0; u < EB; ++u) {
        if (!live[u]) continue;
        const int c = threadIdx.x + (b0 + u) * NT;
        const int rl = c / CPR, cl = (c - rl * CPR) * 8;
        const int row = m0 + rl, col = n0 + cl;
        uint4 w = o[u];
        if (ea.raw_round) w = raw_scale_bias8(w, col, ea);
        float v[8], g[8], r[8];
        unpack8(w, v);
        if constexpr (EPI == OUDJAT_EPI_BIAS_LS_RESID) unpack8(gv[u], g);
        unpack8(rv[u], r);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          if constexpr (EPI == OUDJAT_EPI_BIAS_LS_RESID) v[e] = fmaf(v[e], g[e], r[e]);
          else v[e] = round_bf16(v[e] / (1.0f + expf(-v[e]))) * r[e];
        }
        w.x = cvt_pk_bf16(v[0], v[1]);
        w.y = cvt_pk_bf16(v[2], v[3]);
        w.z = cvt_pk_bf16(v[4], v[5]);
        w.w = cvt_pk_bf16(v[6], v[7]);
        *reinterpret_cast<uint4*>(C + (int64_t)row * ldc + col) = w;
      }
    }
    return;
  }
  for (int c = threadIdx.x; c < BM * CPR; c += NW * 64) {
    const int rl = c / CPR, cl = (c - rl * CPR) * 8;
    const int row = m0 + rl, col = n0 + cl;
    if (row >= M) continue;
    uint4 o = *reinterpret_cast<const uint4*>(ct + rl * LDT + cl);
    if (ea.raw_round) o = raw_scale_bias8(o, col, ea);
    if constexpr (EPI == kEpiSwigluXh) {
      // A 16-element NVFP4 block is the chunk pair of threads 2k, 2k + 1 (one row: CPR is even), both
      // active or both skipped with their row.
      float x2[8], x1[8], ba[8], bb[8], y[8], h[8];
      unpack8(o, x2);
      unpack8(*reinterpret_cast<const uint4*>(ea.resid + (int64_t)row * ea.ldr + col), x1);
      if (ea.b1) {
        unpack8(*reinterpret_cast<const uint4*>(ea.b1 + col), ba);
        unpack8(*reinterpret_cast<const uint4*>(ea.b2 + col), bb);
      }
      swiglu_scaled8(x1, ea.s1, ba, x2, ea.s2, bb, ea.b1 != nullptr, y);
      unpack8(pack8(y), y);  // the bf16 SwiGLU output the quantizer reads
      nvfp4_xhat8_pair(y, *ea.xh_ts, h);
      *reinterpret_cast<uint4*>(C + (int64_t)row * ldc + col) = pack8(h);
      continue;
    }
    if constexpr (EPI != OUDJAT_EPI_BIAS && EPI != kEpiQkv) {
      // 16-byte loads of the per-column gamma and the residual / gate row segment.
      float v[8], g[8], r[8];
      unpack8(o, v);
      if constexpr (EPI == OUDJAT_EPI_BIAS_LS || EPI == OUDJAT_EPI_BIAS_LS_RESID)
        unpack8(*reinterpret_cast<const uint4*>(ea.gamma + col), g);
      if constexpr (EPI == OUDJAT_EPI_BIAS_LS_RESID || EPI == OUDJAT_EPI_BIAS_SILU_MUL)
        unpack8(*reinterpret_cast<const uint4*>(ea.resid + (int64_t)row * ea.ldr + col), r);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if constexpr (EPI == OUDJAT_EPI_BIAS_LS_RESID) v[e] = fmaf(v[e], g[e], r[e]);
        else if constexpr (EPI == OUDJAT_EPI_BIAS_LS) v[e] = v[e] * g[e];
        else v[e] = round_bf16(v[e] / (1.0f + expf(-v[e]))) * r[e];
      }
      o.x = cvt_pk_bf16(v[0], v[1]);
      o.y = cvt_pk_bf16(v[2], v[3]);
      o.z = cvt_pk_bf16(v[4], v[5]);
      o.w = cvt_pk_bf16(v[6], v[7]);
    }
    *reinterpret_cast<uint4*>(C + (int64_t)row * ldc + col) = o;
  }
}

template <int BM, int BN, int FM, int FN, int NW, int EPI>
__device__ __forceinline__ void store_tile(const f32x16_t (&acc)[FM][FN], unsigned char* smem, const uint16_t* lut,
                                           int wm0, int wn0, int m0, int n0, int M, const EpiArgs& ea,
                                           uint16_t* __restrict__ C, int64_t ldc) {
  const int lane = threadIdx.x & 63;
  constexpr int LDT = BN + 8;
  uint16_t* ct = reinterpret_cast<uint16_t*>(smem);
#pragma unroll
  for (int j = 0; j < FN; ++j) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int cl = wn0 + j * 32 + g * 8 + 4 * (lane >> 5);
      float b0 = -0.0f, b1 = -0.0f, b2 = -0.0f, b3 = -0.0f;
      if (ea.bias) {
        const uint2 bw = *reinterpret_cast<const uint2*>(ea.bias + n0 + cl);
        b0 = lo_bf16(bw.x); b1 = hi_bf16(bw.x); b2 = lo_bf16(bw.y); b3 = hi_bf16(bw.y);
      }
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int rl = wm0 + i * 32 + (lane & 31);
        uint2 w;
        w.x = cvt_pk_bf16(__builtin_fmaf(acc[i][j][4 * g + 0], ea.acc_scale, b0),
                          __builtin_fmaf(acc[i][j][4 * g + 1], ea.acc_scale, b1));
        w.y = cvt_pk_bf16(__builtin_fmaf(acc[i][j][4 * g + 2], ea.acc_scale, b2),
                          __builtin_fmaf(acc[i][j][4 * g + 3], ea.acc_scale, b3));
        *reinterpret_cast<uint2*>(ct + rl * LDT + cl) = w;
      }
    }
  }
  __syncthreads();
  store_tile_phase2<BM, BN, NW * 64, EPI>(smem, lut, m0, n0, M, ea, C, ldc);
}

// Copies the GELU table into LDS at `dst` (16-byte aligned).
template <int NT>
__device__ __forceinline__ void load_gelu_table(unsigned char* dst) {
  for (int i = threadIdx.x; i < kGeluLut / 8; i += NT)
    reinterpret_cast<uint4*>(dst)[i] = reinterpret_cast<const uint4*>(g_gelu_lut)[i];
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

// LDS bytes of the direct-to-LDS kernel before the GELU table: two K stages or the epilogue tile.
__host__ __device__ constexpr int dma_lut_offset(int bm, int bn) {
  return 2 * (bm + bn) * 128 > bm * (bn + 8) * 2 ? 2 * (bm + bn) * 128 : bm * (bn + 8) * 2;
}

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
  if constexpr (EPI == OUDJAT_EPI_BIAS_GELU) load_gelu_table<NW * 64>(smem + dma_lut_offset(BM, BN));

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

  // Lane l fills slot l % 8 of its row, i.e. global K chunk (l % 8) ^ swizzle(row).
  const uint16_t* a_src[AG];
  const uint16_t* b_src[BG];
#pragma unroll
  for (int i = 0; i < AG; ++i) {
    const int row = (wave * AG + i) * 8 + lrow;
    a_src[i] = A + (int64_t)min(m0 + row, M - 1) * lda + ((lane & 7) ^ ((row >> 1) & 7)) * 8;
  }
#pragma unroll
  for (int i = 0; i < BG; ++i) {
    const int row = (wave * BG + i) * 8 + lrow;
    b_src[i] = W + (int64_t)min(n0 + row, N - 1) * ldw + ((lane & 7) ^ ((row >> 1) & 7)) * 8;
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
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[j], fa[i], acc[i][j], 0, 0, 0);
    }
  }

  __syncthreads();
  store_tile<BM, BN, FM, FN, NW, EPI>(acc, smem, reinterpret_cast<const uint16_t*>(smem + dma_lut_offset(BM, BN)), wm0,
                                      wn0, m0, n0, M, ea, C, ldc);
}

// ------------------------------------------------------------------------------------------------
// Deep-pipelined direct-to-LDS kernel. K tiles of 32 (64-byte LDS rows), 4 LDS stages, operand
// loads issued three K tiles ahead of the MFMAs that consume them, one workgroup per CU.
//
//   * Swizzle: chunk c of row r sits at 16-byte slot c ^ ((r >> 2) & 3). A wave reading one chunk
//     of 16 consecutive rows (one quarter of a fragment read) then covers all 64 LDS banks once.
//   * Loads: one global_load_lds_dwordx4 fills 16 consecutive 64-byte rows (lane l -> row l / 4,
//     slot l % 4, i.e. global chunk (l % 4) ^ ((l / 16) % 4)). The (BM + BN) / 16 instructions of a
//     K tile are dealt round-robin to the waves.
//   * Per K tile: wait for this wave's loads of the tile (vmcnt), one s_barrier (every wave's loads
//     landed, every wave done reading the stage about to be refilled), issue the loads of tile
//     kt + 3 into that stage, then 2 x FM x FN MFMAs with all fragments read up front.
// ------------------------------------------------------------------------------------------------

static constexpr int kBK3 = 32;
static constexpr int kStages = 4;

__device__ __forceinline__ int swz64(int r, int c) { return r * 64 + ((c ^ ((r >> 2) & 3)) << 4); }

__device__ __forceinline__ void wait_vmcnt_rt(int n) {
  switch (n) {
    case 0: wait_vmcnt<0>(); break;
    case 1: wait_vmcnt<1>(); break;
    case 2: wait_vmcnt<2>(); break;
    case 3: wait_vmcnt<3>(); break;
    case 4: wait_vmcnt<4>(); break;
    case 5: wait_vmcnt<5>(); break;
    case 6: wait_vmcnt<6>(); break;
    case 7: wait_vmcnt<7>(); break;
    case 8: wait_vmcnt<8>(); break;
    case 9: wait_vmcnt<9>(); break;
    case 10: wait_vmcnt<10>(); break;
    case 11: wait_vmcnt<11>(); break;
    case 12: wait_vmcnt<12>(); break;
    case 13: wait_vmcnt<13>(); break;
    case 14: wait_vmcnt<14>(); break;
    case 15: wait_vmcnt<15>(); break;
    case 16: wait_vmcnt<16>(); break;
    case 17: wait_vmcnt<17>(); break;
    case 18: wait_vmcnt<18>(); break;
    case 19: wait_vmcnt<19>(); break;
    case 20: wait_vmcnt<20>(); break;
    case 21: wait_vmcnt<21>(); break;
    case 22: wait_vmcnt<22>(); break;
    case 23: wait_vmcnt<23>(); break;
    default: wait_vmcnt<24>(); break;
  }
}

// LDS bytes of the pipelined kernel before the GELU table: K stages or the epilogue tile.
__host__ __device__ constexpr int pipe_lut_offset(int bm, int bn) {
  return kStages * (bm + bn) * 64 > bm * (bn + 8) * 2 ? kStages * (bm + bn) * 64 : bm * (bn + 8) * 2;
}

template <int BM, int BN, int WGM, int WGN, int EPI>
__global__ __launch_bounds__(WGM * WGN * 64) __attribute__((amdgpu_waves_per_eu(WGM * WGN / 4, WGM * WGN / 4)))
void gemm_bf16_pipe_kernel(const uint16_t* __restrict__ A, int M, int K, int64_t lda, const uint16_t* __restrict__ W,
                           int N, int64_t ldw, EpiArgs ea, uint16_t* __restrict__ C, int64_t ldc, int group_m) {
  constexpr int NW = WGM * WGN;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int FM = WM / 32, FN = WN / 32;
  constexpr int NI = (BM + BN) / 16;              // load instructions per K tile
  constexpr int NLM = (NI + NW - 1) / NW;         // per wave, at most
  constexpr int STAGE = (BM + BN) * 64;
  static_assert(BM % 16 == 0 && BN % 16 == 0 && FM >= 1 && FN >= 1 && WM % 32 == 0 && WN % 32 == 0, "tile shape");

  extern __shared__ __align__(16) unsigned char smem[];
  // LDS: K stages (later the epilogue tile), then the GELU table for the GELU epilogue.
  constexpr int kLutOff = pipe_lut_offset(BM, BN);
  if constexpr (EPI == OUDJAT_EPI_BIAS_GELU) load_gelu_table<NW * 64>(smem + kLutOff);

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
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform, kept in SGPRs
  const int wm0 = (wave / WGN) * WM;
  const int wn0 = (wave % WGN) * WN;

  // This wave's load instructions: i = wave + j * NW.
  const int nl = (NI % NW == 0) ? NI / NW : (NI - wave + NW - 1) / NW;
  const uint16_t* src[NLM];
  int dst[NLM];
  {
    const int lrow = lane >> 2;
    const int lchunk = (lane & 3) ^ ((lane >> 4) & 3);
#pragma unroll
    for (int j = 0; j < NLM; ++j) {
      const int i = min(wave + j * NW, NI - 1);
      dst[j] = i * 1024;
      if (i < BM / 16) {
        src[j] = A + (int64_t)min(m0 + i * 16 + lrow, M - 1) * lda + lchunk * 8;
      } else {
        src[j] = W + (int64_t)min(n0 + (i - BM / 16) * 16 + lrow, N - 1) * ldw + lchunk * 8;
      }
    }
  }
  const int KT = K / kBK3;
  auto issue = [&](int stage, int kt) __attribute__((always_inline)) {
    unsigned char* base = smem + stage * STAGE;
    const int k0 = kt * kBK3;
#pragma unroll
    for (int j = 0; j < NLM; ++j)
      if (j < nl)
        __builtin_amdgcn_global_load_lds((const void*)(src[j] + k0), (lds_ptr_t)(base + dst[j]), 16, 0, 0);
  };

  f32x16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  // Fragment offsets: lane l reads row (l % 32) of each 32-row block at K chunk 2 * ks + l / 32.
  const int sw = (lane >> 2) & 3;
  const int a_lane = (wm0 + (lane & 31)) * 64;
  const int b_lane = BM * 64 + (wn0 + (lane & 31)) * 64;
  const int co0 = ((0 + (lane >> 5)) ^ sw) << 4;
  const int co1 = ((2 + (lane >> 5)) ^ sw) << 4;

  // Fragments of one K tile: [ks][block] for A and B, read one tile ahead of their MFMAs.
  struct Frags {
    bf16x8_t a[2][FM], b[2][FN];
  };
  auto read_frags = [&](Frags& f, int kt) __attribute__((always_inline)) {
    const unsigned char* st = smem + (kt & (kStages - 1)) * STAGE;
#pragma unroll
    for (int i = 0; i < FM; ++i) f.a[0][i] = *reinterpret_cast<const bf16x8_t*>(st + a_lane + i * 2048 + co0);
#pragma unroll
    for (int j = 0; j < FN; ++j) f.b[0][j] = *reinterpret_cast<const bf16x8_t*>(st + b_lane + j * 2048 + co0);
#pragma unroll
    for (int i = 0; i < FM; ++i) f.a[1][i] = *reinterpret_cast<const bf16x8_t*>(st + a_lane + i * 2048 + co1);
#pragma unroll
    for (int j = 0; j < FN; ++j) f.b[1][j] = *reinterpret_cast<const bf16x8_t*>(st + b_lane + j * 2048 + co1);
  };
  // Row blocks at or past M (ragged last tile row) compute on clamped A rows and are never stored;
  // a branch per row block would drain the prefetched fragments at every block boundary.
  auto mfmas = [&](const Frags& f) __attribute__((always_inline)) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.b[ks][j], f.a[ks][i], acc[i][j], 0, 0, 0);
  };
  // Wait until at most `n_after` K tiles of this wave's loads are still in flight.
  auto wait_tiles = [&](int n_after) __attribute__((always_inline)) {
    if constexpr (NI % NW == 0) {
      if (n_after >= 3) wait_vmcnt<3 * (NI / NW)>();
      else if (n_after == 2) wait_vmcnt<2 * (NI / NW)>();
      else if (n_after == 1) wait_vmcnt<NI / NW>();
      else wait_vmcnt<0>();
    } else {
      wait_vmcnt_rt(n_after * nl);
    }
  };

  // Pipeline: at the top of step kt the stages hold tiles kt+1 .. kt+3 (landed or in flight) and
  // tile kt's fragments are already in registers, so tile kt's stage is free for tile kt+4.
  //   wait for tile kt+1; barrier; issue tile kt+4; read tile kt+1's fragments; MFMAs of tile kt.
#pragma unroll
  for (int s = 0; s < kStages; ++s)
    if (s < KT) issue(s, s);
  wait_tiles(min(KT - 1, kStages - 1));
  block_barrier();
  Frags f0, f1;
  read_frags(f0, 0);

  auto step = [&](int kt, Frags& cur, Frags& nxt) __attribute__((always_inline)) {
    if (kt + 1 < KT) {
      wait_tiles(min(KT - 2 - kt, kStages - 2));
      block_barrier();
      if (kt + kStages < KT) issue(kt & (kStages - 1), kt + kStages);
      __builtin_amdgcn_sched_barrier(0);
      read_frags(nxt, kt + 1);
    }
    mfmas(cur);
    __builtin_amdgcn_sched_barrier(0);
  };
  int kt = 0;
  for (; kt + 1 < KT; kt += 2) {
    step(kt, f0, f1);
    step(kt + 1, f1, f0);
  }
  if (kt < KT) step(kt, f0, f1);

  block_barrier();
  store_tile<BM, BN, FM, FN, NW, EPI>(acc, smem, reinterpret_cast<const uint16_t*>(smem + kLutOff), wm0, wn0, m0, n0,
                                      M, ea, C, ldc);
}

// ------------------------------------------------------------------------------------------------
// 16-row-block kernel for M = 144 k-multiples. The correction pass's GEMMs have M = B * (5 + k)
// rows (4176 = 29 x 144 at the headline shape), which 256-row tiles cover badly (17 tile rows, the
// last one 31 % full). Tiles of 144 rows (9 blocks of 16) on v_mfma_f32_16x16x32_bf16 cover it
// exactly: fc1 as 29 x 8 tiles of 144 x 512, the N = C GEMMs as 29 x 8 tiles of 144 x 128 -- 232
// workgroups, one round on 256 CUs.
//   * Waves form a WGM x WGN grid of BM / WGM-row, BN / WGN-column wave tiles; with KSPLIT = 2 two
//     such grids take alternate 32-deep halves of each K tile (doubling the waves per CU for the
//     narrow N = C tiles) and are summed through LDS at the end. With WGM = 2 (288-row tiles of two
//     144-row halves) the epilogue stages one half at a time through LDS.
//   * K tiles of BK (32 or 64) in NST LDS stages, direct-to-LDS loads issued NST - 1 tiles ahead,
//     fragments read one K tile ahead of their MFMAs, one barrier per K tile.
//   * Rows are 2 * BK bytes; chunk c of row r sits at 16-byte slot c ^ ((r / L) % CPRW) with
//     L = rows per 256-byte bank line and CPRW = chunks per row, so a fragment read (16 rows at one
//     chunk per 16 lanes) covers all 64 banks.
// ------------------------------------------------------------------------------------------------

template <int BK>
struct R16Layout {
  static constexpr int kRowBytes = 2 * BK;
  static constexpr int kChunks = BK / 8;             // 16-byte chunks per row
  static constexpr int kRowsPerLine = 256 / kRowBytes;
  static constexpr int kRowsPerLoad = 1024 / kRowBytes;  // rows one global_load_lds instruction fills
  __device__ static __forceinline__ int swz(int r, int c) {
    return r * kRowBytes + ((c ^ ((r / kRowsPerLine) % kChunks)) << 4);
  }
};

// LDS bytes before the GELU table: K stages, or the KSPLIT reduction buffer plus the bf16 tile of one
// wave row (BM / WGM rows), whichever is larger.
__host__ __device__ constexpr int r16_lut_offset(int bm, int bn, int wgm, int wgn, int ksplit, int bk, int nst) {
  const int stages = nst * (bm + bn) * 2 * bk;
  // The whole bf16 tile when it fits next to the GELU table in the 160 KB of LDS (the epilogue then
  // runs in one pass), else one wave row's share.
  const int full = bm * (bn + 8) * 2;
  const int tile = (ksplit == 1 && wgm > 1 && full + 2 * kGeluLut <= 160 * 1024) ? full : (bm / wgm) * (bn + 8) * 2;
  const int red = ksplit > 1 ? wgm * wgn * 64 * (bm / wgm / 16) * (bn / wgn / 16) * 4 * 4 : 0;  // fp32 partials
  const int epi = red + tile;
  return stages > epi ? stages : epi;
}

// Epilogue of the 16-row-block kernels. Block (i, j) of a wave holds the transposed product: lane l,
// register v -> row wm0 + i * 16 + l % 16, column wn0 + j * 16 + 4 (l / 16) + v. With two K groups,
// group 1's partial sums are added into group 0's through LDS first. Then one wave row at a time
// writes bf16(acc + bias) into an LDS tile and every thread finishes the epilogue of those rows.
// The caller's LDS stages must be free (no wave still reads them); this function begins with a barrier.
// TILE_BYTES: LDS the caller can give the bf16 tile (0: unknown). When the whole BM-row tile fits,
// all wave rows write it at once and phase 2 runs once over all rows (one latency chain of its
// loads instead of one per wave row).
template <int BM, int BN, int WGM, int WGN, int KSPLIT, int FMB, int FNB, int EPI, int TILE_BYTES = 0>
__device__ __forceinline__ void r16_epilogue(f32x4_t (&acc)[FMB][FNB], unsigned char* smem, int kLutOff, int kg, int wr,
                                             int wm, int wn0, int lane, int m0, int n0, int M, const EpiArgs& ea,
                                             uint16_t* __restrict__ C, int64_t ldc) {
  constexpr int NWG = WGM * WGN;
  constexpr int NT = NWG * KSPLIT * 64;
  constexpr int WM = BM / WGM;
  constexpr int LDT = BN + 8;
  constexpr int RED = KSPLIT > 1 ? NWG * 64 * FMB * FNB * 4 * 4 : 0;  // fp32 partial bytes
  uint16_t* ct = reinterpret_cast<uint16_t*>(smem + RED);
  block_barrier();
  // With two K groups, group 0 finishes row blocks [0, HB) and group 1 row blocks [HB, FMB): each
  // parks the other's blocks in LDS ([block][register][thread] fp32),
  // adds the blocks parked for it (a + b is the same float in either order) and moves them to
  // acc[0, HB) (selects on the group with static indices, so the accumulators stay in registers).
  // Both groups then write their blocks of the bf16 tile below, at row block i + kg * HB.
  static_assert(KSPLIT <= 2, "two K groups at most");
  constexpr int HB = KSPLIT == 2 ? (FMB + 1) / 2 : FMB;
  if constexpr (KSPLIT == 2) {
    float* red = reinterpret_cast<float*>(smem);
    const int t0 = wr * 64 + lane;
    const bool g0 = kg == 0;
#pragma unroll
    for (int i = 0; i < HB; ++i) {
      if (i + HB >= FMB && g0) continue;
      const int blk = g0 ? i + HB : i;  // block parked: one the other group finishes
#pragma unroll
      for (int j = 0; j < FNB; ++j)
#pragma unroll
        for (int v = 0; v < 4; ++v)
          red[((blk * FNB + j) * 4 + v) * (NWG * 64) + t0] = (i + HB < FMB && g0) ? acc[i + HB < FMB ? i + HB : i][j][v] : acc[i][j][v];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < HB; ++i) {
      if (i + HB >= FMB && !g0) continue;
      const int blk = g0 ? i : i + HB;  // block this group finishes
#pragma unroll
      for (int j = 0; j < FNB; ++j)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float mine = (i + HB < FMB && !g0) ? acc[i + HB < FMB ? i + HB : i][j][v] : acc[i][j][v];
          acc[i][j][v] = mine + red[((blk * FNB + j) * 4 + v) * (NWG * 64) + t0];
        }
    }
  }
  if constexpr (EPI == kEpiPartial) {
    // fp32 partial tile: lane holds 4 consecutive columns of row (lane & 15) of each 16-row block.
    float* P = reinterpret_cast<float*>(C) + (int64_t)blockIdx.y * M * ldc;
    const int rb0 = KSPLIT == 2 ? kg * HB : 0;
#pragma unroll
    for (int j = 0; j < FNB; ++j) {
      const int col = n0 + wn0 + j * 16 + 4 * (lane >> 4);
#pragma unroll
      for (int i = 0; i < HB; ++i) {
        if (rb0 + i >= FMB) continue;
        const int row = m0 + wm * WM + (rb0 + i) * 16 + (lane & 15);
        if (row < M) *reinterpret_cast<f32x4_t*>(P + (int64_t)row * ldc + col) = acc[i][j];
      }
    }
    return;
  }
  if constexpr (WGM > 1 && KSPLIT == 1 && RED == 0 && BM * LDT * 2 <= TILE_BYTES) {
#pragma unroll
    for (int j = 0; j < FNB; ++j) {
      const int cl = wn0 + j * 16 + 4 * (lane >> 4);
      float b0 = -0.0f, b1 = -0.0f, b2 = -0.0f, b3 = -0.0f;
      if (ea.bias) {
        const uint2 bw = *reinterpret_cast<const uint2*>(ea.bias + n0 + cl);
        b0 = lo_bf16(bw.x); b1 = hi_bf16(bw.x); b2 = lo_bf16(bw.y); b3 = hi_bf16(bw.y);
      }
#pragma unroll
      for (int i = 0; i < FMB; ++i) {
        uint2 w;
        w.x = cvt_pk_bf16(__builtin_fmaf(acc[i][j][0], ea.acc_scale, b0), __builtin_fmaf(acc[i][j][1], ea.acc_scale, b1));
        w.y = cvt_pk_bf16(__builtin_fmaf(acc[i][j][2], ea.acc_scale, b2), __builtin_fmaf(acc[i][j][3], ea.acc_scale, b3));
        *reinterpret_cast<uint2*>(ct + (wm * WM + i * 16 + (lane & 15)) * LDT + cl) = w;
      }
    }
    __syncthreads();
    store_tile_phase2<BM, BN, NT, EPI>(reinterpret_cast<unsigned char*>(ct),
                                       reinterpret_cast<const uint16_t*>(smem + kLutOff), m0, n0, M, ea, C, ldc);
    return;
  }
  // One wave row at a time: its waves write bf16(acc + bias) into the LDS tile, then every thread
  // finishes the epilogue of those WM rows.
#pragma unroll
  for (int h = 0; h < WGM; ++h) {
    // Wave rows that start at or past M hold only rows that are never stored (the second half of
    // the last 288-row tile at M = 14.5 x 288): skip them (block-uniform, so the barriers still pair).
    if (m0 + h * WM >= M) break;
    if (h > 0) __syncthreads();
    if (wm == h) {
      const int rb0 = KSPLIT == 2 ? kg * HB : 0;  // row block of acc[0]
#pragma unroll
      for (int j = 0; j < FNB; ++j) {
        const int cl = wn0 + j * 16 + 4 * (lane >> 4);
        float b0 = -0.0f, b1 = -0.0f, b2 = -0.0f, b3 = -0.0f;
        if (ea.bias) {
          const uint2 bw = *reinterpret_cast<const uint2*>(ea.bias + n0 + cl);
          b0 = lo_bf16(bw.x); b1 = hi_bf16(bw.x); b2 = lo_bf16(bw.y); b3 = hi_bf16(bw.y);
        }
#pragma unroll
        for (int i = 0; i < HB; ++i) {
          if (rb0 + i >= FMB) continue;
          uint2 w;
          w.x = cvt_pk_bf16(__builtin_fmaf(acc[i][j][0], ea.acc_scale, b0),
                            __builtin_fmaf(acc[i][j][1], ea.acc_scale, b1));
          w.y = cvt_pk_bf16(__builtin_fmaf(acc[i][j][2], ea.acc_scale, b2),
                            __builtin_fmaf(acc[i][j][3], ea.acc_scale, b3));
          *reinterpret_cast<uint2*>(ct + ((rb0 + i) * 16 + (lane & 15)) * LDT + cl) = w;
        }
      }
    }
    __syncthreads();
    store_tile_phase2<WM, BN, NT, EPI>(reinterpret_cast<unsigned char*>(ct),
                                       reinterpret_cast<const uint16_t*>(smem + kLutOff), m0 + h * WM, n0, M, ea, C,
                                       ldc);
  }
}

// FB: fragments read one K tile ahead (double-buffered registers); without it they are read right
// after the barrier of their own K tile (for wave tiles whose accumulators leave no room).
template <int BM, int BN, int WGM, int WGN, int KSPLIT, int BK, int NST, bool FB, int EPI>
__global__ __launch_bounds__(WGM * WGN * KSPLIT * 64) __attribute__((amdgpu_waves_per_eu(
    (WGM * WGN * KSPLIT + 3) / 4, (WGM * WGN * KSPLIT + 3) / 4)))
void gemm_bf16_r16_kernel(const uint16_t* __restrict__ A, int M, int K, int64_t lda, const uint16_t* __restrict__ W,
                          int N, int64_t ldw, EpiArgs ea, uint16_t* __restrict__ C, int64_t ldc, int group_m) {
  using L = R16Layout<BK>;
  constexpr int NWG = WGM * WGN;                  // waves of one K group
  constexpr int NW = NWG * KSPLIT;
  constexpr int NT = NW * 64;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int FMB = WM / 16, FNB = WN / 16;     // 16 x 16 blocks per wave
  constexpr int SUB = BK / 32;                    // 32-deep MFMA steps per K tile
  constexpr int SUBW = SUB / KSPLIT;              // ... per wave
  constexpr int NI = (BM + BN) / L::kRowsPerLoad; // load instructions per K tile
  constexpr int NLM = (NI + NW - 1) / NW;
  constexpr int STAGE = (BM + BN) * L::kRowBytes;
  static_assert(BM % L::kRowsPerLoad == 0 && BN % L::kRowsPerLoad == 0, "rows must fill whole load instructions");
  static_assert(SUB % KSPLIT == 0 && SUBW >= 1 && WM % 16 == 0 && WN % 16 == 0 && NST >= 2, "tile shape");

  extern __shared__ __align__(16) unsigned char smem[];
  const int tiles = ea.work_tiles > 0 ? ea.work_tiles : (int)gridDim.x;
  if ((int)blockIdx.x >= tiles) {  // a warming workgroup
    warm_lines(ea.warm, ea.warm_lines, (int)blockIdx.x - tiles, (int)gridDim.x - tiles);
    return;
  }
  constexpr int kLutOff = r16_lut_offset(BM, BN, WGM, WGN, KSPLIT, BK, NST);
  if constexpr (EPI == OUDJAT_EPI_BIAS_GELU) load_gelu_table<NT>(smem + kLutOff);
  if constexpr (EPI == kEpiPartial) {  // K slice blockIdx.y of length K (lda, ldw stay the full strides)
    A += (int64_t)blockIdx.y * K;
    W += (int64_t)blockIdx.y * K;
  }

  const int tiles_n = (N + BN - 1) / BN;
  const int tiles_m = (M + BM - 1) / BM;
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
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kg = wave / NWG;                // K group
  const int wr = wave - kg * NWG;           // wave within its K group
  const int wm = wr / WGN;                  // wave row
  const int wm0 = wm * WM;                  // first tile row of the wave
  const int wn0 = (wr % WGN) * WN;          // column strip

  // Loads: instruction i = wave + j * NW fills rows [i * RPL, (i + 1) * RPL) of the stage, A rows
  // first, then W rows, through buffer descriptors: a lane keeps one 32-bit byte offset per operand
  // (its row within instruction j = 0 plus its swizzled chunk) and instruction j adds j * NW * RPL
  // rows, so no per-instruction address registers are live across the K loop. A rows at or past M
  // fall outside the A descriptor and load as zeros.
  static_assert(NW % 2 == 0, "the chunk swizzle of a lane must not depend on j");
  const int nl = (NI - wave + NW - 1) / NW;
  const i32x4_t rsrc_a = make_buffer_rsrc(A, (uint32_t)((int64_t)M * lda * 2));
  const i32x4_t rsrc_w = make_buffer_rsrc(W, (uint32_t)((int64_t)N * ldw * 2));
  uint32_t voff_a, voff_w;
  {
    const int lrow = lane / L::kChunks, lslot = lane % L::kChunks;
    const int row0 = wave * L::kRowsPerLoad + lrow;  // stage row of instruction j = 0
    const int chunk = lslot ^ ((row0 / L::kRowsPerLine) % L::kChunks);
    voff_a = (uint32_t)((m0 + row0) * (uint32_t)lda * 2u + chunk * 16);
    voff_w = (uint32_t)((n0 + row0 - BM) * (uint32_t)ldw * 2u + chunk * 16);
  }
  const uint32_t step_a = (uint32_t)(NW * L::kRowsPerLoad) * (uint32_t)lda * 2u;
  const uint32_t step_w = (uint32_t)(NW * L::kRowsPerLoad) * (uint32_t)ldw * 2u;
  auto issue = [&](int stage, int kt) __attribute__((always_inline)) {
    unsigned char* base = smem + stage * STAGE;
    const uint32_t koff = (uint32_t)(kt * BK * 2);
#pragma unroll
    for (int j = 0; j < NLM; ++j) {
      if (j < NLM - 1 || j < nl) {
        const int i = wave + j * NW;
        if (i < BM / L::kRowsPerLoad)
          buffer_load_lds16(rsrc_a, base + i * 1024, voff_a + (uint32_t)j * step_a + koff);
        else
          buffer_load_lds16(rsrc_w, base + i * 1024, voff_w + (uint32_t)j * step_w + koff);
      }
    }
  };
  // Waves 0 .. NI % NW - 1 issue NLM loads per tile, the others NLM - 1 (all NLM if NW | NI); the
  // vmcnt immediates are compile-time per class, so the wait is a uniform branch, not a switch.
  auto wait_tiles = [&](int n_after) __attribute__((always_inline)) {
    constexpr int NRED = (NI % NW == 0) ? NLM : NLM - 1;
    const bool full = (NI % NW == 0) || wave < NI % NW;
    if (n_after <= 0) {
      wait_vmcnt<0>();
    } else if (n_after == 1) {
      if (full) wait_vmcnt<NLM>(); else wait_vmcnt<NRED>();
    } else if (n_after == 2) {
      if (full) wait_vmcnt<2 * NLM>(); else wait_vmcnt<2 * NRED>();
    } else {
      static_assert(NST <= 4 && 3 * NLM < 64, "vmcnt range");
      if (full) wait_vmcnt<3 * NLM>(); else wait_vmcnt<3 * NRED>();
    }
  };

  f32x4_t acc[FMB][FNB];
#pragma unroll
  for (int i = 0; i < FMB; ++i)
#pragma unroll
    for (int j = 0; j < FNB; ++j) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  // Fragments (16x16x32): lane l reads row l % 16 of a 16-row block at K chunk 4 * sub + l / 16.
  struct Frags {
    bf16x8_t a[SUBW][FMB], b[SUBW][FNB];
  };
  auto read_frags = [&](Frags& f, int kt) __attribute__((always_inline)) {
    const unsigned char* st = smem + (kt % NST) * STAGE;
#pragma unroll
    for (int s = 0; s < SUBW; ++s) {
      const int ch = 4 * (s * KSPLIT + kg) + (lane >> 4);
#pragma unroll
      for (int i = 0; i < FMB; ++i)
        f.a[s][i] = *reinterpret_cast<const bf16x8_t*>(st + L::swz(wm0 + i * 16 + (lane & 15), ch));
#pragma unroll
      for (int j = 0; j < FNB; ++j)
        f.b[s][j] = *reinterpret_cast<const bf16x8_t*>(st + L::swz(BM + wn0 + j * 16 + (lane & 15), ch));
    }
  };
  // Row blocks at or past M (the last tile row of a ragged M) run their MFMAs on clamped A rows and
  // are never stored: skipping them would not shorten the single round of tiles, and a branch per
  // row block would make the compiler drain the prefetched fragments at every block boundary.
  auto mfmas = [&](const Frags& f) __attribute__((always_inline)) {
#pragma unroll
    for (int s = 0; s < SUBW; ++s)
#pragma unroll
      for (int i = 0; i < FMB; ++i)
#pragma unroll
        for (int j = 0; j < FNB; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f.b[s][j], f.a[s][i], acc[i][j], 0, 0, 0);
  };

  const int KT = K / BK;
#pragma unroll
  for (int s = 0; s < NST; ++s)
    if (s < KT) issue(s, s);
  if constexpr (FB) {
    wait_tiles(min(KT - 1, NST - 1));
    block_barrier();
    Frags f0, f1;
    read_frags(f0, 0);
    // Step kt: wait for tile kt + 1, barrier, refill tile kt's stage with tile kt + NST, read tile
    // kt + 1's fragments, MFMAs of tile kt.
    auto step = [&](int kt, Frags& cur, Frags& nxt) __attribute__((always_inline)) {
      if (kt + 1 < KT) {
        wait_tiles(min(KT - 2 - kt, NST - 2));
        block_barrier();
        if (kt + NST < KT) issue(kt % NST, kt + NST);
        __builtin_amdgcn_sched_barrier(0);
        read_frags(nxt, kt + 1);
      }
      mfmas(cur);
      __builtin_amdgcn_sched_barrier(0);
    };
    int kt = 0;
    for (; kt + 1 < KT; kt += 2) {
      step(kt, f0, f1);
      step(kt + 1, f1, f0);
    }
    if (kt < KT) step(kt, f0, f1);
  } else {
    // Step kt: wait for tile kt, barrier (also: every wave is done with tile kt - 1's stage), refill
    // that stage with tile kt - 1 + NST, then the MFMAs of the tile's 32-deep sub-steps with the A
    // fragments streamed four row blocks ahead (a ring of five) and two sub-steps' B fragments, so
    // few fragments are live next to the accumulators. (Two row blocks ahead, re-started at every
    // sub-step, left LDS latency exposed: 44.0 -> 43.2 us on fc2.)
    // Tiles issued before step kt: 0 .. NST - 1 (kt = 0), 0 .. kt - 2 + NST (kt >= 1), so at most
    // NST - 1, resp. NST - 2, tiles after tile kt may still be in flight.
    for (int kt = 0; kt < KT; ++kt) {
      wait_tiles(min(KT - 1 - kt, kt == 0 ? NST - 1 : NST - 2));
      block_barrier();
      if (kt >= 1 && kt - 1 + NST < KT) issue((kt - 1) % NST, kt - 1 + NST);
      __builtin_amdgcn_sched_barrier(0);
      const unsigned char* st = smem + (kt % NST) * STAGE;
      // A fragments streamed RD row blocks ahead through a ring of RD + 1 across the tile's
      // sub-steps, and the next sub-step's B fragments read at the start of the current one.
      constexpr int RD = 4, NB = SUBW * FMB;
      bf16x8_t b[2][FNB], a[RD + 1];
      auto rd_a = [&](int idx) __attribute__((always_inline)) {
        const int s = idx / FMB, i = idx % FMB;
        const int ch = 4 * (s * KSPLIT + kg) + (lane >> 4);
        return *reinterpret_cast<const bf16x8_t*>(st + L::swz(wm0 + i * 16 + (lane & 15), ch));
      };
      auto rd_b = [&](int s, bf16x8_t (&bb)[FNB]) __attribute__((always_inline)) {
        const int ch = 4 * (s * KSPLIT + kg) + (lane >> 4);
#pragma unroll
        for (int j = 0; j < FNB; ++j)
          bb[j] = *reinterpret_cast<const bf16x8_t*>(st + L::swz(BM + wn0 + j * 16 + (lane & 15), ch));
      };
      rd_b(0, b[0]);
#pragma unroll
      for (int x = 0; x < RD && x < NB; ++x) a[x] = rd_a(x);
#pragma unroll
      for (int s = 0; s < SUBW; ++s) {
        if (s + 1 < SUBW) rd_b(s + 1, b[(s + 1) & 1]);
#pragma unroll
        for (int i = 0; i < FMB; ++i) {
          const int x = s * FMB + i;
          if (x + RD < NB) a[(x + RD) % (RD + 1)] = rd_a(x + RD);
#pragma unroll
          for (int j = 0; j < FNB; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(b[s & 1][j], a[x % (RD + 1)], acc[i][j], 0, 0, 0);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  r16_epilogue<BM, BN, WGM, WGN, KSPLIT, FMB, FNB, EPI>(acc, smem, kLutOff, kg, wr, wm, wn0, lane, m0, n0, M, ea, C,
                                                      ldc);
}

// ------------------------------------------------------------------------------------------------
// Ping-pong kernel: BM x BN tiles, 8 waves in two groups of 4, group g owning rows
// [g BM / 2, (g + 1) BM / 2) and waves w, w + 4 sharing SIMD w % 4 (wave tile BM / 2 x BN / 4).
// Between workgroup barriers each group runs one of two kinds of phase, and the groups alternate:
//   * compute phase: only the MFMAs of one 32-deep K step, on fragments already in registers;
//   * memory phase: the LDS fragment reads of the wave's next K step, and the group's share of the
//     direct-to-LDS loads of a later K tile.
//   group 0: mem(0)  comp(0)  mem(1)   comp(1)  ...  mem(S-1)  comp(S-1)  -
//   group 1: -       mem(0)   comp(0)  mem(1)   ...  comp(S-2) mem(S-1)   comp(S-1)
// While one wave of a SIMD issues MFMAs back to back, the other's LDS reads are in flight. (The
// 8-wave kernel above runs both waves of a SIMD in the same order: the older one takes the MFMA
// issue slots first and then waits a third of the K loop at the barrier for the younger one, which
// meanwhile runs alone with its LDS latencies exposed. Measured same-process on MI355X, this
// schedule is 2-3 % faster on the 288-row tiles; a one-barrier-per-step variant, each group reading
// and computing in opposite order within the interval, was not faster.)
// Loads: two 64-deep stages (a K tile is two steps); a load instruction moves 1 KB and the CU's
// vector memory path takes ~16 clocks for it, so a tile's loads (~1100 clocks at 288 x 256) are
// split between the groups, each issuing its half in its first memory phase of the previous tile
// (the stage it reuses was last read in the interval before): group g loads half g of the W rows,
// W first (both groups read them from group 0's next memory phase on), then its own A rows. Group
// 0 waits for all of its loads of tile u + 1 at the end of compute(2u + 1); group 1 for its W rows
// at the end of mem(2u + 1) and for its A rows at the end of compute(2u + 1).
// ------------------------------------------------------------------------------------------------
template <int BM, int BN, int EPI, bool F8 = false>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void gemm_bf16_pp_kernel(const uint16_t* __restrict__ A16, int M, int K, int64_t lda, const uint16_t* __restrict__ W16,
                         int N, int64_t ldw, EpiArgs ea, uint16_t* __restrict__ C, int64_t ldc, int group_m) {
  // F8: the operands are OCP e4m3 codes (one byte per element, A16 / W16 point at bytes, lda / ldw and
  // K count elements) on v_mfma_f32_16x16x128_f8f6f4; the LDS stages hold the same 128-byte rows, so
  // a K tile is 128 elements deep instead of 64.
  constexpr int EB = F8 ? 1 : 2;                   // bytes per operand element
  constexpr int BK = 64, NST = 2, WGM = 2, WGN = 4;
  constexpr int BKE = 2 * BK / EB;                 // K elements per 128-byte LDS row
  using L = R16Layout<BK>;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int FMB = WM / 16, FNB = WN / 16;
  constexpr int RPL = L::kRowsPerLoad;
  constexpr int NIA = BM / RPL, NIW = BN / RPL;  // load instructions per K tile
  constexpr int STAGE = (BM + BN) * L::kRowBytes;
  static_assert(BM % (2 * RPL) == 0 && BN % (2 * RPL) == 0, "rows must split into whole load halves");
  static_assert(WM % 16 == 0 && WN % 16 == 0, "tile shape");

  extern __shared__ __align__(16) unsigned char smem[];
  const int tiles = ea.work_tiles > 0 ? ea.work_tiles : (int)gridDim.x;
  if ((int)blockIdx.x >= tiles) {  // a warming workgroup
    warm_lines(ea.warm, ea.warm_lines, (int)blockIdx.x - tiles, (int)gridDim.x - tiles);
    return;
  }
  constexpr int kLutOff = r16_lut_offset(BM, BN, WGM, WGN, 1, BK, NST);
  const unsigned char* A = reinterpret_cast<const unsigned char*>(A16);
  const unsigned char* W = reinterpret_cast<const unsigned char*>(W16);
  if constexpr (EPI == kEpiPartial) {  // K slice blockIdx.y of length K (lda, ldw stay the full strides)
    A += (int64_t)blockIdx.y * K * EB;
    W += (int64_t)blockIdx.y * K * EB;
  }
  // The GELU table (10 KB) is only needed by the epilogue: its loads are issued here, ahead of the
  // first K tiles (so they retire first and no wait holds the tiles back), and the registers are
  // written to LDS after the K loop.
  constexpr int kLutChunks = kGeluLut / 8;  // 16-byte pieces
  static_assert(kLutChunks <= 2 * 512, "two pieces per thread");
  uint4 lut_lo = make_uint4(0u, 0u, 0u, 0u), lut_hi = lut_lo;
  if constexpr (EPI == OUDJAT_EPI_BIAS_GELU) {
    const uint4* src = reinterpret_cast<const uint4*>(g_gelu_lut);
    lut_lo = src[threadIdx.x];
    if (threadIdx.x + 512 < kLutChunks) lut_hi = src[threadIdx.x + 512];
  }

  const int tiles_n = (N + BN - 1) / BN;
  const int tiles_m = (M + BM - 1) / BM;
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
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = wave >> 2;  // group = wave row
  const int lw = wave & 3;  // wave within its group = wave column
  const int wm0 = g * WM;
  const int wn0 = lw * WN;

  // Loads: a range of the stage's load instructions [ib, ib + CNT) is spread over the group's 4
  // waves, instruction ib + lw + 4 j to wave lw; instruction i fills stage rows [i RPL, (i + 1) RPL)
  // (A rows first, then W rows). Each lane keeps one 32-bit byte offset for its first instruction
  // (its row plus its swizzled chunk); instruction j adds j * 4 * RPL rows. The range starts are
  // even, so a lane's chunk swizzle is the same for all of its instructions. Rows at or past M / N
  // fall outside the buffer descriptors and load as zeros.
  const i32x4_t rsrc_a = make_buffer_rsrc(A, (uint32_t)((int64_t)M * lda * EB));
  const i32x4_t rsrc_w = make_buffer_rsrc(W, (uint32_t)((int64_t)N * ldw * EB));
  const uint32_t step_a = (uint32_t)(4 * RPL) * (uint32_t)lda * (uint32_t)EB;
  const uint32_t step_w = (uint32_t)(4 * RPL) * (uint32_t)ldw * (uint32_t)EB;
  auto lane_offset = [&](int ib, bool w_rows) __attribute__((always_inline)) {
    const int lrow = lane / L::kChunks, lslot = lane % L::kChunks;
    const int row0 = (ib + lw) * RPL + lrow;
    const int chunk = lslot ^ ((row0 / L::kRowsPerLine) % L::kChunks);
    return w_rows ? (uint32_t)((n0 + row0 - BM) * (uint32_t)ldw * (uint32_t)EB + chunk * 16)
                  : (uint32_t)((m0 + row0) * (uint32_t)lda * (uint32_t)EB + chunk * 16);
  };
  const int ib_w = NIA + g * (NIW / 2), ib_a = g * (NIA / 2);
  const uint32_t vw = lane_offset(ib_w, true), va = lane_offset(ib_a, false);
  auto issue_w = [&](int kt) __attribute__((always_inline)) {
    unsigned char* base = smem + (kt % NST) * STAGE;
    const uint32_t koff = (uint32_t)(kt * 2 * BK);
    constexpr int CW = NIW / 2;
#pragma unroll
    for (int j = 0; j < (CW + 3) / 4; ++j)
      if (j < CW / 4 || lw < CW % 4)
        buffer_load_lds16(rsrc_w, base + (ib_w + lw + 4 * j) * 1024, vw + (uint32_t)j * step_w + koff);
  };
  auto issue_a = [&](int kt) __attribute__((always_inline)) {
    unsigned char* base = smem + (kt % NST) * STAGE;
    const uint32_t koff = (uint32_t)(kt * 2 * BK);
    constexpr int CA = NIA / 2;
#pragma unroll
    for (int j = 0; j < (CA + 3) / 4; ++j)
      if (j < CA / 4 || lw < CA % 4)
        buffer_load_lds16(rsrc_a, base + (ib_a + lw + 4 * j) * 1024, va + (uint32_t)j * step_a + koff);
  };
  auto issue_tile = [&](int kt) __attribute__((always_inline)) {
    issue_w(kt);
    issue_a(kt);
  };
  constexpr int QMAX = (NIW / 2 + 3) / 4 + (NIA / 2 + 3) / 4;  // loads per wave and tile, at most
  static_assert(QMAX < 32, "vmcnt range");
  const int n_tile = (NIW / 2) / 4 + (lw < (NIW / 2) % 4 ? 1 : 0) + (NIA / 2) / 4 + (lw < (NIA / 2) % 4 ? 1 : 0);

  f32x4_t acc[FMB][FNB];
#pragma unroll
  for (int i = 0; i < FMB; ++i)
#pragma unroll
    for (int j = 0; j < FNB; ++j) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  // bf16 -- fragments of one 32-deep step (16x16x32): lane l reads row l % 16 of a 16-row block at K
  // chunk 4 * (j % 2) + l / 16 of tile j / 2's stage.
  // F8 -- one v_mfma_f32_16x16x128_f8f6f4 covers a whole 128-deep tile: lane l feeds 32 bytes of row
  // l % 16, chunks 2 (l / 16) and 2 (l / 16) + 1, from both operands alike (an MFMA pairs the same lane
  // group and byte slot of its two sources, so a consistent assignment is all the product needs). The
  // tile's two steps split the row blocks instead of K: step 2u reads the W fragments (kept for both
  // steps) and row blocks [0, FH), step 2u + 1 the row blocks [FH, FMB), which keeps the fragment
  // registers near the bf16 kernel's; the step parity is a compile-time constant of the F8 loop.
  typedef int i32x8_t __attribute__((ext_vector_type(8)));
  constexpr int FH = (FMB + 1) / 2;
  bf16x8_t fa[F8 ? 1 : FMB], fb[F8 ? 1 : FNB];
  i32x8_t fa8[F8 ? FH : 1], fb8[F8 ? FNB : 1];
  const int KT = K / BKE;
  const int S = 2 * KT;
  auto read_frags = [&](int j) __attribute__((always_inline)) {
    const unsigned char* st = smem + ((j >> 1) % NST) * STAGE;
    const int ch = 4 * (j & 1) + (lane >> 4);
#pragma unroll
    for (int i = 0; i < FMB; ++i)
      fa[i] = *reinterpret_cast<const bf16x8_t*>(st + L::swz(wm0 + i * 16 + (lane & 15), ch));
#pragma unroll
    for (int jj = 0; jj < FNB; ++jj)
      fb[jj] = *reinterpret_cast<const bf16x8_t*>(st + L::swz(BM + wn0 + jj * 16 + (lane & 15), ch));
  };
  // Row blocks at or past M compute on zero rows and are never stored (see gemm_bf16_r16_kernel).
  auto mfmas = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < FMB; ++i)
#pragma unroll
      for (int jj = 0; jj < FNB; ++jj)
        acc[i][jj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[jj], fa[i], acc[i][jj], 0, 0, 0);
  };
  auto rd32 = [&](const unsigned char* st, int r) __attribute__((always_inline)) {
    const int c0 = 2 * (lane >> 4);
    const uint4 lo = *reinterpret_cast<const uint4*>(st + L::swz(r, c0));
    const uint4 hi = *reinterpret_cast<const uint4*>(st + L::swz(r, c0 + 1));
    return i32x8_t{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
  };
  auto read_frags8 = [&](int j, auto odd_c) __attribute__((always_inline)) {
    const unsigned char* st = smem + ((j >> 1) % NST) * STAGE;
    if constexpr (!decltype(odd_c)::value) {
#pragma unroll
      for (int jj = 0; jj < FNB; ++jj) fb8[jj] = rd32(st, BM + wn0 + jj * 16 + (lane & 15));
#pragma unroll
      for (int i = 0; i < FH; ++i) fa8[i] = rd32(st, wm0 + i * 16 + (lane & 15));
    } else {
#pragma unroll
      for (int i = 0; i < FMB - FH; ++i) fa8[i] = rd32(st, wm0 + (FH + i) * 16 + (lane & 15));
    }
  };
  auto mfmas8 = [&](auto odd_c) __attribute__((always_inline)) {
    constexpr int I0 = decltype(odd_c)::value ? FH : 0;
    constexpr int NI8 = decltype(odd_c)::value ? FMB - FH : FH;
#pragma unroll
    for (int i = 0; i < NI8; ++i)
#pragma unroll
      for (int jj = 0; jj < FNB; ++jj)
        acc[I0 + i][jj] =
            __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(fb8[jj], fa8[i], acc[I0 + i][jj], 0, 0, 0, 0, 0, 0);
  };
  // n_arows: this wave's A-row loads of a tile (issued after its W rows).
  const int n_arows = (NIA / 2) / 4 + (lw < (NIA / 2) % 4 ? 1 : 0);
  auto wait_n = [&](int n) __attribute__((always_inline)) {
    switch (n) {
#define OUDJAT_PP_WAIT(v) case v: wait_vmcnt<v>(); break;
      OUDJAT_PP_WAIT(1) OUDJAT_PP_WAIT(2) OUDJAT_PP_WAIT(3) OUDJAT_PP_WAIT(4) OUDJAT_PP_WAIT(5) OUDJAT_PP_WAIT(6)
      OUDJAT_PP_WAIT(7) OUDJAT_PP_WAIT(8) OUDJAT_PP_WAIT(9) OUDJAT_PP_WAIT(10) OUDJAT_PP_WAIT(11)
      OUDJAT_PP_WAIT(12) OUDJAT_PP_WAIT(13) OUDJAT_PP_WAIT(14) OUDJAT_PP_WAIT(15)
#undef OUDJAT_PP_WAIT
      default: wait_vmcnt<0>(); break;
    }
  };
  // Memory phase of step j (tile u = j / 2): fragments, then (u >= 1) the group's share of tile
  // u + 1's loads, its W rows at the tile's first step and its A rows at the second (so that every
  // memory phase issues about the same number of loads: with all of them at the first step, those
  // phases outlasted the other group's MFMAs), then (group 1, the tile's last step) a wait for its
  // W rows of tile u + 1, which group 0 reads after the next barrier.
  auto mem_phase = [&](int j) __attribute__((always_inline)) {
    read_frags(j);
    const int u = j >> 1;
    if (u >= 1 && u + 1 < KT) {
      if ((j & 1) == 0) issue_w(u + 1);
      else issue_a(u + 1);
    }
    if (g == 1 && (j & 1) == 1 && u + 1 < KT) wait_n(n_arows);
  };
  auto compute_phase = [&](int j) __attribute__((always_inline)) {
    mfmas();
    if ((j & 1) == 1 && (j >> 1) + 1 < KT) wait_vmcnt<0>();  // group 0: all of tile u + 1; group 1: its A rows
  };
  // The F8 steps: the same phases and loads, the parity fixed at compile time.
  auto step8 = [&](int j, auto odd_c) __attribute__((always_inline)) {
    constexpr bool ODD = decltype(odd_c)::value;
    read_frags8(j, odd_c);
    const int u = j >> 1;
    if (u >= 1 && u + 1 < KT) {
      if constexpr (!ODD) issue_w(u + 1);
      else issue_a(u + 1);
    }
    if constexpr (ODD) {
      if (g == 1 && u + 1 < KT) wait_n(n_arows);
    }
    block_barrier();
    mfmas8(odd_c);
    if constexpr (ODD) {
      if (u + 1 < KT) wait_vmcnt<0>();
    }
    block_barrier();
  };

  issue_tile(0);
  if (KT > 1) {
    issue_tile(1);
    wait_n(n_tile);  // tile 0 landed, tile 1 may be in flight
  } else {
    wait_vmcnt<0>();
  }
  block_barrier();
  if constexpr (F8) {
    using Even = std::false_type;
    using Odd = std::true_type;
    if (g == 1) block_barrier();
    for (int j = 0; j < S; j += 2) {
      step8(j, Even{});
      step8(j + 1, Odd{});
    }
    if (g == 0) block_barrier();
  } else if (g == 0) {
    for (int j = 0; j < S; ++j) {
      mem_phase(j);
      block_barrier();
      compute_phase(j);
      block_barrier();
    }
    block_barrier();
  } else {
    block_barrier();
    for (int j = 0; j < S; ++j) {
      mem_phase(j);
      block_barrier();
      compute_phase(j);
      block_barrier();
    }
  }

  if constexpr (EPI == OUDJAT_EPI_BIAS_GELU) {  // visible after the epilogue's first barrier
    uint4* dst = reinterpret_cast<uint4*>(smem + kLutOff);
    dst[threadIdx.x] = lut_lo;
    if (threadIdx.x + 512 < kLutChunks) dst[threadIdx.x + 512] = lut_hi;
  }
  r16_epilogue<BM, BN, WGM, WGN, 1, FMB, FNB, EPI, kLutOff>(acc, smem, kLutOff, 0, wave, g, wn0, lane, m0, n0, M, ea, C,
                                                           ldc);
}

// Split-K second half: C[m, n] = epilogue(P[0, m, n] + P[1, m, n] + ... + P[S-1, m, n]), the slices
// summed in order (fp32), the epilogue as the tile kernels apply it (epilogue<EPI>'s arithmetic). One
// thread per 8 columns; the per-column bias / gamma and the residual or gate row segment are read as
// vectors (the split path runs only with the aligned epilogue operands of `aligned_io`), and every
// load of a thread is issued before its first add.
template <int EPI>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ P, int S, int M, int N,
                                                            EpiArgs ea, uint16_t* __restrict__ C, int64_t ldc) {
  const int64_t per_row = N >> 3;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (int64_t)M * per_row) return;
  const int64_t row = gid / per_row;
  const int64_t col = (gid - row * per_row) * 8;
  const int64_t slice = (int64_t)M * N;
  const float* p = P + row * N + col;
  float bias[8], side[8], g[8];
  if (ea.bias) {
    const uint2 b0 = *reinterpret_cast<const uint2*>(ea.bias + col);
    const uint2 b1 = *reinterpret_cast<const uint2*>(ea.bias + col + 4);
    bias[0] = lo_bf16(b0.x); bias[1] = hi_bf16(b0.x); bias[2] = lo_bf16(b0.y); bias[3] = hi_bf16(b0.y);
    bias[4] = lo_bf16(b1.x); bias[5] = hi_bf16(b1.x); bias[6] = lo_bf16(b1.y); bias[7] = hi_bf16(b1.y);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) bias[e] = -0.0f;  // fma(a, s, -0) = a * s, the sign of a zero kept
  }
  if constexpr (EPI == OUDJAT_EPI_BIAS_LS || EPI == OUDJAT_EPI_BIAS_LS_RESID)
    unpack8(*reinterpret_cast<const uint4*>(ea.gamma + col), g);
  if constexpr (EPI == OUDJAT_EPI_BIAS_LS_RESID || EPI == OUDJAT_EPI_BIAS_SILU_MUL)
    unpack8(*reinterpret_cast<const uint4*>(ea.resid + row * ea.ldr + col), side);
  float4 a0 = *reinterpret_cast<const float4*>(p), a1 = *reinterpret_cast<const float4*>(p + 4);
  if (S == 2) {
    const float4 b0 = *reinterpret_cast<const float4*>(p + slice);
    const float4 b1 = *reinterpret_cast<const float4*>(p + slice + 4);
    a0.x += b0.x; a0.y += b0.y; a0.z += b0.z; a0.w += b0.w;
    a1.x += b1.x; a1.y += b1.y; a1.z += b1.z; a1.w += b1.w;
  } else {
    for (int sl = 1; sl < S; ++sl) {
      const float4 b0 = *reinterpret_cast<const float4*>(p + sl * slice);
      const float4 b1 = *reinterpret_cast<const float4*>(p + sl * slice + 4);
      a0.x += b0.x; a0.y += b0.y; a0.z += b0.z; a0.w += b0.w;
      a1.x += b1.x; a1.y += b1.y; a1.z += b1.z; a1.w += b1.w;
    }
  }
  const float acc[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float x = round_bf16(__builtin_fmaf(acc[e], ea.acc_scale, bias[e]));
    if (ea.raw_round)
      x = round_bf16(ea.raw_bias ? __builtin_fmaf(x, ea.raw_scale, bf16_to_f32(ea.raw_bias[col + e])) : x * ea.raw_scale);
    if constexpr (EPI == OUDJAT_EPI_BIAS_GELU) x = __uint_as_float(gelu_bf16_bits(__float_as_uint(x) >> 16, g_gelu_lut) << 16);
    else if constexpr (EPI == OUDJAT_EPI_BIAS_LS_RESID) x = fmaf(x, g[e], side[e]);
    else if constexpr (EPI == OUDJAT_EPI_BIAS_LS) x = x * g[e];
    else if constexpr (EPI == OUDJAT_EPI_BIAS_SILU_MUL) x = round_bf16(x / (1.0f + expf(-x))) * side[e];
    v[e] = x;
  }
  *reinterpret_cast<uint4*>(C + row * ldc + col) = pack8(v);
}

// ------------------------------------------------------------------------------------------------
// Configurations and dispatch
// ------------------------------------------------------------------------------------------------

typedef void (*gemm_fn)(const uint16_t*, int, int, int64_t, const uint16_t*, int, int64_t, EpiArgs, uint16_t*,
                        int64_t, int);

struct GemmCfg {
  int bm, bn, wgm, wgn, pf;  // pf: register prefetch depth; 0 = direct-to-LDS; -1 = pipelined; -2 = 16-row
  gemm_fn fn[kNumEpi];       // by epilogue; fn[kEpiQkv] only for the direct-to-LDS families, fn[kEpiPartial]
                             // only for the 16-row-block family
  int bk, nst, ks;           // 16-row kernel: K tile depth, LDS stages, K groups
  int fb;                    // 16-row kernel: fragments read one K tile ahead
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
    gemm_bf16_dma_kernel<BM, BN, WGM, WGN, 4>, gemm_bf16_dma_kernel<BM, BN, WGM, WGN, kEpiQkv>}}

#define OUDJAT_GEMM_PIPE_CFG(BM, BN, WGM, WGN)                                                            \
  {BM, BN, WGM, WGN, -1,                                                                                 \
   {gemm_bf16_pipe_kernel<BM, BN, WGM, WGN, 0>, gemm_bf16_pipe_kernel<BM, BN, WGM, WGN, 1>,               \
    gemm_bf16_pipe_kernel<BM, BN, WGM, WGN, 2>, gemm_bf16_pipe_kernel<BM, BN, WGM, WGN, 3>,               \
    gemm_bf16_pipe_kernel<BM, BN, WGM, WGN, 4>, gemm_bf16_pipe_kernel<BM, BN, WGM, WGN, kEpiQkv>}}

// pf = -2: 16-row-block kernel; wgm x wgn waves per K group, ks K groups.
#define OUDJAT_GEMM_R16_CFG(BM, BN, WGM, WGN, KS, BK, NST, FB)                                            \
  {BM, BN, WGM, WGN, -2,                                                                                 \
   {gemm_bf16_r16_kernel<BM, BN, WGM, WGN, KS, BK, NST, FB, 0>,                                          \
    gemm_bf16_r16_kernel<BM, BN, WGM, WGN, KS, BK, NST, FB, 1>,                                          \
    gemm_bf16_r16_kernel<BM, BN, WGM, WGN, KS, BK, NST, FB, 2>,                                          \
    gemm_bf16_r16_kernel<BM, BN, WGM, WGN, KS, BK, NST, FB, 3>,                                          \
    gemm_bf16_r16_kernel<BM, BN, WGM, WGN, KS, BK, NST, FB, 4>,                                          \
    gemm_bf16_r16_kernel<BM, BN, WGM, WGN, KS, BK, NST, FB, kEpiQkv>,                                    \
    gemm_bf16_r16_kernel<BM, BN, WGM, WGN, KS, BK, NST, FB, kEpiPartial>},                               \
   BK, NST, KS, FB}

// pf = -3: ping-pong kernel (8 waves: a 2 x 4 wave grid, 64-deep K tiles in two stages).
#define OUDJAT_GEMM_PP_CFG(BM, BN)                                                                        \
  {BM, BN, 2, 4, -3,                                                                                     \
   {gemm_bf16_pp_kernel<BM, BN, 0>, gemm_bf16_pp_kernel<BM, BN, 1>, gemm_bf16_pp_kernel<BM, BN, 2>,      \
    gemm_bf16_pp_kernel<BM, BN, 3>, gemm_bf16_pp_kernel<BM, BN, 4>, gemm_bf16_pp_kernel<BM, BN, kEpiQkv>,  \
    gemm_bf16_pp_kernel<BM, BN, kEpiPartial>, gemm_bf16_pp_kernel<BM, BN, kEpiSwigluXh>},                 \
   64, 2, 1, 0}

// pf = -4: the ping-pong kernel on e4m3 operands (oudjat_linear_fp8; no GELU epilogue -- the FP8 route
// serves the SwiGLU blocks' linears -- and no split K).
#define OUDJAT_GEMM_PP8_CFG(BM, BN)                                                                       \
  {BM, BN, 2, 4, -4,                                                                                     \
   {gemm_bf16_pp_kernel<BM, BN, 0, true>, nullptr, gemm_bf16_pp_kernel<BM, BN, 2, true>,                  \
    gemm_bf16_pp_kernel<BM, BN, 3, true>, gemm_bf16_pp_kernel<BM, BN, 4, true>,                           \
    gemm_bf16_pp_kernel<BM, BN, kEpiQkv, true>, nullptr},                                                 \
   64, 2, 1, 0}

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
    OUDJAT_GEMM_PIPE_CFG(256, 256, 2, 4),  // 15
    OUDJAT_GEMM_PIPE_CFG(256, 256, 2, 2),  // 16
    OUDJAT_GEMM_PIPE_CFG(288, 256, 3, 4),  // 17
    OUDJAT_GEMM_PIPE_CFG(256, 128, 2, 2),  // 18
    OUDJAT_GEMM_PIPE_CFG(128, 128, 2, 2),  // 19
    OUDJAT_GEMM_R16_CFG(144, 512, 1, 4, 1, 32, 3, true),   // 20
    OUDJAT_GEMM_R16_CFG(144, 128, 1, 2, 2, 64, 4, true),   // 21
    OUDJAT_GEMM_R16_CFG(144, 512, 1, 8, 1, 32, 3, false),  // 22: fc1-like (N % 512 == 0)
    OUDJAT_GEMM_R16_CFG(144, 128, 1, 4, 2, 64, 4, true),   // 23: N = C GEMMs
    OUDJAT_GEMM_R16_CFG(144, 128, 1, 4, 2, 64, 3, true),   // 24
    OUDJAT_GEMM_R16_CFG(288, 256, 2, 4, 1, 64, 2, false),  // 25: 288 x 256, 128-byte operand rows
    OUDJAT_GEMM_R16_CFG(288, 192, 2, 4, 1, 64, 2, false),  // 26: 288 x 192 (N = 3 C: 240 tiles)
    OUDJAT_GEMM_PP_CFG(288, 256),  // 27: ping-pong 288 x 256
    OUDJAT_GEMM_PP_CFG(288, 192),  // 28: ping-pong 288 x 192
    OUDJAT_GEMM_R16_CFG(144, 128, 1, 4, 2, 128, 2, false),  // 29: N = C GEMMs with K % 128 == 0
    OUDJAT_GEMM_PP_CFG(224, 256),  // 30: ping-pong 224 x 256 (a full round where 288 rows leave CUs idle)
    OUDJAT_GEMM_PP_CFG(192, 256),  // 31: ping-pong 192 x 256 (two rounds or a little less)
    OUDJAT_GEMM_DMA_CFG(128, 32, 4, 1),  // 32: tiny grids (128 x 32, four waves of 32 x 32)
    OUDJAT_GEMM_DMA_CFG(128, 64, 2, 2),  // 33: tiny fused-QKV grids (whole 64-wide heads)
    OUDJAT_GEMM_R16_CFG(128, 256, 2, 4, 1, 64, 3, false),  // 34: long-K products of ~one round of 128 x 256
    OUDJAT_GEMM_PP8_CFG(288, 256),  // 35: FP8 ping-pong tiles
    OUDJAT_GEMM_PP8_CFG(224, 256),  // 36
    OUDJAT_GEMM_PP8_CFG(192, 256),  // 37
    OUDJAT_GEMM_PP8_CFG(128, 256),  // 38
    OUDJAT_GEMM_PP_CFG(224, 384),  // 39: ping-pong 224 x 384 (one round where 256-wide tiles need two)
};
static constexpr int kNumCfgs = sizeof(kCfgs) / sizeof(kCfgs[0]);

// Host side of the GELU table: entry s * kGeluSpan + d holds bf16(gelu(v)) for the bf16 input v
// with sign s and magnitude bits kGeluLo + d, computed as 0.5 v erfc(-v / sqrt 2) in double,
// rounded to fp32 and then to bf16 (nearest even). Copied to each device once, before the first
// GELU launch on it.
static uint16_t host_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static int ensure_gelu_table() {
  static std::once_flag flags[64];
  static int status[64];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(OUDJAT_ERR_HIP, "linear_bf16: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= 64) return set_error(OUDJAT_ERR_HIP, "linear_bf16: device index %d out of range", dev);
  std::call_once(flags[dev], [&] {
    static uint16_t table[kGeluLut];
    for (uint32_t sgn = 0; sgn < 2; ++sgn)
      for (uint32_t d = 0; d < kGeluSpan; ++d) {
        const uint32_t bits = ((sgn << 15) | (kGeluLo + d)) << 16;
        float v;
        memcpy(&v, &bits, 4);
        const double g = 0.5 * (double)v * erfc(-(double)v / sqrt(2.0));
        table[sgn * kGeluSpan + d] = host_f32_to_bf16((float)g);
      }
    hipError_t ce = hipMemcpyToSymbol(HIP_SYMBOL(g_gelu_lut), table, sizeof(table), 0, hipMemcpyHostToDevice);
    status[dev] = ce == hipSuccess ? OUDJAT_OK
                                   : set_error(OUDJAT_ERR_HIP, "linear_bf16: GELU table upload: %s", hipGetErrorString(ce));
  });
  return status[dev];
}

// Rows of output tiles each XCD sweeps before moving to the next tile column (L2 reuse of the W panel).
constexpr int kGroupM = 8;

// A grid of at most 32 tiles of 128 x 128 (ViT-S at B = 1: 103 selected rows) leaves most CUs idle
// and each workgroup streams its whole K alone: 128 x 32 tiles give four times the workgroups at 5/8
// of the operand bytes each. Measured in the ViT-S pass (kernel trace, 128 x 128 -> 128 x 32): proj
// 384 x 384 10.5 -> 7.4 us, fc1 1536 x 384 10.0 -> 7.1 us. Long-K tiny products still split K when
// given a workspace (choose_splitk: ViT-S fc2, K = 1536, 13.4 us in 12 slices against 15.0 us for
// unsplit 128 x 32 tiles, whose weights then stream from HBM).
static bool tiny_grid(int64_t M, int64_t N) { return N % 32 == 0 && cdiv(M, 128) * cdiv(N, 128) <= 32; }

// aligned_io: C, resid 16-byte aligned with ldc, ldr % 8 == 0 and bias 8-byte aligned, which the
// vector epilogues need; otherwise the register-staged kernel with 2-byte stores runs.
static int choose_cfg(int64_t M, int64_t N, int64_t K, bool aligned_io) {
  if (!aligned_io) return 8;
  if (tiny_grid(M, N)) return 32;
  // 256 x 256 pipelined tiles when their grid fills between half and all of the CUs in one round;
  // 128 x 128 direct-to-LDS tiles otherwise (two workgroups per CU balance a ragged second round
  // better); the register-staged kernel for N % 128 != 0.
  if (N % 128 != 0) return 8;
  // 288 x 256 / 288 x 192 (ping-pong) tiles with 128-byte operand rows when they fill three quarters
  // or more of the CUs in one round: ahead of the 256 x 256 pipelined tiles, which they beat at every
  // such shape measured (ViT-7B w1 1656 x 8192 x 4096: 94 against 111 us; a plain 4176 x 3072 x 1024
  // product: 28.5 against 33.3 us).
  const int64_t tiles288 = cdiv(M, 288) * (N / 256);
  // 224 x 256 ping-pong tiles when they fill at least seven eighths of one round that 288 x 256 tiles
  // fill less (ViT-7B w1 / w2, 1656 x 8192 x 4096: 256 against 192 tiles, 92.7 against 103.4 us).
  const int64_t tiles224 = cdiv(M, 224) * (N / 256);
  // Beyond two rounds of 288 x 256 tiles (the approximate pass, every token of the batch: M = B N)
  // those tiles in as many rounds as it takes, in place of 128 x 128 tiles (ViT-L approximate pass
  // 18.1 -> 16.5 ms, ViT-7B 337.7 -> 256.5 ms; 224 x 256 and 192 x 256 tiles came between).
  if (N % 256 == 0 && tiles288 > 512) return 27;
  if (N % 256 == 0 && tiles224 >= 224 && tiles224 <= 256 && tiles288 < tiles224) return 30;
  if (N % 256 == 0 && tiles288 >= 192 && tiles288 <= 256) return 27;
  // One round of 224 x 384 ping-pong tiles where the 256-wide ones need more than one (ViT-7B qkv,
  // 1656 x 12288 x 4096: 256 tiles, 135.1 us, against 170.4 for 432 tiles of 192 x 256 in two uneven
  // rounds and 147.2 for hipBLASLt; 22 % fewer operand bytes per FLOP than 192 x 256).
  const int64_t tiles384 = cdiv(M, 224) * (N / 384);
  if (N % 384 == 0 && tiles384 >= 224 && tiles384 <= 256) return 39;
  // Two rounds of 288-, 224- or 192-row ping-pong tiles 256 wide, whichever fills them most (ViT-L
  // keep 50 %, M = 8272: fc1 4096 wide, 464 tiles of 288 x 256, 62.7 us; qkv 3072 wide, 444 tiles of
  // 224 x 256, 53.7 us, where 128 x 128 tiles took 85.0 and 73.3 us; ViT-7B qkv, 1656 x 12288 x 4096:
  // 432 tiles of 192 x 256, 162.6 us, against 177.9 for a round and a half of 288 x 192 tiles and
  // 185.4 for 128 x 128 tiles; 192 x 256 also takes whole heads of Dh = 128 for the fused QKV
  // epilogue, which 192-wide tiles do not).
  if (N % 256 == 0) {
    const int64_t tiles192 = cdiv(M, 192) * (N / 256);
    int best = -1;
    int64_t best_tiles = 0;
    const int64_t cand_tiles[3] = {tiles288, tiles224, tiles192};
    const int cand_cfg[3] = {27, 30, 31};
    for (int c = 0; c < 3; ++c)
      if (cand_tiles[c] > 256 && cand_tiles[c] <= 512 && cand_tiles[c] > best_tiles) {
        best = cand_cfg[c];
        best_tiles = cand_tiles[c];
      }
    if (best >= 0 && best_tiles > 384) return best;
  }
  const int64_t tiles288n = cdiv(M, 288) * (N / 192);
  if (N % 192 == 0 && tiles288n >= 192 && tiles288n <= 256) return 28;
  // Half a round or more of 256 x 256 tiles: 192 x 256 or 224 x 256 ping-pong tiles if they still fit
  // one round (ViT-L keep 50 %, 8272 x 1024: 176 tiles of 192 x 256, proj 28.7 us and fc2 77.8 us,
  // against 30.6 / 82.3 for 224 x 256 and 34.9 / 101.4 for the 132 pipelined 256 x 256 tiles), else
  // those.
  const int64_t tiles256 = cdiv(M, 256) * cdiv(N, 256);
  if (N % 256 == 0 && tiles256 >= 128 && tiles256 <= 256)
    return cdiv(M, 192) * (N / 256) <= 256 ? 31 : (tiles224 <= 256 ? 30 : 15);
  // 144-row tiles (one round of 128..256 workgroups) when 256 x 256 tiles do not fit one round.
  const int64_t tm144 = cdiv(M, 144);
  if (N % 512 == 0 && tm144 * (N / 512) >= 128 && tm144 * (N / 512) <= 256) return 22;
  // 128-deep K tiles (half the barriers and load batches of the 64-deep ones; the two K groups still
  // take alternate 32-deep steps, so the result is the same bit for bit) when K allows.
  if (tm144 * (N / 128) >= 128 && tm144 * (N / 128) <= 256) return K % 128 == 0 ? 29 : 23;
  // A short-K product of a quarter to a half round of 144 x 128 tiles runs best on 128 x 32 tiles,
  // four to five workgroups per CU (ViT-L keep 10 % proj, 1712 x 1024 x 1024: 16.1 -> 15.1 us; ViT-B
  // proj, 2088 x 768 x 768: 13.5 -> 12.5 us; weights from HBM, HIP graph). 128 x 128 tiles: 20.3 and
  // 16.6 us; at a full round and more (the headline proj, 4176 rows) 128 x 32 tiles lose (27.6 against
  // 17.6 us).
  if (K <= 1024 && tm144 * (N / 128) >= 64 && tm144 * (N / 128) < 128) return 32;
  // A round and a half of 288 x 192 tiles still beats 128 x 128 tiles.
  if (N % 192 == 0 && tiles288n > 256 && tiles288n <= 400) return 28;
  // A long-K product whose 128 x 256 grid fills three quarters to all of one round (ViT-7B proj,
  // 1656 x 4096 x 4096: 208 tiles): 16-row-block 128 x 256 tiles, 8 waves of 64 x 64, three 64-deep
  // stages, in place of two rounds of 128 x 128 tiles (77.6 -> 70.8 us with the weights from HBM).
  const int64_t tiles128w = cdiv(M, 128) * (N / 256);
  if (K >= 2048 && N % 256 == 0 && tiles128w >= 192 && tiles128w <= 256) return 34;
  return 11;
}


// Split K when the output tiles leave most CUs idle: S K-slices side by side (S * tiles <= 256
// workgroups, one round), each a whole number of K tiles. Candidates: the 144 x 128 16-row-block
// tiles with slices at least 1024 deep, and the 288 x 256 ping-pong tiles with slices at least 4096
// deep (measured: ViT-7B w3, 1656 x 4096 x 8192, 138 -> 128 us; with 1024- or 2048-deep slices the
// partial stores and the reduce cost more than the halved operand stream saves: ViT-L fc2 49 ->
// 68 us, ViT-7B proj 78 -> 90 us). Among those whose split fills at least 160 CUs, the one that
// streams the fewest operand bytes per workgroup. Returns the configuration and S (-1 / S = 1: no
// split). Every public epilogue: their tile forms are epilogue<EPI> element by element.
static int choose_splitk(int64_t M, int64_t N, int64_t K, int epi, int* S_out) {
  *S_out = 1;
  if (N % 128 != 0 || epi >= kEpiQkv) return -1;
  struct Cand { int ci, bm, bn, bk, min_slice; };
  const Cand cands[] = {{29, 144, 128, 128, 1024}, {23, 144, 128, 64, 1024}, {27, 288, 256, 64, 4096}};
  int best = -1, best_s = 1;
  int64_t best_bytes = 0;
  for (const Cand& c : cands) {
    if (N % c.bn != 0) continue;
    const int64_t tiles = cdiv(M, c.bm) * (N / c.bn);
    if (tiles >= 128) continue;  // fills the GPU without a split
    // A product of a few dozen 144 x 128 tiles at most with a long K loop (ViT-S at B = 1, fc2: 103
    // rows, 3 tiles, K = 1536) splits deep, down to two K tiles per slice, on those tiles: its partial
    // tiles are a few megabytes at most, while unsplit each workgroup would stream all of K alone on
    // an idle GPU (16.2 against 23.5 us in 12 slices). With K < 1024 the second launch costs more
    // than the split saves (ViT-S proj and fc1, K = 384: 13.7 -> 15.2 and 12.5 -> 14.5 us in 3).
    const bool tiny = c.bm == 144 && tiles <= 32 && K >= 1024;
    const int s_max = tiny ? 16 : 4;
    const int64_t min_slice = tiny ? 2 * c.bk : c.min_slice;
    const int64_t min_wgs = tiny ? 2 * tiles : 160;
    for (int S = (int)std::min<int64_t>(s_max, 256 / std::max<int64_t>(tiles, 1)); S >= 2; --S) {
      if (K % ((int64_t)S * c.bk) != 0 || K / S < min_slice || S * tiles < min_wgs) continue;
      const int64_t bytes = (int64_t)(c.bm + c.bn) * (K / S);
      if (best < 0 || bytes < best_bytes) {
        best = c.ci;
        best_s = S;
        best_bytes = bytes;
      }
      break;
    }
  }
  *S_out = best_s;
  return best;
}

// Fused QKV: tiles must cover whole heads (Dh | BN; a tile may span the q / k / v boundaries).
// 288 x 192 (ping-pong) tiles when the plain choice would leave more CUs idle in its single round.
static int choose_qkv_cfg(int64_t M, int64_t N, int64_t K, int64_t Dh) {
  if (tiny_grid(M, N) && 64 % Dh == 0 && N % 64 == 0) return 33;  // ViT-S at B = 1: 10.5 -> 8.2 us
  // One round of whole-head 224 x 384 tiles (ViT-7B: 179.6 -> 140.3 us per fused QKV in the pass).
  const int64_t t384 = cdiv(M, 224) * (N / 384);
  if (N % 384 == 0 && 384 % Dh == 0 && t384 >= 224 && t384 <= 256) return 39;
  int ci = choose_cfg(M, N, K, true);
  const int64_t tiles288n = cdiv(M, 288) * (N / 192);
  if (N % 192 == 0 && tiles288n >= 192 && tiles288n <= 256 &&
      cdiv(M, kCfgs[ci].bm) * cdiv(N, kCfgs[ci].bn) < tiles288n)
    ci = 28;
  if (kCfgs[ci].pf > 0 || kCfgs[ci].bn % Dh != 0 || N % kCfgs[ci].bn != 0) ci = 11;  // 128 x 128 direct-to-LDS
  return ci;
}

// FP8 products (e4m3 operands: half the operand bytes per K of bf16) on the FP8 ping-pong tiles, chosen
// as for bf16: one round of 224- or 288-row tiles; else two rounds of whichever of 288, 224 and 192 rows
// fills them most; else one round of 192-row tiles; else 128-row tiles (ViT-7B at B = 4, M = 1656: qkv
// 432 tiles of 192 x 256, proj and w3 208 of 128 x 256, w1 / w2 256 of 224 x 256). N % 256 == 0.
static int choose_cfg_fp8(int64_t M, int64_t N) {
  const int64_t t288 = cdiv(M, 288) * (N / 256), t224 = cdiv(M, 224) * (N / 256);
  const int64_t t192 = cdiv(M, 192) * (N / 256);
  if (t224 >= 224 && t224 <= 256 && t288 < t224) return 36;
  if (t288 >= 192 && t288 <= 256) return 35;
  int best = -1;
  int64_t best_tiles = 0;
  const int64_t cand_tiles[3] = {t288, t224, t192};
  const int cand_cfg[3] = {35, 36, 37};
  for (int c = 0; c < 3; ++c)
    if (cand_tiles[c] > 256 && cand_tiles[c] <= 512 && cand_tiles[c] > best_tiles) {
      best = cand_cfg[c];
      best_tiles = cand_tiles[c];
    }
  if (best >= 0 && best_tiles > 384) return best;
  if (t192 >= 192 && t192 <= 256) return 37;
  return 38;
}

// Launches configuration `ci` with epilogue `epi` (arguments already validated).
// Warming workgroups a launch of configuration `cfg` with this many tiles (unsplit) carries: one per
// CU its tiles leave idle, for the 16-row and ping-pong kernels (one workgroup per CU).
static int64_t warm_slots(const GemmCfg& cfg, int64_t tiles) {
  return (cfg.pf == -2 || cfg.pf == -3) && tiles < kNumCus ? kNumCus - tiles : 0;
}

// warm / warm_bytes: a region (4-byte aligned) to read into the caches from the CUs an unsplit launch
// of fewer tiles than CUs leaves idle (one workgroup per CU: the kernels that take it hold a CU's
// registers or LDS), for the launch after the next that reads it; ignored by the other kernels.
static int launch_gemm(int ci, const uint16_t* A, int64_t M, int64_t K, int64_t lda, const uint16_t* W, int64_t N,
                       int64_t ldw, int epi, const EpiArgs& ea_in, uint16_t* C, int64_t ldc, hipStream_t stream,
                       const char* what, int splits = 1, const void* warm = nullptr, int64_t warm_bytes = 0) {
  const GemmCfg& cfg = kCfgs[ci];
  const int64_t tiles = cdiv(M, cfg.bm) * cdiv(N, cfg.bn);
  OUDJAT_REQUIRE(tiles < ((int64_t)1 << 31), OUDJAT_ERR_TOO_LARGE, "%s: too many tiles", what);
  EpiArgs ea = ea_in;
  int64_t grid = tiles;
  if (warm && warm_bytes >= 128 && splits == 1 && warm_slots(cfg, tiles) > 0) {
    ea.warm = static_cast<const uint32_t*>(warm);
    ea.warm_lines = warm_bytes / 128;
    ea.work_tiles = (int)tiles;
    grid = tiles + warm_slots(cfg, tiles);
  }
  // K stages, or (direct-to-LDS kernels) the bf16 output tile of the epilogue if that is larger.
  size_t lds = cfg.pf < 0 ? (size_t)kStages * (cfg.bm + cfg.bn) * 64 : (size_t)2 * (cfg.bm + cfg.bn) * 128;
  if (cfg.pf <= 0) lds = lds > (size_t)cfg.bm * (cfg.bn + 8) * 2 ? lds : (size_t)cfg.bm * (cfg.bn + 8) * 2;
  if (cfg.pf <= -2) lds = r16_lut_offset(cfg.bm, cfg.bn, cfg.wgm, cfg.wgn, cfg.ks, cfg.bk, cfg.nst);
  if (cfg.pf <= 0 && epi == OUDJAT_EPI_BIAS_GELU) lds += kGeluLut * sizeof(uint16_t);
  if (epi == OUDJAT_EPI_BIAS_GELU) {
    const int st = ensure_gelu_table();
    if (st != OUDJAT_OK) return st;
  }
  const gemm_fn fn = cfg.fn[epi];
  OUDJAT_REQUIRE(fn != nullptr, OUDJAT_ERR_UNSUPPORTED_SHAPE, "%s: no kernel for this epilogue", what);
  if (lds > 64 * 1024) {
    // Once per kernel and device (also keeps the call out of captured launch sequences).
    static std::atomic<uint8_t> attr_set[64][kNumCfgs][kNumEpi];
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return set_error(OUDJAT_ERR_HIP, "%s: hipGetDevice: %s", what, hipGetErrorString(e));
    std::atomic<uint8_t>& flag = attr_set[dev & 63][ci][epi];
    if (!flag.load(std::memory_order_acquire)) {
      e = hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      if (e != hipSuccess) return set_error(OUDJAT_ERR_HIP, "%s: hipFuncSetAttribute: %s", what, hipGetErrorString(e));
      flag.store(1, std::memory_order_release);
    }
  }
  const int threads = cfg.wgm * cfg.wgn * (cfg.pf <= -2 ? cfg.ks : 1) * 64;
  // A split launch (epi == kEpiPartial) runs K / splits per workgroup, slice = blockIdx.y.
  hipLaunchKernelGGL(fn, dim3((unsigned)grid, (unsigned)splits), dim3(threads), lds, stream, A, (int)M,
                     (int)(K / splits), lda, W, (int)N, ldw, ea, C, ldc, kGroupM);
  return check_launch(what);
}

// Split-K: the partial launch into the fp32 workspace [S, M, N], then the reduce + epilogue launch.
static int launch_gemm_splitk(int ci, int S, const uint16_t* A, int64_t M, int64_t K, int64_t lda, const uint16_t* W,
                              int64_t N, int64_t ldw, int epi, const EpiArgs& ea, uint16_t* C, int64_t ldc,
                              float* ws, hipStream_t stream, const char* what) {
  int st = launch_gemm(ci, A, M, K, lda, W, N, ldw, kEpiPartial, ea, reinterpret_cast<uint16_t*>(ws), N, stream,
                       what, S);
  if (st != OUDJAT_OK) return st;
  if (epi == OUDJAT_EPI_BIAS_GELU) {
    st = ensure_gelu_table();
    if (st != OUDJAT_OK) return st;
  }
  const int64_t items = M * (N / 8);
  const dim3 grid((unsigned)cdiv(items, 256));
  switch (epi) {
    case OUDJAT_EPI_BIAS:
      splitk_reduce_kernel<OUDJAT_EPI_BIAS><<<grid, 256, 0, stream>>>(ws, S, (int)M, (int)N, ea, C, ldc);
      break;
    case OUDJAT_EPI_BIAS_GELU:
      splitk_reduce_kernel<OUDJAT_EPI_BIAS_GELU><<<grid, 256, 0, stream>>>(ws, S, (int)M, (int)N, ea, C, ldc);
      break;
    case OUDJAT_EPI_BIAS_LS_RESID:
      splitk_reduce_kernel<OUDJAT_EPI_BIAS_LS_RESID><<<grid, 256, 0, stream>>>(ws, S, (int)M, (int)N, ea, C, ldc);
      break;
    case OUDJAT_EPI_BIAS_LS:
      splitk_reduce_kernel<OUDJAT_EPI_BIAS_LS><<<grid, 256, 0, stream>>>(ws, S, (int)M, (int)N, ea, C, ldc);
      break;
    case OUDJAT_EPI_BIAS_SILU_MUL:
      splitk_reduce_kernel<OUDJAT_EPI_BIAS_SILU_MUL><<<grid, 256, 0, stream>>>(ws, S, (int)M, (int)N, ea, C, ldc);
      break;
    default:
      return set_error(OUDJAT_ERR_UNSUPPORTED_SHAPE, "%s: no split-K reduce for epilogue %d", what, epi);
  }
  return check_launch(what);
}

}  // namespace oudjat

using namespace oudjat;

static int linear_bf16_impl(const uint16_t* A, int64_t M, int64_t K, int64_t lda, const uint16_t* W, int64_t N,
                            int64_t ldw, const uint16_t* bias, int epi, const uint16_t* gamma, const uint16_t* resid,
                            int64_t ldr, uint16_t* C, int64_t ldc, float acc_scale, float* workspace,
                            int64_t workspace_elems, const void* warm, int64_t warm_bytes, oudjat_stream_t stream) {
  OUDJAT_REQUIRE(M >= 0 && N >= 0 && K >= 0, OUDJAT_ERR_INVALID_ARGUMENT, "linear_bf16: negative size");
  OUDJAT_REQUIRE(warm_bytes >= 0 && (warm_bytes == 0 || warm), OUDJAT_ERR_INVALID_ARGUMENT,
                 "linear_bf16: bad warm region (bytes < 0, or NULL with bytes > 0)");
  OUDJAT_REQUIRE(warm_bytes == 0 || aligned(warm, 4), OUDJAT_ERR_UNSUPPORTED_LAYOUT,
                 "linear_bf16: the warm region must be 4-byte aligned");
  const int raw_round = (epi & OUDJAT_EPI_RAW_BF16) != 0;
  epi &= ~OUDJAT_EPI_RAW_BF16;
  OUDJAT_REQUIRE(epi >= OUDJAT_EPI_BIAS && epi <= OUDJAT_EPI_BIAS_SILU_MUL, OUDJAT_ERR_INVALID_ARGUMENT,
                 "linear_bf16: bad epilogue %d", epi);
  OUDJAT_REQUIRE(!raw_round || epi != OUDJAT_EPI_BIAS_GELU, OUDJAT_ERR_INVALID_ARGUMENT,
                 "linear_bf16: OUDJAT_EPI_RAW_BF16 does not combine with the GELU epilogue");
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
  const bool aligned_io = aligned(C, 16) && ldc % 8 == 0 && (!bias || aligned(bias, 8)) &&
                          (!gamma || aligned(gamma, 16)) && (!resid || (aligned(resid, 16) && ldr % 8 == 0));
  EpiArgs ea{};
  ea.bias = bias;
  ea.gamma = gamma;
  ea.resid = resid;
  ea.ldr = ldr;
  ea.acc_scale = acc_scale;
  if (raw_round) {  // bf16(acc) at the first rounding point, then the scale and bias
    OUDJAT_REQUIRE(!bias || aligned(bias, 16), OUDJAT_ERR_UNSUPPORTED_LAYOUT,
                   "linear_bf16: a raw-rounded epilogue needs a 16-byte aligned bias");
    ea.raw_round = 1;
    ea.raw_scale = acc_scale;
    ea.raw_bias = bias;
    ea.acc_scale = 1.0f;
    ea.bias = nullptr;
  }
  if (workspace && aligned_io && aligned(workspace, 16)) {
    int S = 1;
    const int ci = choose_splitk(M, N, K, epi, &S);
    if (ci >= 0 && S > 1 && (int64_t)S * M * N <= workspace_elems)
      return launch_gemm_splitk(ci, S, A, M, K, lda, W, N, ldw, epi, ea, C, ldc, workspace, as_stream(stream),
                                "linear_bf16");
  }
  return launch_gemm(choose_cfg(M, N, K, aligned_io), A, M, K, lda, W, N, ldw, epi, ea, C, ldc, as_stream(stream),
                     "linear_bf16", 1, warm, warm_bytes);
}

extern "C" int oudjat_linear_bf16(const uint16_t* A, int64_t M, int64_t K, int64_t lda, const uint16_t* W, int64_t N,
                                  int64_t ldw, const uint16_t* bias, int epi, const uint16_t* gamma,
                                  const uint16_t* resid, int64_t ldr, uint16_t* C, int64_t ldc, float acc_scale,
                                  float* workspace, int64_t workspace_elems, oudjat_stream_t stream) {
  return linear_bf16_impl(A, M, K, lda, W, N, ldw, bias, epi, gamma, resid, ldr, C, ldc, acc_scale, workspace,
                          workspace_elems, nullptr, 0, stream);
}

extern "C" int oudjat_linear_bf16_warm(const uint16_t* A, int64_t M, int64_t K, int64_t lda, const uint16_t* W,
                                       int64_t N, int64_t ldw, const uint16_t* bias, int epi, const uint16_t* gamma,
                                       const uint16_t* resid, int64_t ldr, uint16_t* C, int64_t ldc, float acc_scale,
                                       float* workspace, int64_t workspace_elems, const void* warm,
                                       int64_t warm_bytes, oudjat_stream_t stream) {
  return linear_bf16_impl(A, M, K, lda, W, N, ldw, bias, epi, gamma, resid, ldr, C, ldc, acc_scale, workspace,
                          workspace_elems, warm, warm_bytes, stream);
}

extern "C" int oudjat_linear_swiglu_nvfp4(const uint16_t* A, int64_t M, int64_t K, int64_t lda, const uint16_t* W,
                                          int64_t N, int64_t ldw, const uint16_t* x1, int64_t ld1, float s1,
                                          const uint16_t* b1, float s2, const uint16_t* b2,
                                          const float* tensor_scale, uint16_t* xhat, int64_t ldc,
                                          oudjat_stream_t stream) {
  const char* what = "linear_swiglu_nvfp4";
  OUDJAT_REQUIRE(M >= 0 && N >= 0 && K >= 0, OUDJAT_ERR_INVALID_ARGUMENT, "%s: negative size", what);
  if (M == 0 || N == 0) return OUDJAT_OK;
  OUDJAT_REQUIRE(A && W && x1 && tensor_scale && xhat && (b1 == nullptr) == (b2 == nullptr),
                 OUDJAT_ERR_INVALID_ARGUMENT, "%s: null pointer (both biases or neither)", what);
  OUDJAT_REQUIRE(K > 0 && K % kBK == 0 && N % 256 == 0, OUDJAT_ERR_UNSUPPORTED_SHAPE,
                 "%s: K %% %d == 0 and N %% 256 == 0 required (K=%lld, N=%lld)", what, kBK, (long long)K,
                 (long long)N);
  OUDJAT_REQUIRE(lda % 8 == 0 && ldw % 8 == 0 && ld1 % 8 == 0 && ldc % 8 == 0 && lda >= K && ldw >= K && ld1 >= N &&
                     ldc >= N && aligned(A, 16) && aligned(W, 16) && aligned(x1, 16) && aligned(xhat, 16) &&
                     (!b1 || (aligned(b1, 16) && aligned(b2, 16))),
                 OUDJAT_ERR_UNSUPPORTED_LAYOUT, "%s: 16-byte aligned operands and rows, ld %% 8 == 0", what);
  OUDJAT_REQUIRE(M < ((int64_t)1 << 31) && N < ((int64_t)1 << 31) && K < ((int64_t)1 << 31), OUDJAT_ERR_TOO_LARGE,
                 "%s: dimensions must fit in int32", what);
  EpiArgs ea{};
  ea.acc_scale = 1.0f;  // the tile holds x2 = bf16(acc) exactly (no bias at the first rounding point)
  ea.resid = x1;
  ea.ldr = ld1;
  ea.s1 = s1;
  ea.s2 = s2;
  ea.b1 = b1;
  ea.b2 = b2;
  ea.xh_ts = tensor_scale;
  // The epilogue exists on the ping-pong tiles; shapes whose choice is another family take 192 x 256.
  int ci = choose_cfg(M, N, K, true);
  if (kCfgs[ci].fn[kEpiSwigluXh] == nullptr) ci = 31;
  return launch_gemm(ci, A, M, K, lda, W, N, ldw, kEpiSwigluXh, ea, xhat, ldc, as_stream(stream), what);
}

// The partial GEMM of a split-K product alone (see oudjat.h): the consumer reduces the slices.
extern "C" int oudjat_linear_splitk_partial(const uint16_t* A, int64_t M, int64_t K, int64_t lda, const uint16_t* W,
                                            int64_t N, int64_t ldw, float* workspace, int64_t workspace_elems,
                                            int64_t* slices, oudjat_stream_t stream) {
  OUDJAT_REQUIRE(M > 0 && N > 0 && K > 0, OUDJAT_ERR_INVALID_ARGUMENT, "linear_splitk_partial: bad size");
  OUDJAT_REQUIRE(A && W && workspace && slices, OUDJAT_ERR_INVALID_ARGUMENT, "linear_splitk_partial: null pointer");
  OUDJAT_REQUIRE(K % kBK == 0 && N % 64 == 0, OUDJAT_ERR_UNSUPPORTED_SHAPE,
                 "linear_splitk_partial: K %% %d == 0 and N %% 64 == 0 required", kBK);
  OUDJAT_REQUIRE(lda % 8 == 0 && ldw % 8 == 0 && lda >= K && ldw >= K && aligned(A, 16) && aligned(W, 16) &&
                     aligned(workspace, 16),
                 OUDJAT_ERR_UNSUPPORTED_LAYOUT, "linear_splitk_partial: operands must be 16-byte aligned, ld %% 8 == 0");
  OUDJAT_REQUIRE(M < ((int64_t)1 << 31) && N < ((int64_t)1 << 31) && K < ((int64_t)1 << 31), OUDJAT_ERR_TOO_LARGE,
                 "linear_splitk_partial: dimensions must fit in int32");
  int S = 1;
  const int ci = choose_splitk(M, N, K, OUDJAT_EPI_BIAS_LS, &S);
  OUDJAT_REQUIRE(ci >= 0 && S > 1 && (int64_t)S * M * N <= workspace_elems, OUDJAT_ERR_UNSUPPORTED_SHAPE,
                 "linear_splitk_partial: %lld x %lld x %lld does not split K (or the workspace is short)",
                 (long long)M, (long long)N, (long long)K);
  *slices = S;
  EpiArgs ea{};
  ea.acc_scale = 1.0f;
  return launch_gemm(ci, A, M, K, lda, W, N, ldw, kEpiPartial, ea, reinterpret_cast<uint16_t*>(workspace), N,
                     as_stream(stream), "linear_splitk_partial", S);
}

// fp32 elements of workspace a linear_bf16 call of this shape can use for split K (0: it never splits).
extern "C" int64_t oudjat_linear_workspace_elems(int64_t M, int64_t N, int64_t K, int epi) {
  epi &= ~OUDJAT_EPI_RAW_BF16;
  int S = 1;
  if (M <= 0 || N <= 0 || K <= 0 || choose_splitk(M, N, K, epi, &S) < 0 || S <= 1) return 0;
  return (int64_t)S * M * N;
}

extern "C" int64_t oudjat_linear_warm_slots(int64_t M, int64_t N, int64_t K, int epi) {
  epi &= ~OUDJAT_EPI_RAW_BF16;
  if (M <= 0 || N <= 0 || K <= 0 || N % 64 != 0 || K % kBK != 0 || epi < OUDJAT_EPI_BIAS ||
      epi > OUDJAT_EPI_BIAS_SILU_MUL)
    return 0;
  int S = 1;
  if (choose_splitk(M, N, K, epi, &S) >= 0 && S > 1) return 0;  // split launches take none
  const GemmCfg& c = kCfgs[choose_cfg(M, N, K, true)];
  return warm_slots(c, cdiv(M, c.bm) * cdiv(N, c.bn));
}

static int linear_qkv_rope_kv_impl(const uint16_t* A, int64_t M, int64_t K, int64_t lda, const uint16_t* W,
                                   int64_t ldw, const uint16_t* bias, int64_t H, int64_t Dh, const float* sin_table,
                                   const float* cos_table, int64_t table_stride, const uint8_t* patch_mask,
                                   const int64_t* rope_idx, const int64_t* batch_idx, const int64_t* token_idx,
                                   uint16_t* kv, int64_t kv_stride_b, int64_t kv_stride_n, uint16_t* q_out,
                                   float acc_scale, int raw_round, oudjat_stream_t stream, const void* warm = nullptr,
                                   int64_t warm_bytes = 0) {
  OUDJAT_REQUIRE(M >= 0 && K >= 0 && H > 0 && Dh > 0, OUDJAT_ERR_INVALID_ARGUMENT, "linear_qkv_rope_kv: bad size");
  OUDJAT_REQUIRE(warm_bytes >= 0 && (warm_bytes == 0 || warm), OUDJAT_ERR_INVALID_ARGUMENT,
                 "linear_qkv_rope_kv: bad warm region (bytes < 0, or NULL with bytes > 0)");
  OUDJAT_REQUIRE(warm_bytes == 0 || aligned(warm, 4), OUDJAT_ERR_UNSUPPORTED_LAYOUT,
                 "linear_qkv_rope_kv: the warm region must be 4-byte aligned");
  if (M == 0) return OUDJAT_OK;
  const int64_t N = 3 * H * Dh;
  OUDJAT_REQUIRE(A && W && kv && q_out && sin_table && cos_table && patch_mask && rope_idx && batch_idx && token_idx,
                 OUDJAT_ERR_INVALID_ARGUMENT, "linear_qkv_rope_kv: null pointer");
  OUDJAT_REQUIRE(K > 0 && K % kBK == 0, OUDJAT_ERR_UNSUPPORTED_SHAPE,
                 "linear_qkv_rope_kv: K=%lld must be a multiple of %d", (long long)K, kBK);
  OUDJAT_REQUIRE(Dh % 16 == 0 && 128 % Dh == 0 && (H * Dh) % 128 == 0, OUDJAT_ERR_UNSUPPORTED_SHAPE,
                 "linear_qkv_rope_kv: need Dh in {16, 32, 64, 128} and H*Dh %% 128 == 0 (H=%lld, Dh=%lld)",
                 (long long)H, (long long)Dh);
  OUDJAT_REQUIRE(lda % 8 == 0 && ldw % 8 == 0 && lda >= K && ldw >= K && aligned(A, 16) && aligned(W, 16) &&
                     (!bias || aligned(bias, 8)) && aligned(kv, 16) && aligned(q_out, 16) && kv_stride_b % 8 == 0 &&
                     kv_stride_n % 8 == 0 && table_stride % 4 == 0 && aligned(sin_table, 16) && aligned(cos_table, 16),
                 OUDJAT_ERR_UNSUPPORTED_LAYOUT,
                 "linear_qkv_rope_kv: 16-byte aligned operands and rows, strides %% 8 == 0, tables 16-byte rows");
  OUDJAT_REQUIRE(M < ((int64_t)1 << 31) && N < ((int64_t)1 << 31) && K < ((int64_t)1 << 31), OUDJAT_ERR_TOO_LARGE,
                 "linear_qkv_rope_kv: dimensions must fit in int32");
  EpiArgs ea{};
  ea.bias = bias;
  ea.acc_scale = acc_scale;
  if (raw_round) {  // bf16(acc) at the first rounding point, then the scale and bias
    OUDJAT_REQUIRE(!bias || aligned(bias, 16), OUDJAT_ERR_UNSUPPORTED_LAYOUT,
                   "linear_qkv_rope_kv_nvfp4: 16-byte aligned bias required");
    ea.raw_round = 1;
    ea.raw_scale = acc_scale;
    ea.raw_bias = bias;
    ea.acc_scale = 1.0f;
    ea.bias = nullptr;
  }
  ea.qkv = QkvArgs{(int)H, (int)Dh, sin_table, cos_table, table_stride, patch_mask, rope_idx, batch_idx, token_idx,
                   kv, kv_stride_b, kv_stride_n, q_out};
  return launch_gemm(choose_qkv_cfg(M, N, K, Dh), A, M, K, lda, W, N, ldw, kEpiQkv, ea, nullptr, 0, as_stream(stream),
                     "linear_qkv_rope_kv", 1, warm, warm_bytes);
}

extern "C" int oudjat_linear_qkv_rope_kv(const uint16_t* A, int64_t M, int64_t K, int64_t lda, const uint16_t* W,
                                         int64_t ldw, const uint16_t* bias, int64_t H, int64_t Dh,
                                         const float* sin_table, const float* cos_table, int64_t table_stride,
                                         const uint8_t* patch_mask, const int64_t* rope_idx,
                                         const int64_t* batch_idx, const int64_t* token_idx, uint16_t* kv,
                                         int64_t kv_stride_b, int64_t kv_stride_n, uint16_t* q_out,
                                         float acc_scale, oudjat_stream_t stream) {
  return linear_qkv_rope_kv_impl(A, M, K, lda, W, ldw, bias, H, Dh, sin_table, cos_table, table_stride, patch_mask,
                                 rope_idx, batch_idx, token_idx, kv, kv_stride_b, kv_stride_n, q_out, acc_scale, 0,
                                 stream);
}

extern "C" int oudjat_linear_qkv_rope_kv_warm(const uint16_t* A, int64_t M, int64_t K, int64_t lda, const uint16_t* W,
                                              int64_t ldw, const uint16_t* bias, int64_t H, int64_t Dh,
                                              const float* sin_table, const float* cos_table, int64_t table_stride,
                                              const uint8_t* patch_mask, const int64_t* rope_idx,
                                              const int64_t* batch_idx, const int64_t* token_idx, uint16_t* kv,
                                              int64_t kv_stride_b, int64_t kv_stride_n, uint16_t* q_out,
                                              float acc_scale, const void* warm, int64_t warm_bytes,
                                              oudjat_stream_t stream) {
  return linear_qkv_rope_kv_impl(A, M, K, lda, W, ldw, bias, H, Dh, sin_table, cos_table, table_stride, patch_mask,
                                 rope_idx, batch_idx, token_idx, kv, kv_stride_b, kv_stride_n, q_out, acc_scale, 0,
                                 stream, warm, warm_bytes);
}

extern "C" int oudjat_linear_qkv_rope_kv_nvfp4(const uint16_t* A, int64_t M, int64_t K, int64_t lda,
                                               const uint16_t* W, int64_t ldw, const uint16_t* bias, int64_t H,
                                               int64_t Dh, const float* sin_table, const float* cos_table,
                                               int64_t table_stride, const uint8_t* patch_mask,
                                               const int64_t* rope_idx, const int64_t* batch_idx,
                                               const int64_t* token_idx, uint16_t* kv, int64_t kv_stride_b,
                                               int64_t kv_stride_n, uint16_t* q_out, float out_scale,
                                               oudjat_stream_t stream) {
  return linear_qkv_rope_kv_impl(A, M, K, lda, W, ldw, bias, H, Dh, sin_table, cos_table, table_stride, patch_mask,
                                 rope_idx, batch_idx, token_idx, kv, kv_stride_b, kv_stride_n, q_out, out_scale, 1,
                                 stream);
}

static int kernel_name_of(const GemmCfg& c, int epi, char* buf, int64_t buflen);

// Kernel a linear_bf16 call of this shape would launch, as the demangled name profilers print
// (aligned operands assumed). For matching profile summaries to the running build.
extern "C" int oudjat_linear_kernel_name(int64_t M, int64_t N, int64_t K, int epi, char* buf, int64_t buflen) {
  OUDJAT_REQUIRE(buf && buflen > 0, OUDJAT_ERR_INVALID_ARGUMENT, "linear_kernel_name: no buffer");
  OUDJAT_REQUIRE(M > 0 && N > 0 && K > 0 && epi >= 0 && epi <= kEpiQkv, OUDJAT_ERR_INVALID_ARGUMENT,
                 "linear_kernel_name: bad arguments");
  int S = 1;
  const int sk = epi == kEpiQkv ? -1 : choose_splitk(M, N, K, epi, &S);
  if (sk >= 0 && S > 1) epi = kEpiPartial;  // split K (with a workspace): the partial kernel, then the reduce
  const GemmCfg& c = kCfgs[sk >= 0 && S > 1 ? sk : (epi == kEpiQkv ? choose_qkv_cfg(M, N, K, 64) : choose_cfg(M, N, K, true))];
  return kernel_name_of(c, epi, buf, buflen);
}

// The same for oudjat_linear_fp8 (epi = 5: oudjat_linear_qkv_rope_kv_fp8).
extern "C" int oudjat_linear_fp8_kernel_name(int64_t M, int64_t N, int64_t K, int epi, char* buf, int64_t buflen) {
  OUDJAT_REQUIRE(buf && buflen > 0, OUDJAT_ERR_INVALID_ARGUMENT, "linear_fp8_kernel_name: no buffer");
  OUDJAT_REQUIRE(M > 0 && N > 0 && K > 0 && N % 256 == 0 && epi >= 0 && epi <= kEpiQkv, OUDJAT_ERR_INVALID_ARGUMENT,
                 "linear_fp8_kernel_name: bad arguments");
  return kernel_name_of(kCfgs[choose_cfg_fp8(M, N)], epi, buf, buflen);
}

static int kernel_name_of(const GemmCfg& c, int epi, char* buf, int64_t buflen) {
  int n;
  if (c.pf == -4)
    n = snprintf(buf, (size_t)buflen, "oudjat::gemm_bf16_pp_kernel<%d, %d, %d, true>", c.bm, c.bn, epi);
  else if (c.pf == -3)
    n = snprintf(buf, (size_t)buflen, "oudjat::gemm_bf16_pp_kernel<%d, %d, %d>", c.bm, c.bn, epi);
  else if (c.pf == -2)
    n = snprintf(buf, (size_t)buflen, "oudjat::gemm_bf16_r16_kernel<%d, %d, %d, %d, %d, %d, %d, %s, %d>", c.bm, c.bn,
                 c.wgm, c.wgn, c.ks, c.bk, c.nst, c.fb ? "true" : "false", epi);
  else if (c.pf == -1)
    n = snprintf(buf, (size_t)buflen, "oudjat::gemm_bf16_pipe_kernel<%d, %d, %d, %d, %d>", c.bm, c.bn, c.wgm, c.wgn, epi);
  else if (c.pf == 0)
    n = snprintf(buf, (size_t)buflen, "oudjat::gemm_bf16_dma_kernel<%d, %d, %d, %d, %d>", c.bm, c.bn, c.wgm, c.wgn, epi);
  else
    n = snprintf(buf, (size_t)buflen, "oudjat::gemm_bf16_kernel<%d, %d, %d, %d, %d, %d>", c.bm, c.bn, c.wgm, c.wgn, c.pf,
                 epi);
  OUDJAT_REQUIRE(n >= 0 && n < buflen, OUDJAT_ERR_INVALID_ARGUMENT, "linear_kernel_name: buffer too small");
  return OUDJAT_OK;
}

// ------------------------------------------------------------------------------------------------
// FP8 (e4m3fn) products: torch._scaled_mm of FastFP8Linear (fp8_fast_linear.py:174-196) on the
// native FP8 MFMA. Operand and output rules as oudjat_linear_bf16 except: one byte per operand
// element, K % 128 == 0, N % 256 == 0, lda % 16 == 0 and ldw % 16 == 0 (16-byte rows), aligned
// epilogue operands, no GELU epilogue, no split K.
// ------------------------------------------------------------------------------------------------

static int check_fp8_operands(const uint8_t* A, int64_t M, int64_t K, int64_t lda, const uint8_t* W, int64_t N,
                              int64_t ldw, const char* what) {
  OUDJAT_REQUIRE(A && W, OUDJAT_ERR_INVALID_ARGUMENT, "%s: null operand", what);
  OUDJAT_REQUIRE(K > 0 && K % 128 == 0 && N % 256 == 0, OUDJAT_ERR_UNSUPPORTED_SHAPE,
                 "%s: need K %% 128 == 0 and N %% 256 == 0 (K=%lld, N=%lld)", what, (long long)K, (long long)N);
  OUDJAT_REQUIRE(lda % 16 == 0 && ldw % 16 == 0 && lda >= K && ldw >= K && aligned(A, 16) && aligned(W, 16),
                 OUDJAT_ERR_UNSUPPORTED_LAYOUT, "%s: 16-byte aligned operand rows required", what);
  OUDJAT_REQUIRE(M < ((int64_t)1 << 31) && N < ((int64_t)1 << 31) && M * lda < ((int64_t)1 << 32) &&
                     N * ldw < ((int64_t)1 << 32),
                 OUDJAT_ERR_TOO_LARGE, "%s: operands beyond 4 GiB or 2^31 rows", what);
  return OUDJAT_OK;
}

extern "C" int oudjat_linear_fp8(const uint8_t* A, int64_t M, int64_t K, int64_t lda, const uint8_t* W, int64_t N,
                                 int64_t ldw, const uint16_t* bias, int epi, const uint16_t* gamma,
                                 const uint16_t* resid, int64_t ldr, uint16_t* C, int64_t ldc, float acc_scale,
                                 oudjat_stream_t stream) {
  OUDJAT_REQUIRE(M >= 0 && N >= 0 && K >= 0, OUDJAT_ERR_INVALID_ARGUMENT, "linear_fp8: negative size");
  OUDJAT_REQUIRE(epi == OUDJAT_EPI_BIAS || epi == OUDJAT_EPI_BIAS_LS_RESID || epi == OUDJAT_EPI_BIAS_LS ||
                     epi == OUDJAT_EPI_BIAS_SILU_MUL,
                 OUDJAT_ERR_INVALID_ARGUMENT, "linear_fp8: unsupported epilogue %d", epi);
  if (M == 0 || N == 0) return OUDJAT_OK;
  const int st = check_fp8_operands(A, M, K, lda, W, N, ldw, "linear_fp8");
  if (st != OUDJAT_OK) return st;
  OUDJAT_REQUIRE(C, OUDJAT_ERR_INVALID_ARGUMENT, "linear_fp8: null output");
  OUDJAT_REQUIRE((epi != OUDJAT_EPI_BIAS_LS && epi != OUDJAT_EPI_BIAS_LS_RESID) || gamma, OUDJAT_ERR_INVALID_ARGUMENT,
                 "linear_fp8: epilogue needs gamma");
  OUDJAT_REQUIRE((epi != OUDJAT_EPI_BIAS_LS_RESID && epi != OUDJAT_EPI_BIAS_SILU_MUL) || resid,
                 OUDJAT_ERR_INVALID_ARGUMENT, "linear_fp8: epilogue needs resid");
  OUDJAT_REQUIRE(aligned(C, 16) && ldc % 8 == 0 && ldc >= N && (!bias || aligned(bias, 8)) &&
                     (!gamma || aligned(gamma, 16)) && (!resid || (aligned(resid, 16) && ldr % 8 == 0)),
                 OUDJAT_ERR_UNSUPPORTED_LAYOUT, "linear_fp8: 16-byte aligned output, residual and gamma rows required");
  EpiArgs ea{};
  ea.bias = bias;
  ea.gamma = gamma;
  ea.resid = resid;
  ea.ldr = ldr;
  ea.acc_scale = acc_scale;
  return launch_gemm(choose_cfg_fp8(M, N), reinterpret_cast<const uint16_t*>(A), M, K, lda,
                     reinterpret_cast<const uint16_t*>(W), N, ldw, epi, ea, C, ldc, as_stream(stream), "linear_fp8");
}

extern "C" int oudjat_linear_qkv_rope_kv_fp8(const uint8_t* A, int64_t M, int64_t K, int64_t lda, const uint8_t* W,
                                             int64_t ldw, const uint16_t* bias, int64_t H, int64_t Dh,
                                             const float* sin_table, const float* cos_table, int64_t table_stride,
                                             const uint8_t* patch_mask, const int64_t* rope_idx,
                                             const int64_t* batch_idx, const int64_t* token_idx, uint16_t* kv,
                                             int64_t kv_stride_b, int64_t kv_stride_n, uint16_t* q_out,
                                             float acc_scale, oudjat_stream_t stream) {
  OUDJAT_REQUIRE(M >= 0 && K >= 0 && H > 0 && Dh > 0, OUDJAT_ERR_INVALID_ARGUMENT, "linear_qkv_rope_kv_fp8: bad size");
  if (M == 0) return OUDJAT_OK;
  const int64_t N = 3 * H * Dh;
  OUDJAT_REQUIRE(kv && q_out && sin_table && cos_table && patch_mask && rope_idx && batch_idx && token_idx,
                 OUDJAT_ERR_INVALID_ARGUMENT, "linear_qkv_rope_kv_fp8: null pointer");
  OUDJAT_REQUIRE(Dh % 16 == 0 && 128 % Dh == 0, OUDJAT_ERR_UNSUPPORTED_SHAPE,
                 "linear_qkv_rope_kv_fp8: need Dh in {16, 32, 64, 128} (Dh=%lld)", (long long)Dh);
  const int st = check_fp8_operands(A, M, K, lda, W, N, ldw, "linear_qkv_rope_kv_fp8");
  if (st != OUDJAT_OK) return st;
  OUDJAT_REQUIRE((!bias || aligned(bias, 8)) && aligned(kv, 16) && aligned(q_out, 16) && kv_stride_b % 8 == 0 &&
                     kv_stride_n % 8 == 0 && table_stride % 4 == 0 && aligned(sin_table, 16) && aligned(cos_table, 16),
                 OUDJAT_ERR_UNSUPPORTED_LAYOUT,
                 "linear_qkv_rope_kv_fp8: 16-byte aligned outputs and rows, strides %% 8 == 0, tables 16-byte rows");
  EpiArgs ea{};
  ea.bias = bias;
  ea.acc_scale = acc_scale;
  ea.qkv = QkvArgs{(int)H, (int)Dh, sin_table, cos_table, table_stride, patch_mask, rope_idx, batch_idx, token_idx,
                   kv, kv_stride_b, kv_stride_n, q_out};
  return launch_gemm(choose_cfg_fp8(M, N), reinterpret_cast<const uint16_t*>(A), M, K, lda,
                     reinterpret_cast<const uint16_t*>(W), N, ldw, kEpiQkv, ea, nullptr, 0, as_stream(stream),
                     "linear_qkv_rope_kv_fp8");
}
