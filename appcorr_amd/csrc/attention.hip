// Sparse-query attention against the full K/V cache.
//
// Queries: the T selected rows of each image (packed [B*T, H, Dh]); keys/values: all N cached rows of
// the same image, read in place from the [B, N, 2, H, Dh] cache (K after RoPE, V raw), no mask.
//
// Formulation: each wave owns 32 queries and computes the transposed products
//     S^T = K . Q^T          (32 keys x 32 queries per v_mfma_f32_32x32x16_bf16 block)
//     O^T += V^T . P^T       (32 head dims x 32 queries)
// so that, in the 32x32 accumulator layout, one query is one lane pair (lanes l and l^32) and all of
// its scores sit in that pair's registers:
//   * the online-softmax max / sum of a query is a register reduction plus one xor-32 exchange;
//   * P^T feeds the second MFMA straight from registers (no LDS round trip). The contraction order
//     of that MFMA is taken from the accumulator layout: lane group g supplies keys
//     16j + 4g + {0..3} and 16j + 8 + 4g + {0..3} of k-step j, and V^T is read in that same order;
//   * K (the A operand of the first product) is read from LDS in its natural row layout.
// V stays in its natural [key][dim] rows in LDS, like K; the V^T operand comes from them through
// the LDS transpose read (ds_read_tr16_b64, its lane mapping described above the buffer-load
// kernel).
//
// One workgroup per (image, head) covers up to 10 query waves = 320 queries (8 for Dh = 128); larger T
// is split evenly over several workgroups. At the headline shape (T = 261: 8 full waves and a last
// wave of 5 queries, 256 workgroups for B*H = 256, one per CU) the buffer-load kernel shares the
// last wave's key tiles among 4 waves, so each workgroup runs 12. K/V tiles of 64 keys are double-buffered in LDS with the next tile's global loads in
// flight during the current tile's MFMAs, so each (image, head) streams its K/V once.
#include <stdlib.h>

#include <type_traits>

#include "common.hpp"
#include "fp8.hpp"

namespace oudjat {

static constexpr int kKeyTile = 64;
static constexpr int kMaxWaves64 = 10;   // Dh = 64: 3 waves per SIMD, <= 170 VGPRs
static constexpr int kLightParts = 4;     // waves that share a light (<= 16-query) last wave, one per SIMD
static constexpr int kDmaMaxWaves = 12;   // buffer-load kernel: up to 8 full waves + kLightParts
static constexpr int kMaxWaves128 = 8;   // Dh = 128: 2 waves per SIMD, <= 256 VGPRs
static constexpr int kMinWaves = 4;

typedef float f32x8_t __attribute__((ext_vector_type(8)));

// Eight fp32 -> bf16 (RNE) as four packed converts.
__device__ __forceinline__ bf16x8_t pack_bf16x8(const float* f) {
  const f32x8_t v = {f[0], f[1], f[2], f[3], f[4], f[5], f[6], f[7]};
  return __builtin_convertvector(v, bf16x8_t);
}

// Reference maximum of the online softmax: it moves to the running maximum only when that exceeds it
// by more than 8 in the exp2 domain (and always from -inf), so most tiles keep the same reference and
// skip rescaling the output; probabilities stay below 2^8 and the final O / l is unchanged.
__device__ __forceinline__ float softmax_ref_max(float m_ref, float tile_max, float scale_log2) {
  const float m_run = fmaxf(m_ref, tile_max);
  return (m_run - m_ref) * scale_log2 > 8.0f ? m_run : m_ref;
}

// Sum of one query's probabilities over a key tile, taken from the bf16 values the O^T MFMAs
// multiply (so numerator and normaliser use the same weights): packed dot products against (1, 1),
// then the partner lane's half (lanes l and l ^ 32 hold the two halves of a query's keys).
// Lane exchange with lane l ^ 32 through v_permlane32_swap (a VALU op, no LDS round trip): swapping
// the halves of two copies of x leaves x_l and x_{l^32} in the two results of every lane.
__device__ __forceinline__ float xor32_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// The same with lane l ^ 16 through v_permlane16_swap (rows of 16 lanes swapped pairwise).
__device__ __forceinline__ float xor16_max(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor16_sum(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float prob_row_sum(const bf16x8_t (&pf)[4]) {
  typedef __bf16 bf16x2v_t __attribute__((ext_vector_type(2)));
  const bf16x2v_t ones = {(__bf16)1.0f, (__bf16)1.0f};
  float r[4];  // one short chain per k-step, combined as a tree
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    r[j] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(pf[j], pf[j], 0, 1), ones, 0.0f, false);
    r[j] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(pf[j], pf[j], 2, 3), ones, r[j], false);
    r[j] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(pf[j], pf[j], 4, 5), ones, r[j], false);
    r[j] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(pf[j], pf[j], 6, 7), ones, r[j], false);
  }
  return xor32_sum((r[0] + r[1]) + (r[2] + r[3]));
}

// MINW: fewest waves a launch of this instance uses (sizes the per-thread share of a K/V tile);
// DOUBLE_SET: prefetch K/V two tiles ahead through two register sets (needs the registers that only
// the Dh = 64, >= 8-wave instance has to spare).
// LSE: also write each query's row log-sum-exp (natural log) of the scaled scores to lse[b][h][t],
// from an fp32 sum of the unrounded probabilities kept beside the bf16-weight sum that normalises
// the output (the output is the same bit for bit either way).
// F8OUT: the output row is written instead as the e4m3fn codes of its bf16 values times *f8s, the
// consuming FP8 linear's activation quantizer (fp8_act_code) applied in the store: out8, one byte per
// element, row stride ors.
template <int DH, int MINW, bool DOUBLE_SET, bool LSE = false, bool F8OUT = false>
__global__ __launch_bounds__((DH == 64 ? kMaxWaves64 : kMaxWaves128) * 64) void sq_attention_kernel(
    const uint16_t* __restrict__ q, int64_t qrs, int T, const uint16_t* __restrict__ kv, int64_t kvb, int64_t kvn,
    int64_t kvkv, int64_t kvh, int N, float scale_log2, uint16_t* __restrict__ out, int64_t ors,
    int waves_per_wg, float* __restrict__ lse, uint8_t* __restrict__ out8 = nullptr,
    const float* __restrict__ f8s = nullptr) {
  constexpr int CPR = DH / 8;                 // 16-byte chunks per K / V row
  constexpr int KROWB = DH * 2;               // bytes per K / V row in LDS
  constexpr int KSTAGE = kKeyTile * KROWB;
  constexpr int VSTAGE = kKeyTile * KROWB;
  constexpr int STAGE = KSTAGE + VSTAGE;
  constexpr int QK_STEPS = DH / 16;
  constexpr int OB = DH / 32;
  constexpr int ITEMS = kKeyTile * CPR;       // 16-byte chunks per K (or V) tile
  constexpr int IT = (ITEMS + MINW * 64 - 1) / (MINW * 64);

  extern __shared__ __align__(16) unsigned char smem[];
  typedef short i16x4_t __attribute__((ext_vector_type(4)));

  // The query workgroups of one (image, head) all stream the same K/V: numbered so that they run on
  // one XCD (dispatch places workgroup i on XCD i % 8) and share its L2. Workgroup i = x + 8 s on
  // XCD x takes query block s % nq of pair 8 (s / nq) + x; a bijection when the pair count is a
  // multiple of 8, else the launch order is kept.
  int qblk = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  {
    const int nq = gridDim.x, pairs = gridDim.y * gridDim.z;
    if (nq > 1 && pairs % 8 == 0) {
      const int lin = blockIdx.x + nq * (blockIdx.y + gridDim.y * blockIdx.z);
      const int x = lin & 7, sl = lin >> 3;
      const int pair = 8 * (sl / nq) + x;
      qblk = sl % nq;
      h = pair % gridDim.y;
      b = pair / gridDim.y;
    }
  }
  const int nthreads = blockDim.x;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, g = lane >> 5;
  const int q0 = (qblk * waves_per_wg + wave) * 32;
  const bool active = q0 < T;

  // Q^T fragments (B operand of S^T): lane -> query q0 + l32, head dims ks*16 + 8g .. +7.
  bf16x8_t qf[QK_STEPS];
  {
    const int qr = q0 + l32;
#pragma unroll
    for (int ks = 0; ks < QK_STEPS; ++ks) {
      uint4 v = make_uint4(0, 0, 0, 0);
      if (qr < T) v = *reinterpret_cast<const uint4*>(q + ((int64_t)b * T + qr) * qrs + (int64_t)h * DH + ks * 16 + 8 * g);
      qf[ks] = as_bf16x8(v);
    }
  }

  f32x16_t o[OB];
#pragma unroll
  for (int d = 0; d < OB; ++d)
#pragma unroll
    for (int v = 0; v < 16; ++v) o[d][v] = 0.0f;
  float m_i = -INFINITY, l_i = 0.0f;
  float lf = 0.0f;  // LSE: this lane's half of the fp32 probability sum

  const uint16_t* kbase = kv + (int64_t)b * kvb + (int64_t)h * kvh;
  const uint16_t* vbase = kbase + kvkv;
  const int ntiles = (N + kKeyTile - 1) / kKeyTile;

  // K/V tiles travel global -> registers -> LDS. Two register sets let the global loads of tile
  // t + 2 be in flight while tile t is computed and tile t + 1 is written to LDS.
  struct TileRegs {
    u32x4_t k[IT], v[IT];
  };
  auto load_tile = [&](TileRegs& r, int t) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int c = tid + i * nthreads;
      r.k[i] = u32x4_t{0, 0, 0, 0};
      r.v[i] = u32x4_t{0, 0, 0, 0};
      if (c < ITEMS) {
        const int kk = c / CPR, kc = c - kk * CPR;       // K: row-major, 8 lanes per 128-byte row
        const int nk = t * kKeyTile + kk;
        if (nk < N) r.k[i] = *reinterpret_cast<const u32x4_t*>(kbase + (int64_t)nk * kvn + kc * 8);
        if (nk < N) r.v[i] = *reinterpret_cast<const u32x4_t*>(vbase + (int64_t)nk * kvn + kc * 8);
      }
    }
  };
  auto store_tile = [&](const TileRegs& r, int stage) __attribute__((always_inline)) {
    unsigned char* ks = smem + stage * STAGE;
    unsigned char* vs = ks + KSTAGE;
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int c = tid + i * nthreads;
      if (c < ITEMS) {
        const int kk = c / CPR, kc = c - kk * CPR;
        const int slot = kk * KROWB + ((kc ^ (kk & (CPR - 1))) << 4);
        *reinterpret_cast<u32x4_t*>(ks + slot) = r.k[i];
        *reinterpret_cast<u32x4_t*>(vs + slot) = r.v[i];
      }
    }
  };

  // V^T fragment sources of d-block d: lane (g, 16-lane half hh, s = lane % 16) addresses dims
  // 32 d + 16 hh + 4 (s % 4) .. + 3 of key 4 g + s / 4 (first run of k-step 0) and of that key + 8
  // (second run); k-step j adds 16 j keys, whose swizzle is the same.
  int voff[OB][2];
  {
    const int sl = lane & 15, hh = (lane >> 4) & 1;
#pragma unroll
    for (int d = 0; d < OB; ++d) {
      const int dcol = 32 * d + 16 * hh + 4 * (sl & 3);
#pragma unroll
      for (int run = 0; run < 2; ++run) {
        const int key = 4 * g + (sl >> 2) + 8 * run;
        voff[d][run] = KSTAGE + key * KROWB + (((dcol >> 3) ^ (key & (CPR - 1))) << 4) + ((dcol >> 2) & 1) * 8;
      }
    }
  }

  auto compute = [&](int stage, int t) __attribute__((always_inline)) {
    const unsigned char* ks = smem + stage * STAGE;
    // S^T blocks: s[kb][v] = S^T[key kb*32 + 8(v/4) + 4g + v%4][query l32]
    // The K fragments of a 32-key block (both blocks for Dh = 64) are read before its MFMAs so the
    // reads overlap.
    constexpr int KB_BATCH = DH == 64 ? 2 : 1;
    f32x16_t s[2];
#pragma unroll
    for (int kb0 = 0; kb0 < 2; kb0 += KB_BATCH) {
      bf16x8_t kf[KB_BATCH][QK_STEPS];
#pragma unroll
      for (int kb = 0; kb < KB_BATCH; ++kb) {
        const int key = (kb0 + kb) * 32 + l32;
#pragma unroll
        for (int kstep = 0; kstep < QK_STEPS; ++kstep) {
          const int ch = kstep * 2 + g;
          kf[kb][kstep] =
              as_bf16x8(*reinterpret_cast<const uint4*>(ks + key * KROWB + ((ch ^ (key & (CPR - 1))) << 4)));
        }
      }
#pragma unroll
      for (int kb = 0; kb < KB_BATCH; ++kb) {
#pragma unroll
        for (int v = 0; v < 16; ++v) s[kb0 + kb][v] = 0.0f;
#pragma unroll
        for (int kstep = 0; kstep < QK_STEPS; ++kstep)
          s[kb0 + kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[kb][kstep], qf[kstep], s[kb0 + kb], 0, 0, 0);
      }
    }
    if ((t + 1) * kKeyTile > N) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int v = 0; v < 16; ++v)
          if (t * kKeyTile + kb * 32 + 8 * (v >> 2) + 4 * g + (v & 3) >= N) s[kb][v] = -INFINITY;
    }
    float mx = s[0][0];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int v = 0; v < 16; ++v) mx = fmaxf(mx, s[kb][v]);
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    // exp2 is the bare v_exp_f32 (no subnormal range reduction: a probability below 2^-126 adds
    // nothing to a sum that contains a term >= 1).
    const float m_new = softmax_ref_max(m_i, mx, scale_log2);
    const float alpha = __builtin_amdgcn_exp2f((m_i - m_new) * scale_log2);
    const float mc = m_new * scale_log2;
    if constexpr (LSE) lf *= alpha;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        s[kb][v] = __builtin_amdgcn_exp2f(fmaf(s[kb][v], scale_log2, -mc));
        if constexpr (LSE) lf += s[kb][v];
      }
    // P^T fragments: k-step j covers keys 16j + {4g..4g+3} and 16j + 8 + {4g..4g+3}.
    bf16x8_t pf[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float tmp[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) tmp[e] = s[j >> 1][8 * (j & 1) + e];
      pf[j] = pack_bf16x8(tmp);
    }
    const float rs = prob_row_sum(pf);
    l_i = l_i * alpha + rs;
    m_i = m_new;
    // Rescale the output only when some query's reference max moved (alpha != 1 somewhere in the
    // wave).
    if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
#pragma unroll
      for (int d = 0; d < OB; ++d)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[d][v] *= alpha;
    }
#pragma unroll
    for (int d = 0; d < OB; ++d) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) i16x4_t*)(ks + voff[d][0] + j * 16 * KROWB));
        const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) i16x4_t*)(ks + voff[d][1] + j * 16 * KROWB));
        typedef short i16x8_t __attribute__((ext_vector_type(8)));
        const i16x8_t both = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        o[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, both), pf[j], o[d], 0, 0, 0);
      }
    }
  };

  if constexpr (DOUBLE_SET) {
    TileRegs ra, rb;
    load_tile(ra, 0);
    if (ntiles > 1) load_tile(rb, 1);
    store_tile(ra, 0);
    __syncthreads();
    // Iteration t: loads of tile t + 2 into the set that held tile t, compute tile t, store tile
    // t + 1 (loaded one iteration earlier) into the other LDS stage.
    auto step = [&](int t, TileRegs& cur_next, TileRegs& other) __attribute__((always_inline)) {
      if (t + 2 < ntiles) load_tile(cur_next, t + 2);
      if (active) compute(t & 1, t);
      if (t + 1 < ntiles) store_tile(other, (t + 1) & 1);
      __syncthreads();
    };
    int t = 0;
    for (; t + 1 < ntiles; t += 2) {
      step(t, ra, rb);
      step(t + 1, rb, ra);
    }
    if (t < ntiles) step(t, ra, rb);
  } else {
    TileRegs r;
    load_tile(r, 0);
    store_tile(r, 0);
    __syncthreads();
    for (int t = 0; t < ntiles; ++t) {
      if (t + 1 < ntiles) load_tile(r, t + 1);
      if (active) compute(t & 1, t);
      if (t + 1 < ntiles) store_tile(r, (t + 1) & 1);
      __syncthreads();
    }
  }

  // O^T[d][q]: lane l, register v of block db -> d = db*32 + 8(v/4) + 4g + v%4 (4 consecutive d per
  // group of 4 registers -> one 8-byte store), q = q0 + l32.
  const int qr = q0 + l32;
  if (F8OUT && active && qr < T) {
    const float inv = 1.0f / l_i;
    const float s8 = *f8s;
    uint8_t* orow = out8 + ((int64_t)b * T + qr) * ors + (int64_t)h * DH;
#pragma unroll
    for (int d = 0; d < OB; ++d)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        uint32_t w = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) w |= fp8_act_code(round_bf16(o[d][4 * r4 + e] * inv), s8) << (8 * e);
        *reinterpret_cast<uint32_t*>(orow + d * 32 + 8 * r4 + 4 * g) = w;
      }
  } else if (active && qr < T) {
    const float inv = 1.0f / l_i;
    uint16_t* orow = out + ((int64_t)b * T + qr) * ors + (int64_t)h * DH;
#pragma unroll
    for (int d = 0; d < OB; ++d)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
        bf16x4_t w;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = (__bf16)(o[d][4 * r4 + e] * inv);
        *reinterpret_cast<bf16x4_t*>(orow + d * 32 + 8 * r4 + 4 * g) = w;
      }
  }
  if constexpr (LSE) {
    // lse = ln(sum_k exp(s_k * scale)) = (m * scale * log2 e + log2 l) * ln 2, with the probabilities
    // exp2(s * scale * log2 e - m * scale * log2 e) of the loop (m the reference max).
    if (active) {
      const float lt = xor32_sum(lf);
      if (g == 0 && qr < T)
        lse[((int64_t)b * gridDim.y + h) * T + qr] = (m_i * scale_log2 + log2f(lt)) * 0.6931471805599453f;
    }
  }
}


// ------------------------------------------------------------------------------------------------
// Dh = 64, >= 8 waves: K and V tiles reach LDS by buffer loads straight from the cache (no register
// staging), both in their natural [key][dim] rows, NST stages deep. Waves 0..7 each load 8 rows of K
// and 8 rows of V per tile (one 1 KB instruction each); keys past N fall outside the per-(image,
// head) descriptors and load as zeros (their scores are masked). The A operand of O^T += V^T . P^T
// comes from V's rows through the LDS transpose read: in each 16-lane group, source lane s addresses
// 4 dims (8 bytes) of key k0 + s / 4 at dim c0 + 4 (s % 4), and lane j receives dim c0 + j for keys
// k0 .. k0 + 3. Rows are 128 bytes; 16-byte chunk c of key row r sits in slot c ^ kv_swz(r) (below).
// The arithmetic (MFMA order, softmax, P rounding) is that of sq_attention_kernel, so both give
// bit-identical outputs.
// ------------------------------------------------------------------------------------------------

// Slot of 16-byte chunk `chunk` in 128-byte key row `row`: chunk ^ sw(row), sw a permutation of the
// row pair m = (row >> 1) & 7 (so 16 consecutive keys at one chunk cover all 64 banks) that also
// flips bit 2 on odd pairs (so keys k and k + 2 -- one 4x16 transpose read -- use opposite halves
// of the row). sw(row + 16 j) = sw(row).
__device__ __forceinline__ int kv_swz(int row) {
  const int m = (row >> 1) & 7;
  return m ^ ((m & 1) << 2);
}
__device__ __forceinline__ int kv_slot(int row, int chunk) { return row * 128 + ((chunk ^ kv_swz(row)) << 4); }

// light_split: 0, or kLightParts when the launch has one workgroup per (image, head) whose last
// query wave is light; that wave's work is then done by kLightParts waves (the last ones), part p
// taking the key tiles t with t % NST == p, and merged at the end (see the light path below).
// full_split: 1, or 2 (small T, one workgroup per (image, head)): each full query wave's work is done
// by two waves, part p taking the tiles of stages p and p + 2, merged at the end like the light
// parts, so that a workgroup of few query waves still puts two or three waves on every SIMD.
// full_split is a template parameter so that without it the full waves' stage mask is a constant and
// each tile's S^T MFMAs and the previous tile's softmax stay in one basic block (interleaved).
// Key-part workspace of a split launch, per (image, head, part): the running max of each query
// (kv_part_rows(T) floats, T rounded up to 4 so the rows below stay 16-byte aligned), its sum (as
// many), then its unnormalised 64-dim output rows (T x 64).
__host__ __device__ __forceinline__ int64_t kv_part_rows(int64_t T) { return (T + 3) & ~(int64_t)3; }
__host__ __device__ __forceinline__ int64_t kv_part_stride(int64_t T) { return 2 * kv_part_rows(T) + 64 * T; }

template <int NST, int FSPLIT, bool KVS>
__global__ __launch_bounds__(kDmaMaxWaves * 64) void sq_attention_dma_kernel(
    const uint16_t* __restrict__ q, int64_t qrs, int T, const uint16_t* __restrict__ kv, int64_t kvb, int64_t kvn,
    int64_t kvkv, int64_t kvh, int N, float scale_log2, uint16_t* __restrict__ out, int64_t ors,
    int waves_per_wg, int light_split, float* __restrict__ part_ws, int kv_parts) {
  constexpr int full_split = FSPLIT;
  static_assert(FSPLIT == 1 || FSPLIT == 2, "full_split");
  constexpr int DH = 64, QK_STEPS = 4, OB = 2;
  constexpr int TILEB = kKeyTile * 128;  // one K (or V) tile: 64 rows of 128 bytes
  constexpr int STAGE = 2 * TILEB;
  static_assert(NST >= 2, "stages");
  typedef short i16x4_t __attribute__((ext_vector_type(4)));

  extern __shared__ __align__(16) unsigned char smem[];

  const int b = blockIdx.z, h = blockIdx.y;
  // KVS: one query workgroup per (image, head) and blockIdx.x = key part (contiguous tile ranges).
  const int qblk = KVS ? 0 : (int)blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l32 = lane & 31, g = lane >> 5;
  // Query wave of this wave, its part of a split full wave (fpart, 0 without a split) and its part of
  // a split light wave (lpart, -1: not split). Full query waves 0 .. nfq - 1 take waves
  // [0, nfq * full_split), the split light wave the kLightParts waves after them.
  const int nfq = light_split ? waves_per_wg - 1 : waves_per_wg;
  const int lpart = (light_split && wave >= nfq * full_split) ? wave - nfq * full_split : -1;
  const int fpart = lpart >= 0 ? 0 : wave % full_split;
  const int qwave = lpart >= 0 ? waves_per_wg - 1 : wave / full_split;
  const int q0 = (qblk * waves_per_wg + qwave) * 32;
  const bool active = q0 < T;
  const bool merged = light_split || full_split > 1;  // the parts meet in LDS after the key loop

  const uint16_t* kbase = kv + (int64_t)b * kvb + (int64_t)h * kvh;
  const uint32_t bytes = (uint32_t)((int64_t)N * kvn * 2);
  const i32x4_t rsrc_k = make_buffer_rsrc(kbase, bytes);
  const i32x4_t rsrc_v = make_buffer_rsrc(kbase + kvkv, bytes);
  const bool loader = wave < 8;
  const int lrow = 8 * wave + (lane >> 3);                  // tile row this lane loads
  const uint32_t tstep = (uint32_t)kKeyTile * (uint32_t)kvn * 2u;
  // Key tiles of this workgroup: [tb, tb + ntiles); tiles are numbered from tb in the loops below.
  int tb = 0, ntiles = (N + kKeyTile - 1) / kKeyTile;
  if constexpr (KVS) {
    const int per = (ntiles + kv_parts - 1) / kv_parts;
    tb = (int)blockIdx.x * per;
    ntiles = min(per, ntiles - tb);
  }
  const uint32_t off0 = (uint32_t)lrow * (uint32_t)kvn * 2u + (uint32_t)(((lane & 7) ^ kv_swz(lrow)) << 4) +
                        (uint32_t)tb * tstep;
  auto issue = [&](int stage, int t) __attribute__((always_inline)) {
    if (loader) {
      unsigned char* base = smem + stage * STAGE + wave * 1024;
      buffer_load_lds16(rsrc_k, base, off0 + (uint32_t)t * tstep);
      buffer_load_lds16(rsrc_v, base + TILEB, off0 + (uint32_t)t * tstep);
    }
  };
  // At most n tiles after the one needed may still be in flight (two loads per tile per loader).
  static_assert(NST <= 5, "wait_tiles covers up to three tiles in flight");
  auto wait_tiles = [&](int n) __attribute__((always_inline)) {
    if (n <= 0) wait_vmcnt<0>();
    else if (n == 1) wait_vmcnt<2>();
    else if (n == 2) wait_vmcnt<4>();
    else wait_vmcnt<6>();
  };

  // Query fragments, loaded before the K/V prologue so that their latency overlaps the first tiles'
  // (the prologue's vmcnt waits then cover them as older loads). Full wave (T - q0 > 16): query
  // q0 + lane % 32, dims 16 ks + 8 (lane / 32) .. + 7; light wave: query q0 + lane % 16, dims
  // 32 ks + 8 (lane / 16) .. + 7, ks < 2.
  const bool full_wave = T - q0 > 16;
  uint4 qraw[QK_STEPS];
  {
    const int qr = q0 + (full_wave ? l32 : (lane & 15));
    const int dim0 = full_wave ? 8 * g : 8 * (lane >> 4);
    const int kstride = full_wave ? 16 : 32;
    const uint16_t* qrow = q + ((int64_t)b * T + qr) * qrs + (int64_t)h * DH + dim0;
#pragma unroll
    for (int ks = 0; ks < QK_STEPS; ++ks) {
      qraw[ks] = make_uint4(0, 0, 0, 0);
      if (qr < T && (full_wave || ks < 2)) qraw[ks] = *reinterpret_cast<const uint4*>(qrow + ks * kstride);
    }
  }

  // The prologue of the K/V pipeline is common to both wave kinds below.
  static_assert(NST == 4, "the unrolled loops below are written for four stages");
#pragma unroll
  for (int st = 0; st < NST - 1; ++st)
    if (st < ntiles) issue(st, st);
  wait_tiles(min(NST - 2, ntiles - 1));
  block_barrier();

  // Iteration t of either loop: wait for tile t + 1 (tiles issued so far: 0 .. t + NST - 2),
  // barrier (tile t + 1 visible to every wave; every wave done with tile t - 1's stage), refill that
  // stage with tile t + NST - 1, issue the S^T MFMAs of tile t + 1, then tile t's softmax (VALU,
  // overlapping those MFMAs) and its O^T MFMAs. Unrolled by NST so every stage base is a constant.
  // Both loops pass the same barriers in the same order.
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  // `stages`: bit s set when this wave computes the tiles held in stage s (all of them, except for
  // the parts of a split light wave).
  // `act`: `active`, or std::true_type where the caller knows the wave is active (the full waves:
  // T - q0 > 16), so that no branch separates a tile's S^T MFMAs from the previous tile's softmax and
  // the scheduler can interleave them. The steps of the main loop never hold the last (ragged) key
  // tile, so their softmax has no masking branch either (`mask_c` false).
  using BF = std::false_type;
  using BT = std::true_type;
  auto pipeline = [&](auto& sa, auto& sb, auto&& scores, auto&& finish, auto stages, auto act)
                      __attribute__((always_inline)) {
    if (act && (stages & 1)) scores(sa, smem);
    auto step = [&](auto stage_c, int t, auto& cur, auto& nxt, auto last_c) __attribute__((always_inline)) {
      constexpr int SG = decltype(stage_c)::value;  // stage of tile t
      constexpr bool TAIL = decltype(last_c)::value;  // the step may hold the last tile
      if (!TAIL || t + 1 < ntiles) {
        wait_tiles(min(NST - 3, ntiles - 2 - t));
        block_barrier();
        if (t + NST - 1 < ntiles) issue((SG + NST - 1) % NST, t + NST - 1);
        if (act && ((stages >> ((SG + 1) % NST)) & 1)) scores(nxt, smem + ((SG + 1) % NST) * STAGE);
      }
      if (act && ((stages >> SG) & 1)) finish(cur, smem + SG * STAGE, t, last_c);
    };
    int t = 0;
    for (; t + NST < ntiles; t += NST) {
      step(I0{}, t, sa, sb, BF{});
      step(I1{}, t + 1, sb, sa, BF{});
      step(I2{}, t + 2, sa, sb, BF{});
      step(I3{}, t + 3, sb, sa, BF{});
    }
    if (t < ntiles) step(I0{}, t, sa, sb, BT{});
    if (t + 1 < ntiles) step(I1{}, t + 1, sb, sa, BT{});
    if (t + 2 < ntiles) step(I2{}, t + 2, sa, sb, BT{});
    if (t + 3 < ntiles) step(I3{}, t + 3, sb, sa, BT{});
  };

  if (full_wave) {
    // ---- Full wave: 32 queries on v_mfma_f32_32x32x16_bf16 (layout in the file comment). ----
    bf16x8_t qf[QK_STEPS];
#pragma unroll
    for (int ks = 0; ks < QK_STEPS; ++ks) qf[ks] = as_bf16x8(qraw[ks]);
    f32x16_t o[OB];
#pragma unroll
    for (int d = 0; d < OB; ++d)
#pragma unroll
      for (int v = 0; v < 16; ++v) o[d][v] = 0.0f;
    float m_i = -INFINITY, l_i = 0.0f;

    // Per-lane LDS offsets, fixed for the whole loop: the swizzle of a key row is the same for key
    // and key + 16 j (and key + 32 kb), so the k-step / key block / stage parts of every fragment
    // address are compile-time offsets.
    int koff[QK_STEPS];
#pragma unroll
    for (int kstep = 0; kstep < QK_STEPS; ++kstep) koff[kstep] = kv_slot(l32, kstep * 2 + g);
    int voff[OB][2];
    {
      const int sl = lane & 15, hh = (lane >> 4) & 1;
#pragma unroll
      for (int db = 0; db < OB; ++db) {
        const int dcol = 32 * db + 16 * hh + 4 * (sl & 3);  // first of the 4 dims this lane addresses
        const int k1 = 4 * g + (sl >> 2);                   // key of k-step 0 (first run)
        voff[db][0] = TILEB + kv_slot(k1, dcol >> 3) + ((dcol >> 2) & 1) * 8;
        voff[db][1] = TILEB + kv_slot(k1 + 8, dcol >> 3) + ((dcol >> 2) & 1) * 8;
      }
    }

    // S^T of one tile: s[kb][v] = S^T[key kb*32 + 8(v/4) + 4g + v%4][query l32].
    struct Scores {
      f32x16_t s[2];
    };
    auto scores = [&](Scores& sc, const unsigned char* st) __attribute__((always_inline)) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        bf16x8_t kf[QK_STEPS];
#pragma unroll
        for (int kstep = 0; kstep < QK_STEPS; ++kstep)
          kf[kstep] = as_bf16x8(*reinterpret_cast<const uint4*>(st + koff[kstep] + kb * 32 * 128));
        const f32x16_t zero = {};
        sc.s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[0], qf[0], zero, 0, 0, 0);
#pragma unroll
        for (int kstep = 1; kstep < QK_STEPS; ++kstep)
          sc.s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[kstep], qf[kstep], sc.s[kb], 0, 0, 0);
      }
    };
    // Online softmax of tile t and O^T += V^T . P^T with V from stage `st`.
    auto finish = [&](Scores& sc, const unsigned char* st, int t, auto mask_c) __attribute__((always_inline)) {
      f32x16_t (&s)[2] = sc.s;
      if (decltype(mask_c)::value && (tb + t + 1) * kKeyTile > N) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int v = 0; v < 16; ++v)
            if ((tb + t) * kKeyTile + kb * 32 + 8 * (v >> 2) + 4 * g + (v & 3) >= N) s[kb][v] = -INFINITY;
      }
      float mq[4];  // four short chains, combined as a tree
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        mq[q4] = s[q4 >> 1][8 * (q4 & 1)];
#pragma unroll
        for (int v = 1; v < 8; ++v) mq[q4] = fmaxf(mq[q4], s[q4 >> 1][8 * (q4 & 1) + v]);
      }
      const float mx = xor32_max(fmaxf(fmaxf(mq[0], mq[1]), fmaxf(mq[2], mq[3])));
      const float m_new = softmax_ref_max(m_i, mx, scale_log2);
      const float alpha = __builtin_amdgcn_exp2f((m_i - m_new) * scale_log2);
      const float mc = m_new * scale_log2;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int v = 0; v < 16; ++v) s[kb][v] = __builtin_amdgcn_exp2f(fmaf(s[kb][v], scale_log2, -mc));
      bf16x8_t pf[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float tmp[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) tmp[e] = s[j >> 1][8 * (j & 1) + e];
        pf[j] = pack_bf16x8(tmp);
      }
      const float rs = prob_row_sum(pf);
      l_i = l_i * alpha + rs;
      m_i = m_new;
      if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
#pragma unroll
        for (int d = 0; d < OB; ++d)
#pragma unroll
          for (int v = 0; v < 16; ++v) o[d][v] *= alpha;
      }
      // V^T fragment of d-block db, k-step j: elements 0..3 = keys 16j + 4g + {0..3}, elements 4..7 =
      // keys 16j + 8 + 4g + {0..3}, at dim 32 db + l32 (the P^T order above).
#pragma unroll
      for (int db = 0; db < OB; ++db) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) i16x4_t*)(st + voff[db][0] + j * 16 * 128));
          const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) i16x4_t*)(st + voff[db][1] + j * 16 * 128));
          typedef short i16x8_t __attribute__((ext_vector_type(8)));
          const i16x8_t both = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, both), pf[j], o[db], 0, 0, 0);
        }
      }
    };
    Scores sa, sb;
    if constexpr (FSPLIT > 1)
      pipeline(sa, sb, scores, finish, 0x5 << fpart, BT{});
    else
      pipeline(sa, sb, scores, finish, std::integral_constant<int, (1 << NST) - 1>{}, BT{});

    if (merged) {
      // Every wave has passed its last tile's reads after the first barrier, so the stages are free.
      // Full-wave parts park behind the light parts' area: m, l, o[2][16] for 64 lanes per wave.
      constexpr int LIGHT_AREA = (kLightParts - 1) * 18 * 64;
      constexpr int FSTRIDE = 34 * 64;
      float* fpark = reinterpret_cast<float*>(smem) + LIGHT_AREA + qwave * FSTRIDE;
      block_barrier();
      if (full_split > 1 && fpart == 1) {
        fpark[lane] = m_i;
        fpark[64 + lane] = l_i;
#pragma unroll
        for (int d = 0; d < OB; ++d)
#pragma unroll
          for (int v = 0; v < 16; ++v) fpark[(2 + 16 * d + v) * 64 + lane] = o[d][v];
      }
      block_barrier();
      if (full_split > 1 && fpart == 0) {
        const float m1 = fpark[lane], l1 = fpark[64 + lane];
        const float m = fmaxf(m_i, m1);  // part 0 holds tile 0: m is finite
        const float a0 = __builtin_amdgcn_exp2f((m_i - m) * scale_log2);
        const float a1 = __builtin_amdgcn_exp2f((m1 - m) * scale_log2);
        l_i = fmaf(l1, a1, l_i * a0);
        m_i = m;  // l_i and o are now relative to m (read by a key-part write)
#pragma unroll
        for (int d = 0; d < OB; ++d)
#pragma unroll
          for (int v = 0; v < 16; ++v) o[d][v] = fmaf(fpark[(2 + 16 * d + v) * 64 + lane], a1, o[d][v] * a0);
      }
    }
    const int qr = q0 + l32;
    if (KVS && active && qr < T && fpart == 0) {
      // This key part's unnormalised output, running max and sum (sq_attention_merge_kernel).
      float* ws = part_ws + ((int64_t)(b * (int)gridDim.y + h) * kv_parts + (int)blockIdx.x) * kv_part_stride(T);
      if (g == 0) {
        ws[qr] = m_i;
        ws[kv_part_rows(T) + qr] = l_i;
      }
      float* orow = ws + 2 * (int64_t)kv_part_rows(T) + (int64_t)qr * DH;
#pragma unroll
      for (int d = 0; d < OB; ++d)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4)
          *reinterpret_cast<f32x4_t*>(orow + d * 32 + 8 * r4 + 4 * g) =
              f32x4_t{o[d][4 * r4], o[d][4 * r4 + 1], o[d][4 * r4 + 2], o[d][4 * r4 + 3]};
    } else if (active && qr < T && fpart == 0) {
      const float inv = 1.0f / l_i;
      uint16_t* orow = out + ((int64_t)b * T + qr) * ors + (int64_t)h * DH;
#pragma unroll
      for (int d = 0; d < OB; ++d)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
          bf16x4_t w;
#pragma unroll
          for (int e = 0; e < 4; ++e) w[e] = (__bf16)(o[d][4 * r4 + e] * inv);
          *reinterpret_cast<bf16x4_t*>(orow + d * 32 + 8 * r4 + 4 * g) = w;
        }
    }
  } else {
    // ---- Light wave (<= 16 queries left, e.g. the 5 of T = 261 after 8 full waves): 16 queries on
    // v_mfma_f32_16x16x32_bf16, half the MFMA and softmax work of a full wave. 8 full waves and one
    // light wave would put three waves on one SIMD, which every other SIMD then waits for at each
    // tile's barrier; so, split (light_split), the light wave's keys are shared by kLightParts
    // waves, one per SIMD, part p taking a quarter of every tile (below). Each part keeps its
    // own running max, sum and output; parts 1.. park them in LDS after the loop and part 0 merges
    // them (rescaled to the largest reference max, summed in part order) and stores the rows.
    // Layout: lane l, 16-lane group G = l / 16. S^T = K . Q^T per 16-key block kb (A = K rows
    // 16 kb + l % 16, dims 32 ks + 8 G; B = Q^T, query l % 16): s16[kb][v] = S^T[key 16 kb + 4 G + v]
    // [query l % 16], so a query's 64 keys lie in the four groups (max / sum over xor 16, xor 32).
    // O^T = V^T . P^T per 16-dim block db and 32-key k-step j: group G supplies keys 32 j + 4 G +
    // {0..3} and 32 j + 16 + 4 G + {0..3} (P from s16[2j], s16[2j + 1]), and V^T is read in the same
    // order with the LDS transpose read (in each 16-lane group, lane i receives dim 16 db + i of 4
    // consecutive keys).
    const int l16 = lane & 15, G = lane >> 4;
    bf16x8_t qf[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) qf[ks] = as_bf16x8(qraw[ks]);
    f32x4_t o[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) o[d] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    float m_i = -INFINITY, l_i = 0.0f;
    int koff[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) koff[ks] = kv_slot(l16, 4 * ks + G);
    int voff[4][2];
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const int dcol = 16 * db + 4 * (l16 & 3);  // first of the 4 dims this lane addresses
      const int k1 = 4 * G + (l16 >> 2);         // key of k-step 0 (first run)
      voff[db][0] = TILEB + kv_slot(k1, dcol >> 3) + ((dcol >> 2) & 1) * 8;
      voff[db][1] = TILEB + kv_slot(k1 + 16, dcol >> 3) + ((dcol >> 2) & 1) * 8;
    }
    struct Scores16 {
      f32x4_t s[4];
    };
    auto scores = [&](Scores16& sc, const unsigned char* st) __attribute__((always_inline)) {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        const bf16x8_t k0 = as_bf16x8(*reinterpret_cast<const uint4*>(st + koff[0] + kb * 16 * 128));
        const bf16x8_t k1 = as_bf16x8(*reinterpret_cast<const uint4*>(st + koff[1] + kb * 16 * 128));
        const f32x4_t zero = {};
        sc.s[kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k0, qf[0], zero, 0, 0, 0);
        sc.s[kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k1, qf[1], sc.s[kb], 0, 0, 0);
      }
    };
    auto finish = [&](Scores16& sc, const unsigned char* st, int t, auto mask_c) __attribute__((always_inline)) {
      f32x4_t (&s)[4] = sc.s;
      if (decltype(mask_c)::value && (tb + t + 1) * kKeyTile > N) {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int v = 0; v < 4; ++v)
            if ((tb + t) * kKeyTile + 16 * kb + 4 * G + v >= N) s[kb][v] = -INFINITY;
      }
      float mq[4];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) mq[kb] = fmaxf(fmaxf(s[kb][0], s[kb][1]), fmaxf(s[kb][2], s[kb][3]));
      float mx = fmaxf(fmaxf(mq[0], mq[1]), fmaxf(mq[2], mq[3]));
      mx = xor32_max(xor16_max(mx));
      const float m_new = softmax_ref_max(m_i, mx, scale_log2);
      const float alpha = __builtin_amdgcn_exp2f((m_i - m_new) * scale_log2);
      const float mc = m_new * scale_log2;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int v = 0; v < 4; ++v) s[kb][v] = __builtin_amdgcn_exp2f(fmaf(s[kb][v], scale_log2, -mc));
      bf16x8_t pf[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const float tmp[8] = {s[2 * j][0], s[2 * j][1], s[2 * j][2], s[2 * j][3],
                              s[2 * j + 1][0], s[2 * j + 1][1], s[2 * j + 1][2], s[2 * j + 1][3]};
        pf[j] = pack_bf16x8(tmp);
      }
      typedef __bf16 bf16x2v_t __attribute__((ext_vector_type(2)));
      const bf16x2v_t ones = {(__bf16)1.0f, (__bf16)1.0f};
      float r[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        r[j] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(pf[j], pf[j], 0, 1), ones, 0.0f, false);
        r[j] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(pf[j], pf[j], 2, 3), ones, r[j], false);
        r[j] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(pf[j], pf[j], 4, 5), ones, r[j], false);
        r[j] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(pf[j], pf[j], 6, 7), ones, r[j], false);
      }
      const float rs = xor32_sum(xor16_sum(r[0] + r[1]));
      l_i = l_i * alpha + rs;
      m_i = m_new;
      if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
#pragma unroll
        for (int d = 0; d < 4; ++d) o[d] *= alpha;
      }
#pragma unroll
      for (int db = 0; db < 4; ++db) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) i16x4_t*)(st + voff[db][0] + j * 32 * 128));
          const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) i16x4_t*)(st + voff[db][1] + j * 32 * 128));
          typedef short i16x8_t __attribute__((ext_vector_type(8)));
          const i16x8_t both = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          o[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, both), pf[j], o[db], 0, 0, 0);
        }
      }
    };
    using AllStages = std::integral_constant<int, (1 << NST) - 1>;
    if (lpart >= 0) {
      // Split light wave: part p takes keys 16 p .. 16 p + 15 of every tile, so every SIMD gets the
      // same share of the light work at every step. S^T of the slice is one 16-key block (A = K rows
      // 16 p + l % 16): sq.s[v] = S^T[key 16 p + 4 G + v][query l % 16]. O^T += V^T . P^T on
      // v_mfma_f32_16x16x16_bf16 per 16-dim block db: B = P^T in that same layout (keys 16 p + 4 G +
      // {0..3} of query l % 16), A = V^T from one transpose read (dim 16 db + l % 16 of those keys).
      static_assert(kLightParts * 16 == kKeyTile, "one 16-key slice per light part");
      const int pofs = lpart * 16 * 128;
      int kq[2], vq[4];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) kq[ks] = koff[ks] + pofs;
#pragma unroll
      for (int db = 0; db < 4; ++db) vq[db] = voff[db][0] + pofs;
      struct ScoresQ {
        f32x4_t s;
      };
      auto scores_q = [&](ScoresQ& sc, const unsigned char* st) __attribute__((always_inline)) {
        const bf16x8_t k0 = as_bf16x8(*reinterpret_cast<const uint4*>(st + kq[0]));
        const bf16x8_t k1 = as_bf16x8(*reinterpret_cast<const uint4*>(st + kq[1]));
        const f32x4_t zero = {};
        sc.s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k0, qf[0], zero, 0, 0, 0);
        sc.s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k1, qf[1], sc.s, 0, 0, 0);
      };
      auto finish_q = [&](ScoresQ& sc, const unsigned char* st, int t, auto mask_c) __attribute__((always_inline)) {
        f32x4_t& sv = sc.s;
        const int key0 = (tb + t) * kKeyTile + 16 * lpart;  // first key of the slice
        if (decltype(mask_c)::value && key0 + 16 > N) {
          if (key0 >= N) return;  // no key in the slice: the part's running state stays as it is
#pragma unroll
          for (int v = 0; v < 4; ++v)
            if (key0 + 4 * G + v >= N) sv[v] = -INFINITY;
        }
        const float mx = xor32_max(xor16_max(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]))));
        const float m_new = softmax_ref_max(m_i, mx, scale_log2);
        const float alpha = __builtin_amdgcn_exp2f((m_i - m_new) * scale_log2);
        const float mc = m_new * scale_log2;
#pragma unroll
        for (int v = 0; v < 4; ++v) sv[v] = __builtin_amdgcn_exp2f(fmaf(sv[v], scale_log2, -mc));
        typedef __bf16 bf16x4v_t __attribute__((ext_vector_type(4)));
        const bf16x4v_t pb = __builtin_convertvector(sv, bf16x4v_t);
        typedef __bf16 bf16x2v_t __attribute__((ext_vector_type(2)));
        const bf16x2v_t ones = {(__bf16)1.0f, (__bf16)1.0f};
        float r = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(pb, pb, 0, 1), ones, 0.0f, false);
        r = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(pb, pb, 2, 3), ones, r, false);
        l_i = l_i * alpha + xor32_sum(xor16_sum(r));
        m_i = m_new;
        if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
#pragma unroll
          for (int d = 0; d < 4; ++d) o[d] *= alpha;
        }
        const i16x4_t pbits = __builtin_bit_cast(i16x4_t, pb);
#pragma unroll
        for (int db = 0; db < 4; ++db) {
          const i16x4_t vt = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) i16x4_t*)(st + vq[db]));
          o[db] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(vt, pbits, o[db], 0, 0, 0);
        }
      };
      ScoresQ qa, qb;
      pipeline(qa, qb, scores_q, finish_q, AllStages{}, active);
    } else {
      Scores16 sa, sb;
      pipeline(sa, sb, scores, finish, AllStages{}, active);
    }

    if (merged) {
      // Every wave has passed its last tile's reads after the first barrier, so the stages are free.
      constexpr int PSTRIDE = 18 * 64;  // floats per part: m, l, o[4][4] for 64 lanes
      float* park = reinterpret_cast<float*>(smem);
      block_barrier();
      if (light_split && lpart > 0) {
        float* pp = park + (lpart - 1) * PSTRIDE;
        pp[lane] = m_i;
        pp[64 + lane] = l_i;
#pragma unroll
        for (int d = 0; d < 4; ++d)
#pragma unroll
          for (int e = 0; e < 4; ++e) pp[(2 + 4 * d + e) * 64 + lane] = o[d][e];
      }
      block_barrier();
      if (light_split && lpart == 0) {
        float mp[kLightParts], lp[kLightParts];
        mp[0] = m_i;
        lp[0] = l_i;
#pragma unroll
        for (int p = 1; p < kLightParts; ++p) {
          mp[p] = park[(p - 1) * PSTRIDE + lane];
          lp[p] = park[(p - 1) * PSTRIDE + 64 + lane];
        }
        float m = mp[0];
#pragma unroll
        for (int p = 1; p < kLightParts; ++p) m = fmaxf(m, mp[p]);
        // Part 0 holds key 0 of the first tile, so m is finite; a part whose slices held no key has
        // m = -inf, l = 0, o = 0.
        float a[kLightParts];
#pragma unroll
        for (int p = 0; p < kLightParts; ++p) a[p] = __builtin_amdgcn_exp2f((mp[p] - m) * scale_log2);
        l_i = lp[0] * a[0];
#pragma unroll
        for (int p = 1; p < kLightParts; ++p) l_i = fmaf(lp[p], a[p], l_i);
        m_i = m;  // l_i and o are now relative to m (read by a key-part write)
#pragma unroll
        for (int d = 0; d < 4; ++d)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float v = o[d][e] * a[0];
#pragma unroll
            for (int p = 1; p < kLightParts; ++p) v = fmaf(park[(p - 1) * PSTRIDE + (2 + 4 * d + e) * 64 + lane], a[p], v);
            o[d][e] = v;
          }
      }
    }

    // O^T[16 db + 4 G + v][query l16]: 4 consecutive dims per lane and block.
    const int qr = q0 + l16;
    if (KVS && active && qr < T && lpart <= 0) {
      float* ws = part_ws + ((int64_t)(b * (int)gridDim.y + h) * kv_parts + (int)blockIdx.x) * kv_part_stride(T);
      if (G == 0) {
        ws[qr] = m_i;
        ws[kv_part_rows(T) + qr] = l_i;
      }
      float* orow = ws + 2 * (int64_t)kv_part_rows(T) + (int64_t)qr * DH;
#pragma unroll
      for (int d = 0; d < 4; ++d) *reinterpret_cast<f32x4_t*>(orow + 16 * d + 4 * G) = o[d];
    } else if (active && qr < T && lpart <= 0) {
      const float inv = 1.0f / l_i;
      uint16_t* orow = out + ((int64_t)b * T + qr) * ors + (int64_t)h * DH;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
        bf16x4_t w;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = (__bf16)(o[d][e] * inv);
        *reinterpret_cast<bf16x4_t*>(orow + 16 * d + 4 * G) = w;
      }
    }
  }
}

static constexpr int kAttnStages = 4;
static constexpr int kNumCus = 256;     // MI355X
static constexpr int kMaxKvParts = 8;
static constexpr int kMinTilesSaved = 8;

// Merge of the key parts of a split launch. Per (row, head) part p left its running (reference) max
// m_p, its sum l_p and its unnormalised output o_p, both relative to m_p; with m = max_p m_p and
// a_p = 2^((m_p - m) * scale_log2): l = sum_p a_p l_p, out = bf16((sum_p a_p o_p) * (1 / l)), summed
// in part order. Every part holds at least one key, so every m_p is finite. Thread = (row, head, 8 dims).
template <int P>
__global__ __launch_bounds__(256) void sq_attention_merge_kernel(const float* __restrict__ ws, int B, int T, int H,
                                                                 float scale_log2, uint16_t* __restrict__ out,
                                                                 int64_t ors) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)B * T * H * 8) return;
  const int c = (int)(i & 7);
  const int64_t rh = i >> 3;
  const int h = (int)(rh % H);
  const int64_t row = rh / H;  // b * T + query
  const int b = (int)(row / T), qr = (int)(row - (int64_t)b * T);
  const int64_t pstride = kv_part_stride(T);
  const int64_t tp = kv_part_rows(T);
  const float* base = ws + (int64_t)(b * H + h) * P * pstride;
  // Every load first (one round of memory latency), then the arithmetic.
  float mp[P], lp[P];
  f32x4_t x0[P], x1[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const float* pb = base + p * pstride;
    mp[p] = pb[qr];
    lp[p] = pb[tp + qr];
    const f32x4_t* src = reinterpret_cast<const f32x4_t*>(pb + 2 * tp + (int64_t)qr * 64 + 8 * c);
    x0[p] = src[0];
    x1[p] = src[1];
  }
  float m = mp[0];
#pragma unroll
  for (int p = 1; p < P; ++p) m = fmaxf(m, mp[p]);
  float l = 0.0f, o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = 0.0f;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const float a = __builtin_amdgcn_exp2f((mp[p] - m) * scale_log2);
    l = fmaf(lp[p], a, l);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      o[e] = fmaf(x0[p][e], a, o[e]);
      o[4 + e] = fmaf(x1[p][e], a, o[4 + e]);
    }
  }
  const float inv = 1.0f / l;
  typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
  bf16x4_t w0, w1;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    w0[e] = (__bf16)(o[e] * inv);
    w1[e] = (__bf16)(o[4 + e] * inv);
  }
  uint16_t* orow = out + row * ors + (int64_t)h * 64 + 8 * c;
  *reinterpret_cast<bf16x4_t*>(orow) = w0;
  *reinterpret_cast<bf16x4_t*>(orow + 4) = w1;
}

// Two waves per full query wave (the buffer-load kernel's full_split) when a single workgroup per
// (image, head) would otherwise have fewer than 8 waves, as long as the split still has the 8 loader
// waves, fits the workgroup and leaves room for the parked partials (4 full waves at most).
static int full_split_for(int64_t n_wg, int64_t nfq, int light_parts) {
  if (n_wg != 1 || nfq > 4) return 1;
  const int64_t waves = 2 * nfq + light_parts;
  return (waves >= 8 && waves <= kDmaMaxWaves && nfq + (light_parts ? 1 : 0) < 8) ? 2 : 1;
}

}  // namespace oudjat

using namespace oudjat;

// Launch shape of a sparse_query_attention call: query workgroups per (image, head), waves per
// workgroup, and for the buffer-load kernel its light split, full split and key parts.
struct AttnShape {
  int64_t n_wg;
  int w;
  bool dma;
  int split, nfq, fsplit, kv_parts;
};

static AttnShape attn_shape(int64_t B, int64_t T, int64_t H, int64_t Dh, int64_t N, bool offsets_fit) {
  AttnShape s{};
  const int64_t waves = cdiv(T, 32);
  s.n_wg = cdiv(waves, Dh == 64 ? kMaxWaves64 : kMaxWaves128);
  s.w = (int)cdiv(waves, s.n_wg);
  if (s.w < kMinWaves) s.w = kMinWaves;
  // Buffer-load kernel for Dh = 64 with >= 8 waves, counting the waves of split full and light
  // query waves (its byte offsets must fit 31 bits); the register-staged kernel otherwise.
  const int w = s.w;
  const bool small_split = s.n_wg == 1 && w < 8 && full_split_for(s.n_wg, (T - (w - 1) * 32 <= 16) ? w - 1 : w,
                                                                 (T - (w - 1) * 32 <= 16) ? kLightParts : 0) > 1;
  s.dma = Dh == 64 && (w >= 8 || small_split) && offsets_fit;
  s.kv_parts = 1;
  if (!s.dma) return s;
  // One workgroup per (image, head) whose last query wave is light (1..16 queries): that wave is
  // split over kLightParts waves (its merge area, 3 parts of 18 x 64 floats, fits the stages).
  const int64_t last = T - (w - 1) * 32;
  s.split = (s.n_wg == 1 && last >= 1 && last <= 16 && w - 1 + kLightParts <= kDmaMaxWaves) ? kLightParts : 0;
  s.nfq = s.split ? w - 1 : w;
  s.fsplit = full_split_for(s.n_wg, s.nfq, s.split);
  // Key parts: with one workgroup per (image, head) and fewer than half as many (image, head) pairs
  // as CUs, the key tiles are dealt to up to kMaxKvParts workgroups per pair in contiguous ranges
  // (as many as one round of workgroups on the CUs holds), and a merge launch combines them.
  const int64_t pairs = B * H;
  const int64_t ntiles = cdiv(N, kKeyTile);
  if (s.n_wg == 1 && 2 * pairs <= kNumCus) {
    int64_t parts = std::min<int64_t>(std::min<int64_t>(kNumCus / pairs, ntiles), kMaxKvParts);
    const int64_t per = cdiv(ntiles, parts);
    parts = cdiv(ntiles, per);
    // Worth it only when each workgroup is spared at least kMinTilesSaved key tiles (~1 us each),
    // against the merge launch (~3-5 us).
    if (parts >= 2 && ntiles - per >= kMinTilesSaved) s.kv_parts = (int)parts;
  }
  return s;
}

// fp32 elements of the key-part workspace: per (image, head, part) the running max and sum of each
// query and its unnormalised output row.
static int64_t attn_workspace_elems(int64_t B, int64_t T, int64_t H, int kv_parts) {
  return kv_parts > 1 ? B * H * kv_parts * kv_part_stride(T) : 0;
}

static int sparse_query_attention_impl(const uint16_t* q, int64_t qrs, int64_t B, int64_t T, int64_t H, int64_t Dh,
                                       const uint16_t* kv, int64_t kvb, int64_t kvn, int64_t kvkv, int64_t kvh,
                                       int64_t N, float scale, uint16_t* out, int64_t ors, float* workspace,
                                       int64_t workspace_elems, float* lse, oudjat_stream_t stream) {
  OUDJAT_REQUIRE(B >= 0 && T >= 0 && H >= 0 && N >= 0, OUDJAT_ERR_INVALID_ARGUMENT,
                 "sparse_query_attention: negative size");
  if (B == 0 || T == 0 || H == 0) return OUDJAT_OK;
  OUDJAT_REQUIRE(q && kv && out, OUDJAT_ERR_INVALID_ARGUMENT, "sparse_query_attention: null pointer");
  OUDJAT_REQUIRE(N > 0, OUDJAT_ERR_UNSUPPORTED_SHAPE, "sparse_query_attention: no keys");
  OUDJAT_REQUIRE(Dh == 64 || Dh == 128, OUDJAT_ERR_UNSUPPORTED_SHAPE, "sparse_query_attention: Dh=%lld (64 or 128)",
                 (long long)Dh);
  OUDJAT_REQUIRE(qrs % 8 == 0 && kvb % 8 == 0 && kvn % 8 == 0 && kvkv % 8 == 0 && kvh % 8 == 0 && ors % 4 == 0 &&
                     aligned(q, 16) && aligned(kv, 16) && aligned(out, 8),
                 OUDJAT_ERR_UNSUPPORTED_LAYOUT, "sparse_query_attention: 16-byte aligned q and kv rows required");
  OUDJAT_REQUIRE(B <= 65535 && H <= 65535, OUDJAT_ERR_TOO_LARGE, "sparse_query_attention: grid too large");
  OUDJAT_REQUIRE(N < ((int64_t)1 << 30) && T < ((int64_t)1 << 30), OUDJAT_ERR_TOO_LARGE,
                 "sparse_query_attention: N or T too large");
  const float scale_log2 = scale * 1.4426950408889634f;
  const AttnShape s = attn_shape(B, T, H, Dh, N, N * kvn * 2 < ((int64_t)1 << 31));
  const int w = s.w;
  dim3 grid((unsigned)s.n_wg, (unsigned)H, (unsigned)B);
  hipStream_t st = as_stream(stream);
  if (lse) {
    // The register-staged kernel with the row log-sum-exp (at Dh = 128 the kernel every call runs;
    // at Dh = 64 its output equals the buffer-load kernel's on every row of a full query wave).
    OUDJAT_REQUIRE(aligned(lse, 4), OUDJAT_ERR_UNSUPPORTED_LAYOUT, "sparse_query_attention: lse alignment");
    const size_t lds = 2 * 2 * (size_t)kKeyTile * Dh * 2;
    if (Dh == 128)
      sq_attention_kernel<128, kMinWaves, false, true><<<grid, w * 64, lds, st>>>(
          q, qrs, (int)T, kv, kvb, kvn, kvkv, kvh, (int)N, scale_log2, out, ors, w, lse);
    else if (w >= 8)
      sq_attention_kernel<64, 8, true, true><<<grid, w * 64, lds, st>>>(q, qrs, (int)T, kv, kvb, kvn, kvkv, kvh,
                                                                      (int)N, scale_log2, out, ors, w, lse);
    else
      sq_attention_kernel<64, kMinWaves, false, true><<<grid, w * 64, lds, st>>>(
          q, qrs, (int)T, kv, kvb, kvn, kvkv, kvh, (int)N, scale_log2, out, ors, w, lse);
    return check_launch("sparse_query_attention (lse)");
  }
  if (s.dma) {
    const size_t lds_dma = (size_t)kAttnStages * 2 * kKeyTile * 128;
    static_assert((size_t)kAttnStages * 2 * kKeyTile * 128 <= 64 * 1024, "needs no larger-LDS attribute");
    static_assert((kLightParts - 1) * 18 * 64 * 4 <= kAttnStages * 2 * kKeyTile * 128, "merge area");
    static_assert(((kLightParts - 1) * 18 + 4 * 34) * 64 * 4 <= kAttnStages * 2 * kKeyTile * 128,
                  "merge area of the light parts and of four split full waves");
    const int threads = (s.nfq * s.fsplit + (s.split ? kLightParts : 0)) * 64;
    const int split = s.split;
    const bool kvs = s.kv_parts > 1 && workspace && aligned(workspace, 16) &&
                     attn_workspace_elems(B, T, H, s.kv_parts) <= workspace_elems;
    if (kvs) {
      dim3 pgrid((unsigned)s.kv_parts, (unsigned)H, (unsigned)B);
      if (s.fsplit > 1)
        sq_attention_dma_kernel<kAttnStages, 2, true><<<pgrid, threads, lds_dma, st>>>(
            q, qrs, (int)T, kv, kvb, kvn, kvkv, kvh, (int)N, scale_log2, out, ors, w, split, workspace, s.kv_parts);
      else
        sq_attention_dma_kernel<kAttnStages, 1, true><<<pgrid, threads, lds_dma, st>>>(
            q, qrs, (int)T, kv, kvb, kvn, kvkv, kvh, (int)N, scale_log2, out, ors, w, split, workspace, s.kv_parts);
      const int rc = check_launch("sparse_query_attention");
      if (rc != OUDJAT_OK) return rc;
      const unsigned mgrid = (unsigned)cdiv(B * T * H * 8, 256);
      switch (s.kv_parts) {
#define OUDJAT_MERGE(PV)                                                                                     \
  case PV:                                                                                                    \
    sq_attention_merge_kernel<PV><<<mgrid, 256, 0, st>>>(workspace, (int)B, (int)T, (int)H, scale_log2, out, ors); \
    break;
        OUDJAT_MERGE(2)
        OUDJAT_MERGE(3)
        OUDJAT_MERGE(4)
        OUDJAT_MERGE(5)
        OUDJAT_MERGE(6)
        OUDJAT_MERGE(7)
        OUDJAT_MERGE(8)
#undef OUDJAT_MERGE
        default:
          return set_error(OUDJAT_ERR_INVALID_ARGUMENT, "sparse_query_attention: %d key parts", s.kv_parts);
      }
      return check_launch("sparse_query_attention (merge)");
    }
    if (s.fsplit > 1)
      sq_attention_dma_kernel<kAttnStages, 2, false><<<grid, threads, lds_dma, st>>>(q, qrs, (int)T, kv, kvb, kvn, kvkv,
                                                                                      kvh, (int)N, scale_log2, out, ors,
                                                                                      w, split, nullptr, 1);
    else
      sq_attention_dma_kernel<kAttnStages, 1, false><<<grid, threads, lds_dma, st>>>(q, qrs, (int)T, kv, kvb, kvn, kvkv,
                                                                                      kvh, (int)N, scale_log2, out, ors,
                                                                                      w, split, nullptr, 1);
    return check_launch("sparse_query_attention");
  }
  // Two stages of one K and one V tile (64 keys x Dh bf16 each): 32 KB at Dh = 64, 64 KB at
  // Dh = 128, within the default dynamic LDS limit.
  const size_t lds = 2 * 2 * (size_t)kKeyTile * Dh * 2;
  if (Dh == 128)
    sq_attention_kernel<128, kMinWaves, false><<<grid, w * 64, lds, st>>>(q, qrs, (int)T, kv, kvb, kvn, kvkv, kvh,
                                                                          (int)N, scale_log2, out, ors, w, nullptr);
  else if (w >= 8)
    sq_attention_kernel<64, 8, true><<<grid, w * 64, lds, st>>>(q, qrs, (int)T, kv, kvb, kvn, kvkv, kvh, (int)N,
                                                                scale_log2, out, ors, w, nullptr);
  else
    sq_attention_kernel<64, kMinWaves, false><<<grid, w * 64, lds, st>>>(q, qrs, (int)T, kv, kvb, kvn, kvkv, kvh,
                                                                         (int)N, scale_log2, out, ors, w, nullptr);
  return check_launch("sparse_query_attention");
}

extern "C" int oudjat_sparse_query_attention(const uint16_t* q, int64_t qrs, int64_t B, int64_t T, int64_t H,
                                             int64_t Dh, const uint16_t* kv, int64_t kvb, int64_t kvn, int64_t kvkv,
                                             int64_t kvh, int64_t N, float scale, uint16_t* out, int64_t ors,
                                             oudjat_stream_t stream) {
  return sparse_query_attention_impl(q, qrs, B, T, H, Dh, kv, kvb, kvn, kvkv, kvh, N, scale, out, ors, nullptr, 0,
                                     nullptr, stream);
}

extern "C" int oudjat_sparse_query_attention_ws(const uint16_t* q, int64_t qrs, int64_t B, int64_t T, int64_t H,
                                                int64_t Dh, const uint16_t* kv, int64_t kvb, int64_t kvn,
                                                int64_t kvkv, int64_t kvh, int64_t N, float scale, uint16_t* out,
                                                int64_t ors, float* workspace, int64_t workspace_elems,
                                                oudjat_stream_t stream) {
  OUDJAT_REQUIRE(workspace_elems >= 0, OUDJAT_ERR_INVALID_ARGUMENT, "sparse_query_attention: negative workspace size");
  return sparse_query_attention_impl(q, qrs, B, T, H, Dh, kv, kvb, kvn, kvkv, kvh, N, scale, out, ors, workspace,
                                     workspace_elems, nullptr, stream);
}

extern "C" int oudjat_sparse_query_attention_lse(const uint16_t* q, int64_t qrs, int64_t B, int64_t T, int64_t H,
                                                 int64_t Dh, const uint16_t* kv, int64_t kvb, int64_t kvn,
                                                 int64_t kvkv, int64_t kvh, int64_t N, float scale, uint16_t* out,
                                                 int64_t ors, float* lse, oudjat_stream_t stream) {
  OUDJAT_REQUIRE(lse != nullptr || B == 0 || T == 0 || H == 0, OUDJAT_ERR_INVALID_ARGUMENT,
                 "sparse_query_attention: null lse");
  return sparse_query_attention_impl(q, qrs, B, T, H, Dh, kv, kvb, kvn, kvkv, kvh, N, scale, out, ors, nullptr, 0,
                                     lse, stream);
}

extern "C" int oudjat_sparse_query_attention_fp8(const uint16_t* q, int64_t qrs, int64_t B, int64_t T, int64_t H,
                                                 int64_t Dh, const uint16_t* kv, int64_t kvb, int64_t kvn,
                                                 int64_t kvkv, int64_t kvh, int64_t N, float scale,
                                                 const float* act_inv_scale, uint8_t* out, int64_t ors,
                                                 oudjat_stream_t stream) {
  OUDJAT_REQUIRE(B >= 0 && T >= 0 && H >= 0 && N >= 0, OUDJAT_ERR_INVALID_ARGUMENT,
                 "sparse_query_attention_fp8: negative size");
  if (B == 0 || T == 0 || H == 0) return OUDJAT_OK;
  OUDJAT_REQUIRE(q && kv && out && act_inv_scale, OUDJAT_ERR_INVALID_ARGUMENT,
                 "sparse_query_attention_fp8: null pointer");
  OUDJAT_REQUIRE(N > 0, OUDJAT_ERR_UNSUPPORTED_SHAPE, "sparse_query_attention_fp8: no keys");
  OUDJAT_REQUIRE(Dh == 128, OUDJAT_ERR_UNSUPPORTED_SHAPE, "sparse_query_attention_fp8: Dh=%lld (128 only)",
                 (long long)Dh);
  OUDJAT_REQUIRE(qrs % 8 == 0 && kvb % 8 == 0 && kvn % 8 == 0 && kvkv % 8 == 0 && kvh % 8 == 0 && ors % 4 == 0 &&
                     aligned(q, 16) && aligned(kv, 16) && aligned(out, 4) && aligned(act_inv_scale, 4),
                 OUDJAT_ERR_UNSUPPORTED_LAYOUT, "sparse_query_attention_fp8: 16-byte aligned q and kv rows, "
                 "4-byte aligned output rows required");
  OUDJAT_REQUIRE(B <= 65535 && H <= 65535 && N < ((int64_t)1 << 30) && T < ((int64_t)1 << 30), OUDJAT_ERR_TOO_LARGE,
                 "sparse_query_attention_fp8: too large");
  const AttnShape s = attn_shape(B, T, H, Dh, N, true);
  dim3 grid((unsigned)s.n_wg, (unsigned)H, (unsigned)B);
  const size_t lds = 2 * 2 * (size_t)kKeyTile * Dh * 2;
  sq_attention_kernel<128, kMinWaves, false, false, true><<<grid, s.w * 64, lds, as_stream(stream)>>>(
      q, qrs, (int)T, kv, kvb, kvn, kvkv, kvh, (int)N, scale * 1.4426950408889634f, nullptr, ors, s.w, nullptr, out,
      act_inv_scale);
  return check_launch("sparse_query_attention_fp8");
}

extern "C" int64_t oudjat_sparse_query_attention_workspace_elems(int64_t B, int64_t T, int64_t H, int64_t Dh,
                                                                 int64_t N) {
  if (B <= 0 || T <= 0 || H <= 0 || N <= 0 || Dh != 64 || B > 65535 || H > 65535 || N >= ((int64_t)1 << 30) ||
      T >= ((int64_t)1 << 30))
    return 0;
  const AttnShape s = attn_shape(B, T, H, Dh, N, true);
  return s.dma ? attn_workspace_elems(B, T, H, s.kv_parts) : 0;
}
