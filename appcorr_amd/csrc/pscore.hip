// Server patch scores of the approximate pass (the cache producer of the correction path):
//   cls_attn_prob / patch_pseudo_attn_prob   one query per (image, head), softmax over all keys,
//                                             mean over heads (attention.py:254-271)
//   the pseudo query of patch_pseudo_attn_prob (attention.py:254-259)
//
// The reference evaluates these with eager torch ops on bf16 tensors, so every op's output is a
// bf16 rounding of an fp32 computation. These kernels reproduce those rounding points and evaluate
// each fp32 accumulation exactly (float64 partial sums of exact fp32 products, one rounding to fp32)
// and each exponential in float64 (one rounding to fp32): the correctly rounded value of every step,
// independent of the reduction order, hence deterministic and equal bit for bit to the CPU restatement.
#include <mutex>

#include "common.hpp"

namespace oudjat {
namespace {

// Correctly rounded fp32 division and square root of fp32 operands, evaluated in float64 and rounded
// once: float64 carries more than 2 * 24 + 2 bits, so the double rounding cannot differ from a direct
// one (and the result does not depend on how the compiler lowers fp32 division and sqrt).
__device__ __forceinline__ float div_rn(float a, float b) { return (float)((double)a / (double)b); }
__device__ __forceinline__ float sqrt_rn(float a) { return (float)sqrt((double)a); }

constexpr int kPsThreads = 256;
constexpr int kPsMaxKeys = 8192;  // LDS row of fp32 scores per (image, head)

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Sum over the `width` lanes of an aligned lane group (width a power of two <= 64).
__device__ __forceinline__ double group_sum_f64(double v, int width) {
  for (int o = width >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Block-wide reductions over kPsThreads threads; `red` holds one slot per wave.
__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float m = red[0];
#pragma unroll
  for (int i = 1; i < kPsThreads / 64; ++i) m = fmaxf(m, red[i]);
  return m;
}
__device__ __forceinline__ double block_sum_f64(double v, double* red) {
  v = wave_sum_f64(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  double s = 0.0;
#pragma unroll
  for (int i = 0; i < kPsThreads / 64; ++i) s += red[i];  // fixed order
  return s;
}

// Exact dot product piece: 8 bf16 x 8 bf16, each product exact in fp32, summed in float64.
__device__ __forceinline__ double dot8_f64(const float* a, const uint4& kv) {
  float b[8];
  unpack8(kv, b);
  double s = 0.0;
#pragma unroll
  for (int e = 0; e < 8; ++e) s += (double)(a[e] * b[e]);
  return s;
}

// One workgroup per (head h, image b): p[n] = bf16(e_n / sum e), e_n = exp(s_n - max s),
// s_n = bf16(bf16(q . k_n) * scale), written as fp32 to ws[(b * H + h) * N + n].
// L = Dh / 8 lanes share one key row (16 bytes each).
template <int L>
__global__ void __launch_bounds__(kPsThreads) query_prob_kernel(const uint16_t* __restrict__ q, int64_t q_sb,
                                                                int64_t q_sh, const uint16_t* __restrict__ k,
                                                                int64_t k_sb, int64_t k_sn, int64_t k_sh, int N,
                                                                int H, float scale, float* __restrict__ ws) {
  __shared__ float srow[kPsMaxKeys];
  __shared__ float red_f[kPsThreads / 64];
  __shared__ double red_d[kPsThreads / 64];
  const int h = blockIdx.x, b = blockIdx.y;
  const int lane_in_key = threadIdx.x % L;
  const int key_slot = threadIdx.x / L;
  constexpr int kKeysPerIter = kPsThreads / L;

  float qa[8];
  unpack8(*reinterpret_cast<const uint4*>(q + b * q_sb + h * q_sh + lane_in_key * 8), qa);
  const uint16_t* kb = k + b * k_sb + h * k_sh + lane_in_key * 8;
  // kUnroll key rows per thread group in flight before their dot products (each sum is exact, so the
  // grouping changes no bit).
  constexpr int kUnroll = 8;
  for (int n0 = 0; n0 < N; n0 += kKeysPerIter * kUnroll) {
    uint4 kr[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int n = n0 + u * kKeysPerIter + key_slot;
      kr[u] = make_uint4(0, 0, 0, 0);
      if (n < N) kr[u] = *reinterpret_cast<const uint4*>(kb + (int64_t)n * k_sn);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int n = n0 + u * kKeysPerIter + key_slot;
      const double dot = group_sum_f64(dot8_f64(qa, kr[u]), L);
      if (n < N && lane_in_key == 0) srow[n] = round_bf16(round_bf16((float)dot) * scale);
    }
  }
  __syncthreads();
  float m = -INFINITY;
  for (int n = threadIdx.x; n < N; n += kPsThreads) m = fmaxf(m, srow[n]);
  m = block_max(m, red_f);
  double part = 0.0;
  for (int n = threadIdx.x; n < N; n += kPsThreads) {
    const float e = (float)exp((double)(srow[n] - m));
    srow[n] = e;
    part += (double)e;
  }
  const float tot = (float)block_sum_f64(part, red_d);
  float* out = ws + ((int64_t)b * H + h) * N;
  for (int n = threadIdx.x; n < N; n += kPsThreads) out[n] = round_bf16(div_rn(srow[n], tot));
}

// out[b, n] = bf16(fl(sum_h p[b, h, n]) * factor), summed exactly in float64.
__global__ void __launch_bounds__(kPsThreads) head_mean_kernel(const float* __restrict__ ws, int B, int H, int N,
                                                               float factor, void* __restrict__ out,
                                                               int64_t out_sb, int out_bf16) {
  const int64_t i = (int64_t)blockIdx.x * kPsThreads + threadIdx.x;
  if (i >= (int64_t)B * N) return;
  const int b = (int)(i / N), n = (int)(i % N);
  const float* p = ws + (int64_t)b * H * N + n;
  double s = 0.0;
  for (int h = 0; h < H; ++h) s += (double)p[(int64_t)h * N];
  const uint32_t bits = f32_to_bf16((float)s * factor);
  if (out_bf16)
    reinterpret_cast<uint16_t*>(out)[b * out_sb + n] = (uint16_t)bits;
  else
    reinterpret_cast<float*>(out)[b * out_sb + n] = __uint_as_float(bits << 16);
}

// The pseudo query of one (head h, image b) from its P patch queries (rows t = 0..P-1 at q_st):
//   q_mean = bf16(fl(sum_t q_t) * fl(1/P));  qmn = max(bf16(sqrt(fl(|q_mean|^2))), 2^-7)
//   target = bf16(fl(sum_t bf16(sqrt(fl(|q_t|^2)))) * fl(1/P));  out = bf16(q_mean * bf16(target / qmn))
template <int L>
__global__ void __launch_bounds__(kPsThreads) pseudo_query_kernel(const uint16_t* __restrict__ q, int64_t q_sb,
                                                                  int64_t q_st, int64_t q_sh, int P,
                                                                  float inv_p, uint16_t* __restrict__ out) {
  constexpr int kGroups = kPsThreads / L;  // token rows per iteration
  constexpr int kDh = 8 * L;
  __shared__ double dsum[kGroups][kDh];
  __shared__ double nsum[kGroups];
  __shared__ double red_d[kPsThreads / 64];
  __shared__ float qmean[kDh];
  const int h = blockIdx.x, b = blockIdx.y, H = gridDim.x;
  const int lane_in_row = threadIdx.x % L;
  const int group = threadIdx.x / L;
  const uint16_t* qb = q + b * q_sb + h * q_sh + lane_in_row * 8;
  double acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  double norm_acc = 0.0;
  for (int t0 = 0; t0 < P; t0 += kGroups) {
    const int t = t0 + group;
    double sq = 0.0;
    if (t < P) {
      float v[8];
      unpack8(*reinterpret_cast<const uint4*>(qb + (int64_t)t * q_st), v);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        acc[e] += (double)v[e];
        sq += (double)(v[e] * v[e]);
      }
    }
    sq = group_sum_f64(sq, L);
    if (t < P && lane_in_row == 0) norm_acc += (double)round_bf16(sqrt_rn((float)sq));
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) dsum[group][lane_in_row * 8 + e] = acc[e];
  if (lane_in_row == 0) nsum[group] = norm_acc;
  __syncthreads();
  double sq = 0.0;
  if (threadIdx.x < kDh) {
    double s = 0.0;
    for (int g = 0; g < kGroups; ++g) s += dsum[g][threadIdx.x];  // fixed order, exact
    const float qm = round_bf16((float)s * inv_p);
    qmean[threadIdx.x] = qm;
    sq = (double)(qm * qm);
  }
  const double qsq = block_sum_f64(sq, red_d);
  if (threadIdx.x < kDh) {
    double ns = 0.0;  // the head's norm sum, read by every output thread in the same fixed order
    for (int g = 0; g < kGroups; ++g) ns += nsum[g];
    const float qmn = fmaxf(round_bf16(sqrt_rn((float)qsq)), 0.0078125f);
    const float target = round_bf16((float)ns * inv_p);
    const float ratio = round_bf16(div_rn(target, qmn));
    out[((int64_t)b * H + h) * kDh + threadIdx.x] = (uint16_t)f32_to_bf16(qmean[threadIdx.x] * ratio);
  }
}

}  // namespace

// Workspace of oudjat_query_attention_prob_noalloc: the per-head probabilities of one call, B*H*N fp32.
// Each GPU the library runs on holds its own copy until the process ends; host code must use the
// address hipGetSymbolAddress returns for the current device, never the array's name.
constexpr int64_t kNoAllocMaxElems = OUDJAT_QUERY_PROB_NOALLOC_MAX;  // 4 MiB of fp32
static __device__ __align__(256) float scratch[kNoAllocMaxElems];

static std::once_flag g_scratch_once[64];
static float* g_scratch_ptr[64];
static hipError_t g_scratch_err[64];

// The current device's address of `scratch`, looked up once per device (at library init by
// oudjat_selftest, else at the first no-alloc call on that device).
int noalloc_scratch(float** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(OUDJAT_ERR_HIP, "noalloc scratch: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= 64) return set_error(OUDJAT_ERR_HIP, "noalloc scratch: device index %d out of range", dev);
  std::call_once(g_scratch_once[dev], [dev] {
    void* p = nullptr;
    g_scratch_err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_scratch_ptr[dev] = static_cast<float*>(p);
  });
  if (g_scratch_err[dev] != hipSuccess || g_scratch_ptr[dev] == nullptr)
    return set_error(OUDJAT_ERR_HIP, "noalloc scratch: hipGetSymbolAddress: %s", hipGetErrorString(g_scratch_err[dev]));
  if (out) *out = g_scratch_ptr[dev];
  return OUDJAT_OK;
}

}  // namespace oudjat

using namespace oudjat;

extern "C" int oudjat_query_attention_prob(const uint16_t* q, int64_t q_stride_b, int64_t q_stride_h, int64_t B,
                                           int64_t H, int64_t Dh, const uint16_t* k, int64_t k_stride_b,
                                           int64_t k_stride_n, int64_t k_stride_h, int64_t N, float scale,
                                           float* workspace, void* out, int64_t out_stride_b, int out_bf16,
                                           oudjat_stream_t stream) {
  OUDJAT_REQUIRE(q && k && workspace && out, OUDJAT_ERR_INVALID_ARGUMENT, "query_attention_prob: null pointer");
  OUDJAT_REQUIRE(B >= 0 && H > 0 && N > 0, OUDJAT_ERR_INVALID_ARGUMENT, "query_attention_prob: bad sizes");
  OUDJAT_REQUIRE(Dh == 64 || Dh == 128, OUDJAT_ERR_UNSUPPORTED_SHAPE, "query_attention_prob: Dh %lld not in {64, 128}",
                 (long long)Dh);
  OUDJAT_REQUIRE(N <= kPsMaxKeys, OUDJAT_ERR_TOO_LARGE, "query_attention_prob: N %lld > %d", (long long)N, kPsMaxKeys);
  OUDJAT_REQUIRE(B <= 65535 && H <= 65535 && B * N < (1ll << 31), OUDJAT_ERR_TOO_LARGE,
                 "query_attention_prob: grid too large");
  OUDJAT_REQUIRE(aligned(q, 16) && aligned(k, 16) && q_stride_b % 8 == 0 && q_stride_h % 8 == 0 &&
                     k_stride_b % 8 == 0 && k_stride_n % 8 == 0 && k_stride_h % 8 == 0,
                 OUDJAT_ERR_UNSUPPORTED_LAYOUT, "query_attention_prob: q/k rows must be 16-byte aligned");
  if (B == 0) return OUDJAT_OK;
  hipStream_t s = as_stream(stream);
  const dim3 grid((unsigned)H, (unsigned)B);
  if (Dh == 64)
    query_prob_kernel<8><<<grid, kPsThreads, 0, s>>>(q, q_stride_b, q_stride_h, k, k_stride_b, k_stride_n,
                                                     k_stride_h, (int)N, (int)H, scale, workspace);
  else
    query_prob_kernel<16><<<grid, kPsThreads, 0, s>>>(q, q_stride_b, q_stride_h, k, k_stride_b, k_stride_n,
                                                      k_stride_h, (int)N, (int)H, scale, workspace);
  int st = check_launch("query_attention_prob");
  if (st != OUDJAT_OK) return st;
  const float factor = 1.0f / (float)H;
  head_mean_kernel<<<(unsigned)cdiv(B * N, kPsThreads), kPsThreads, 0, s>>>(workspace, (int)B, (int)H, (int)N,
                                                                           factor, out, out_stride_b, out_bf16);
  return check_launch("query_attention_prob(head mean)");
}

extern "C" int oudjat_pseudo_query(const uint16_t* q, int64_t q_stride_b, int64_t q_stride_t, int64_t q_stride_h,
                                   int64_t B, int64_t P, int64_t H, int64_t Dh, uint16_t* out,
                                   oudjat_stream_t stream) {
  OUDJAT_REQUIRE(q && out, OUDJAT_ERR_INVALID_ARGUMENT, "pseudo_query: null pointer");
  OUDJAT_REQUIRE(B >= 0 && P > 0 && H > 0, OUDJAT_ERR_INVALID_ARGUMENT, "pseudo_query: bad sizes");
  OUDJAT_REQUIRE(Dh == 64 || Dh == 128, OUDJAT_ERR_UNSUPPORTED_SHAPE, "pseudo_query: Dh %lld not in {64, 128}",
                 (long long)Dh);
  OUDJAT_REQUIRE(B <= 65535 && H <= 65535 && P < (1 << 24), OUDJAT_ERR_TOO_LARGE, "pseudo_query: too large");
  OUDJAT_REQUIRE(aligned(q, 16) && aligned(out, 16) && q_stride_b % 8 == 0 && q_stride_t % 8 == 0 &&
                     q_stride_h % 8 == 0,
                 OUDJAT_ERR_UNSUPPORTED_LAYOUT, "pseudo_query: q rows must be 16-byte aligned");
  if (B == 0) return OUDJAT_OK;
  hipStream_t s = as_stream(stream);
  const dim3 grid((unsigned)H, (unsigned)B);
  const float inv_p = 1.0f / (float)P;
  if (Dh == 64)
    pseudo_query_kernel<8><<<grid, kPsThreads, 0, s>>>(q, q_stride_b, q_stride_t, q_stride_h, (int)P, inv_p, out);
  else
    pseudo_query_kernel<16><<<grid, kPsThreads, 0, s>>>(q, q_stride_b, q_stride_t, q_stride_h, (int)P, inv_p, out);
  return check_launch("pseudo_query");
}

// oudjat_query_attention_prob with the library's own device array as the workspace (no allocation;
// calls on one GPU share the array, so calls that overlap in time on one GPU race). The array needs
// no clearing: the first kernel writes every one of the B*H*N entries the second reads.
extern "C" int oudjat_query_attention_prob_noalloc(const uint16_t* q, int64_t q_stride_b, int64_t q_stride_h,
                                                   int64_t B, int64_t H, int64_t Dh, const uint16_t* k,
                                                   int64_t k_stride_b, int64_t k_stride_n, int64_t k_stride_h,
                                                   int64_t N, float scale, void* out, int64_t out_stride_b,
                                                   int out_bf16, oudjat_stream_t stream) {
  OUDJAT_REQUIRE(B >= 0 && H > 0 && N > 0 && B <= 65535 && H <= 65535 && N <= kPsMaxKeys,
                 OUDJAT_ERR_INVALID_ARGUMENT, "query_attention_prob_noalloc: bad sizes");
  OUDJAT_REQUIRE(B * H * N <= kNoAllocMaxElems, OUDJAT_ERR_TOO_LARGE,
                 "query_attention_prob_noalloc: B*H*N = %lld exceeds the %lld-element scratch array",
                 (long long)(B * H * N), (long long)kNoAllocMaxElems);
  float* ws = nullptr;
  const int st = noalloc_scratch(&ws);
  if (st != OUDJAT_OK) return st;
  return oudjat_query_attention_prob(q, q_stride_b, q_stride_h, B, H, Dh, k, k_stride_b, k_stride_n, k_stride_h, N,
                                     scale, ws, out, out_stride_b, out_bf16, stream);
}
