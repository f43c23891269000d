// Pixel-residual importance and image-residual token pruning: the server side of the importance
// producer.
//
// patch_residual_score: per ph x pw patch of HWC images, the residual d = curr - prev (fp32; prev may
// be absent when the input already is a residual) scored as sqrt(mean(d^2)) ("rms"), sum(d^2)
// ("energy") or sqrt(sum(d^2)) ("l2"). Each square is rounded to fp32 (the materialised square of the reference); the sum is
// taken in float64 in a fixed order (exact for 8- and 16-bit integer pixels), then rounded once. One
// workgroup per (patch row, image); one thread per (patch, pixel row) pair, reading that row's pw * C
// contiguous values.
//
// residual_prune_keep / residual_prune_compact: keep a candidate patch when its residual RMS reaches the
// threshold or it is among the min_keep largest (ties to the lower candidate index, NaN largest, as
// the top-k plan), count and sum the kept / all residuals, then compact the kept candidates into the
// pruned dindice at the host-chosen width.
#include <atomic>
#include <cmath>

#include "common.hpp"
#include "select.hpp"

namespace oudjat {

static constexpr int kResThreads = 256;
static constexpr int64_t kMaxResPairs = 8192;  // gw * ph partial sums of float64 in LDS (64 KiB)
static constexpr int64_t kMaxPruneCandidates = 16384;

template <typename T>
__device__ __forceinline__ float load_px(const T* p, int64_t i) {
  return (float)p[i];
}

template <typename T>
__global__ __launch_bounds__(kResThreads) void patch_residual_score_kernel(const T* __restrict__ curr,
                                                                           const T* __restrict__ prev,
                                                                           const int64_t* __restrict__ img_idx,
                                                                           int64_t n_images, int H, int W, int C,
                                                                           int ph, int pw, int mode,
                                                                           float* __restrict__ out) {
  extern __shared__ double part[];
  const int gi = blockIdx.x;
  const int bo = blockIdx.y;
  const int gw = W / pw, gh = H / ph;
  const int64_t b = img_idx ? img_idx[bo] : bo;
  float* o = out + (int64_t)bo * gh * gw + (int64_t)gi * gw;
  if (b < 0 || b >= n_images) {  // an image index outside the batch scores NaN
    for (int j = threadIdx.x; j < gw; j += kResThreads) o[j] = __int_as_float(0x7fc00000);
    return;
  }
  const int span = pw * C;
  const int pairs = gw * ph;
  for (int idx = threadIdx.x; idx < pairs; idx += kResThreads) {
    const int j = idx / ph, r = idx - j * ph;
    const int64_t base = ((b * H + (int64_t)gi * ph + r) * W + (int64_t)j * pw) * C;
    double acc = 0.0;
    for (int e = 0; e < span; ++e) {
      float d = load_px(curr, base + e);
      if (prev) d = d - load_px(prev, base + e);
      const float sq = d * d;
      acc += (double)sq;
    }
    part[idx] = acc;
  }
  __syncthreads();
  const double n = (double)ph * pw * C;
  for (int j = threadIdx.x; j < gw; j += kResThreads) {
    double t = 0.0;
    for (int r = 0; r < ph; ++r) t += part[j * ph + r];
    float v;
    if (mode == 1) {          // energy: sum d^2
      v = (float)t;
    } else if (mode == 2) {   // rms: sqrt(mean d^2), correctly rounded fp32 square root of the fp32 mean
      const float mean = (float)(t / n);
      v = (float)sqrt((double)mean);
    } else {                  // l2: sqrt(sum d^2)
      v = (float)sqrt((double)(float)t);
    }
    o[j] = v;
  }
}

__device__ __forceinline__ double block_sum_f64(double v, double* sh) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  if (lane == 0) sh[w] = v;
  __syncthreads();
  double t = 0.0;
  for (int i = 0; i < kPlanWaves; ++i) t += sh[i];
  __syncthreads();
  return t;
}

__global__ __launch_bounds__(kPlanThreads) void residual_prune_keep_kernel(
    const float* __restrict__ rms, int64_t rsb, int G, const int64_t* __restrict__ spatial, int64_t ssb, int P,
    float thres, int min_keep, uint8_t* __restrict__ keep, int32_t* __restrict__ count_out,
    float* __restrict__ kept_mass, float* __restrict__ full_mass) {
  extern __shared__ uint32_t keys[];
  __shared__ uint32_t hist[256];
  __shared__ uint32_t scan_sh[kPlanWaves];
  __shared__ uint32_t sel_sh[2];
  __shared__ double red_sh[kPlanWaves];

  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t* sp = spatial + (int64_t)b * ssb;
  const float* r = rms + (int64_t)b * rsb;
  auto value = [&](int i) -> float {
    const int64_t s = sp[i];
    return (s >= 0 && s < G) ? r[s] : __int_as_float(0x7fc00000);
  };
  for (int i = tid; i < P; i += kPlanThreads) keys[i] = order_key(value(i));
  __syncthreads();

  const int k = min(min_keep, P);
  const bool top_all = k >= P;
  const bool top_none = k <= 0;
  uint32_t thr = 0u, remaining = (uint32_t)max(k, 0);
  if (!top_all && !top_none) thr = radix_select_kth(keys, P, remaining, hist, sel_sh, &remaining);

  const int per = (P + kPlanThreads - 1) / kPlanThreads;
  const int beg = min(tid * per, P);
  const int end = min(beg + per, P);
  uint32_t n_eq = 0u;
  if (!top_all && !top_none)
    for (int i = beg; i < end; ++i) n_eq += keys[i] == thr;
  uint32_t eq_rank = block_excl_scan(n_eq, scan_sh);

  uint32_t n_kept = 0u;
  double kept = 0.0, full = 0.0;
  for (int i = beg; i < end; ++i) {
    const uint32_t key = keys[i];
    bool top;
    if (top_all) top = true;
    else if (top_none) top = false;
    else {
      top = key > thr;
      if (key == thr) {
        top = eq_rank < remaining;
        ++eq_rank;
      }
    }
    const float v = value(i);
    const bool kp = top || v >= thres;
    keep[(int64_t)b * P + i] = kp ? 1 : 0;
    n_kept += kp;
    full += (double)v;
    kept += (double)(v * (kp ? 1.0f : 0.0f));
  }
  const double tot_full = block_sum_f64(full, red_sh);
  const double tot_kept = block_sum_f64(kept, red_sh);
  const double tot_n = block_sum_f64((double)n_kept, red_sh);
  if (tid == 0) {
    count_out[b] = (int32_t)tot_n;
    full_mass[b] = (float)tot_full;
    kept_mass[b] = (float)tot_kept;
  }
}

__global__ __launch_bounds__(kPlanThreads) void residual_prune_compact_kernel(
    const uint8_t* __restrict__ keep, int P, const int64_t* __restrict__ spatial, int64_t ssb,
    const int64_t* __restrict__ dind, int64_t dsb, int npre, int W, int64_t* __restrict__ pruned,
    int64_t* __restrict__ local_idx) {
  __shared__ uint32_t scan_sh[kPlanWaves];
  __shared__ uint32_t count_sh;
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const uint8_t* kp = keep + (int64_t)b * P;
  const int per = (P + kPlanThreads - 1) / kPlanThreads;
  const int beg = min(tid * per, P);
  const int end = min(beg + per, P);
  uint32_t n = 0u;
  for (int i = beg; i < end; ++i) n += kp[i] != 0;
  uint32_t pos = block_excl_scan(n, scan_sh);
  if (tid == kPlanThreads - 1) count_sh = pos + n;
  __syncthreads();
  const int count = (int)count_sh;
  const int T = npre + W;
  int64_t* out = pruned + (int64_t)b * T;
  int64_t* li = local_idx + (int64_t)b * W;
  for (int i = beg; i < end; ++i) {
    if (!kp[i]) continue;
    const int rnk = (int)pos++;
    if (rnk >= W) continue;
    out[npre + rnk] = spatial[(int64_t)b * ssb + i] + npre;
    li[rnk] = i;
  }
  for (int j = min(count, W) + tid; j < W; j += kPlanThreads) {
    out[npre + j] = npre;  // a zero spatial index, shifted past the pretokens
    li[j] = 0;
  }
  for (int j = tid; j < npre; j += kPlanThreads) out[j] = dind[(int64_t)b * dsb + j];
}

template <typename K>
int raise_lds_limit(K kernel, const char* what) {
  static std::atomic<uint8_t> attr_set[64];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(OUDJAT_ERR_HIP, "%s: hipGetDevice: %s", what, hipGetErrorString(e));
  if (!attr_set[dev & 63].load(std::memory_order_acquire)) {
    e = hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, 64 * 1024);
    if (e != hipSuccess) return set_error(OUDJAT_ERR_HIP, "%s: hipFuncSetAttribute: %s", what, hipGetErrorString(e));
    attr_set[dev & 63].store(1, std::memory_order_release);
  }
  return OUDJAT_OK;
}

template <typename T>
int launch_residual_score(const void* curr, const void* prev, const int64_t* image_idx, int64_t n_images, int64_t H,
                          int64_t W, int64_t C, int64_t ph, int64_t pw, int mode, float* out, dim3 grid, size_t lds,
                          oudjat_stream_t stream) {
  if (lds > 48 * 1024) {
    const int rc = raise_lds_limit(patch_residual_score_kernel<T>, "patch_residual_score");
    if (rc != OUDJAT_OK) return rc;
  }
  patch_residual_score_kernel<T><<<grid, kResThreads, lds, as_stream(stream)>>>(
      (const T*)curr, (const T*)prev, image_idx, n_images, (int)H, (int)W, (int)C, (int)ph, (int)pw, mode, out);
  return OUDJAT_OK;
}

}  // namespace oudjat

using namespace oudjat;

extern "C" int oudjat_patch_residual_score(const void* curr, const void* prev, int dtype, int64_t n_images,
                                           const int64_t* image_idx, int64_t n_out, int64_t H, int64_t W, int64_t C,
                                           int64_t ph, int64_t pw, int mode, float* out, oudjat_stream_t stream) {
  OUDJAT_REQUIRE(n_images >= 0 && n_out >= 0 && H >= 0 && W >= 0 && C > 0 && ph > 0 && pw > 0,
                 OUDJAT_ERR_INVALID_ARGUMENT, "patch_residual_score: bad size");
  OUDJAT_REQUIRE(dtype >= 0 && dtype <= 2, OUDJAT_ERR_INVALID_ARGUMENT, "patch_residual_score: dtype %d", dtype);
  OUDJAT_REQUIRE(mode >= 0 && mode <= 2, OUDJAT_ERR_INVALID_ARGUMENT, "patch_residual_score: mode %d", mode);
  OUDJAT_REQUIRE(H % ph == 0 && W % pw == 0, OUDJAT_ERR_UNSUPPORTED_LAYOUT,
                 "patch_residual_score: image %lldx%lld not divisible by patch %lldx%lld", (long long)H, (long long)W,
                 (long long)ph, (long long)pw);
  OUDJAT_REQUIRE(image_idx || n_out <= n_images, OUDJAT_ERR_INVALID_ARGUMENT,
                 "patch_residual_score: %lld outputs from %lld images without an index list", (long long)n_out,
                 (long long)n_images);
  const int64_t gh = H / ph, gw = W / pw;
  if (n_out == 0 || gh == 0 || gw == 0) return OUDJAT_OK;
  OUDJAT_REQUIRE(curr && out, OUDJAT_ERR_INVALID_ARGUMENT, "patch_residual_score: null pointer");
  OUDJAT_REQUIRE(gw * ph <= kMaxResPairs && gh < 65536 && n_out < 65536 && pw * C < (1 << 20), OUDJAT_ERR_TOO_LARGE,
                 "patch_residual_score: too large");
  const size_t lds = (size_t)(gw * ph) * sizeof(double);
  const dim3 grid((unsigned)gh, (unsigned)n_out);
  int rc;
  if (dtype == 0)
    rc = launch_residual_score<uint8_t>(curr, prev, image_idx, n_images, H, W, C, ph, pw, mode, out, grid, lds, stream);
  else if (dtype == 1)
    rc = launch_residual_score<int16_t>(curr, prev, image_idx, n_images, H, W, C, ph, pw, mode, out, grid, lds, stream);
  else
    rc = launch_residual_score<float>(curr, prev, image_idx, n_images, H, W, C, ph, pw, mode, out, grid, lds, stream);
  if (rc != OUDJAT_OK) return rc;
  return check_launch("patch_residual_score");
}

extern "C" int oudjat_residual_prune_keep(const float* rms, int64_t B, int64_t rms_stride_b, int64_t G,
                                          const int64_t* spatial, int64_t spatial_stride_b, int64_t P, float thres,
                                          int64_t min_keep, uint8_t* keep, int32_t* kept_count, float* kept_mass,
                                          float* full_mass, oudjat_stream_t stream) {
  OUDJAT_REQUIRE(B >= 0 && P >= 0 && G >= 0 && min_keep >= 0, OUDJAT_ERR_INVALID_ARGUMENT,
                 "residual_prune_keep: negative size");
  if (B == 0) return OUDJAT_OK;
  OUDJAT_REQUIRE(kept_count && kept_mass && full_mass && (P == 0 || (rms && spatial && keep)),
                 OUDJAT_ERR_INVALID_ARGUMENT, "residual_prune_keep: null pointer");
  OUDJAT_REQUIRE(P <= kMaxPruneCandidates, OUDJAT_ERR_TOO_LARGE, "residual_prune_keep: P=%lld exceeds %lld",
                 (long long)P, (long long)kMaxPruneCandidates);
  OUDJAT_REQUIRE(rms_stride_b >= G && spatial_stride_b >= P && G < ((int64_t)1 << 31), OUDJAT_ERR_UNSUPPORTED_LAYOUT,
                 "residual_prune_keep: row strides");
  const size_t lds = (size_t)P * 4;
  if (lds > 48 * 1024) {
    const int rc = raise_lds_limit(residual_prune_keep_kernel, "residual_prune_keep");
    if (rc != OUDJAT_OK) return rc;
  }
  residual_prune_keep_kernel<<<(unsigned)B, kPlanThreads, lds, as_stream(stream)>>>(
      rms, rms_stride_b, (int)G, spatial, spatial_stride_b, (int)P, thres, (int)std::min<int64_t>(min_keep, P), keep,
      kept_count, kept_mass, full_mass);
  return check_launch("residual_prune_keep");
}

extern "C" int oudjat_residual_prune_compact(const uint8_t* keep, int64_t B, int64_t P, const int64_t* spatial,
                                             int64_t spatial_stride_b, const int64_t* dindice, int64_t dindice_stride_b,
                                             int64_t num_pre, int64_t width, int64_t* pruned_dindice,
                                             int64_t* kept_local_idx, oudjat_stream_t stream) {
  OUDJAT_REQUIRE(B >= 0 && P >= 0 && num_pre >= 0 && width >= 0 && width <= P, OUDJAT_ERR_INVALID_ARGUMENT,
                 "residual_prune_compact: bad size");
  if (B == 0) return OUDJAT_OK;
  OUDJAT_REQUIRE(pruned_dindice && dindice && (width == 0 || kept_local_idx) && (P == 0 || (keep && spatial)),
                 OUDJAT_ERR_INVALID_ARGUMENT, "residual_prune_compact: null pointer");
  OUDJAT_REQUIRE(P <= kMaxPruneCandidates && B < ((int64_t)1 << 31), OUDJAT_ERR_TOO_LARGE,
                 "residual_prune_compact: too large");
  OUDJAT_REQUIRE(spatial_stride_b >= P && dindice_stride_b >= num_pre, OUDJAT_ERR_UNSUPPORTED_LAYOUT,
                 "residual_prune_compact: row strides");
  residual_prune_compact_kernel<<<(unsigned)B, kPlanThreads, 0, as_stream(stream)>>>(
      keep, (int)P, spatial, spatial_stride_b, dindice, dindice_stride_b, (int)num_pre, (int)width, pruned_dindice,
      kept_local_idx);
  return check_launch("residual_prune_compact");
}
