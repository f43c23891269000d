// Top-k token selection and the sync-free packed query plan.
//
// One 1024-thread workgroup per image. The scores of the image are turned into order-preserving
// uint32 keys in LDS; a 4-round radix select (8-bit digits, LDS histograms) finds the k-th largest
// key; kept candidates are then compacted in ascending candidate order with two block-wide prefix
// sums (equal-to-threshold rank, then kept rank). Ties on the threshold key go to the lowest
// candidate index, which makes the selected set a pure function of the scores.
//
// The same workgroup writes the whole PackedQueryState of its image (update_indice, batch/pos/token
// index, patch mask, RoPE table row) and, if asked, the per-token slot map that the fused
// reconstruct kernel uses. Nothing here needs the host: k is a launch argument.
//
// Threshold selection (score >= threshold) has its own kernels below: the kept mask and count, and the
// plan at a fixed width, built with the same candidate-order compaction.
#include <atomic>

#include "common.hpp"
#include "select.hpp"

namespace oudjat {

static constexpr int64_t kMaxCandidates = 16384;
static constexpr int64_t kMaxPlanLds = 144 * 1024;

__global__ __launch_bounds__(kPlanThreads) void topk_plan_kernel(
    const float* __restrict__ scores, int P, int64_t ssb, int k, const int64_t* __restrict__ dind, int64_t dsb,
    int npre, int ntok, int64_t* __restrict__ upd, int64_t* __restrict__ abat, int64_t* __restrict__ apos,
    int64_t* __restrict__ atok, uint8_t* __restrict__ pmask, int64_t* __restrict__ ridx, uint8_t* __restrict__ keep,
    int32_t* __restrict__ slot_map) {
  extern __shared__ uint32_t smem[];
  uint32_t* keys = smem;
  int32_t* lmap = reinterpret_cast<int32_t*>(smem + P);
  __shared__ uint32_t hist[256];
  __shared__ uint32_t scan_sh[kPlanWaves];
  __shared__ uint32_t sel_sh[2];

  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const float* s = scores + (int64_t)b * ssb;
  const int64_t* d = dind + (int64_t)b * dsb;
  const int T = npre + k;
  const int64_t row0 = (int64_t)b * T;

  for (int i = tid; i < P; i += kPlanThreads) keys[i] = order_key(s[i]);
  if (slot_map)
    for (int i = tid; i < ntok; i += kPlanThreads) lmap[i] = -1;
  __syncthreads();

  const bool keep_all = k >= P;
  const bool keep_none = k <= 0;
  uint32_t thr = 0u;
  uint32_t remaining = (uint32_t)(k > 0 ? k : 0);
  if (!keep_all && !keep_none) thr = radix_select_kth(keys, P, remaining, hist, sel_sh, &remaining);

  // Each thread owns a contiguous run of candidates, so thread order is candidate order.
  const int per = (P + kPlanThreads - 1) / kPlanThreads;
  const int beg = min(tid * per, P);
  const int end = min(beg + per, P);

  uint32_t n_eq = 0u;
  if (!keep_all && !keep_none)
    for (int i = beg; i < end; ++i) n_eq += keys[i] == thr;
  uint32_t eq_rank = block_excl_scan(n_eq, scan_sh);

  uint32_t kept_bits = 0u;  // bit (i - beg) set if candidate i is kept; per <= 16
  uint32_t n_kept = 0u;
  for (int i = beg; i < end; ++i) {
    bool kept;
    if (keep_all) kept = true;
    else if (keep_none) kept = false;
    else {
      const uint32_t key = keys[i];
      kept = key > thr;
      if (key == thr) {
        kept = eq_rank < remaining;
        ++eq_rank;
      }
    }
    if (kept) {
      kept_bits |= 1u << (i - beg);
      ++n_kept;
    }
  }
  uint32_t pos = block_excl_scan(n_kept, scan_sh);

  for (int i = beg; i < end; ++i) {
    const bool kept = (kept_bits >> (i - beg)) & 1u;
    if (keep) keep[(int64_t)b * P + i] = kept ? 1 : 0;
    if (!kept) continue;
    const int slot = npre + (int)pos;
    ++pos;
    const int64_t tok = d[npre + i];
    const int64_t r = row0 + slot;
    upd[r] = tok;
    abat[r] = b;
    apos[r] = slot;
    atok[r] = tok;
    pmask[r] = tok >= npre ? 1 : 0;
    ridx[r] = tok > npre ? tok - npre : 0;
    if (slot_map && tok >= 0 && tok < ntok) lmap[tok] = (int32_t)r;
  }
  for (int j = tid; j < npre; j += kPlanThreads) {
    const int64_t tok = d[j];
    const int64_t r = row0 + j;
    upd[r] = tok;
    abat[r] = b;
    apos[r] = j;
    atok[r] = tok;
    pmask[r] = tok >= npre ? 1 : 0;
    ridx[r] = tok > npre ? tok - npre : 0;
    if (slot_map && tok >= 0 && tok < ntok) lmap[tok] = (int32_t)r;
  }
  if (slot_map) {
    __syncthreads();
    for (int i = tid; i < ntok; i += kPlanThreads) slot_map[(int64_t)b * ntok + i] = lmap[i];
  }
}

// Threshold selection: keep[b, p] = scores[b, p] >= thres, compared in fp32 (NaN never kept), and the
// per-image kept count. One 256-thread workgroup per image.
static constexpr int kKeepThreads = 256;

__global__ __launch_bounds__(kKeepThreads) void threshold_keep_kernel(const float* __restrict__ scores, int P,
                                                                      int64_t ssb, float thres,
                                                                      uint8_t* __restrict__ keep,
                                                                      int32_t* __restrict__ count_out) {
  __shared__ uint32_t part[kKeepThreads / 64];
  const int b = blockIdx.x, tid = threadIdx.x;
  const float* s = scores + (int64_t)b * ssb;
  uint32_t n = 0;
  for (int i = tid; i < P; i += kKeepThreads) {
    const bool k = s[i] >= thres;
    n += k;
    if (keep) keep[(int64_t)b * P + i] = k ? 1 : 0;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) n += __shfl_xor(n, o, 64);
  if ((tid & 63) == 0) part[tid >> 6] = n;
  __syncthreads();
  if (tid == 0) {
    uint32_t t = 0;
    for (int w = 0; w < kKeepThreads / 64; ++w) t += part[w];
    count_out[b] = (int32_t)t;
  }
}

// Threshold selection and its packed plan at a fixed width of W patch slots (T = npre + W rows per
// image). One 1024-thread workgroup per image; each thread owns a contiguous run of candidates, so a
// block-wide prefix sum over the per-thread kept counts ranks the kept candidates in candidate order
// (the row-major order of nonzero()). Kept rank r < W goes to slot npre + r. Slots past the kept
// count are filled by `fill`:
//   0 (fixed width): the image's last kept candidate, candidate 0 if it keeps none; every slot valid.
//   1 (padded): update_indice holds token 0 and query_valid is 0; the packed rows repeat the image's
//     last valid row (last kept candidate, else its last pretoken), so that the duplicated row
//     computes and writes back exactly what the valid row does.
// row_slot maps each token to the first slot that holds it (atomicMin in LDS), so it is a pure
// function of the inputs even where slots repeat a token.
__global__ __launch_bounds__(kPlanThreads) void threshold_plan_kernel(
    const float* __restrict__ scores, int P, int64_t ssb, float thres, int W, int fill,
    const int64_t* __restrict__ dind, int64_t dsb, int npre, int ntok, int64_t* __restrict__ upd,
    int64_t* __restrict__ abat, int64_t* __restrict__ apos, int64_t* __restrict__ atok, uint8_t* __restrict__ pmask,
    int64_t* __restrict__ ridx, uint8_t* __restrict__ qvalid, uint8_t* __restrict__ keep,
    int32_t* __restrict__ count_out, int32_t* __restrict__ slot_map) {
  extern __shared__ int32_t lmap[];
  __shared__ uint32_t scan_sh[kPlanWaves];
  __shared__ int32_t info_sh[2];  // kept count, last kept candidate (0 if none)

  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const float* s = scores + (int64_t)b * ssb;
  const int64_t* d = dind + (int64_t)b * dsb;
  const int T = npre + W;
  const int64_t row0 = (int64_t)b * T;

  if (slot_map)
    for (int i = tid; i < ntok; i += kPlanThreads) lmap[i] = 0x7fffffff;
  if (tid == 0) {
    info_sh[0] = 0;
    info_sh[1] = 0;
  }

  const int per = (P + kPlanThreads - 1) / kPlanThreads;
  const int beg = min(tid * per, P);
  const int end = min(beg + per, P);
  uint32_t bits = 0u, n = 0u;  // per <= 16
  int last_i = -1;
  for (int i = beg; i < end; ++i) {
    if (s[i] >= thres) {
      bits |= 1u << (i - beg);
      ++n;
      last_i = i;
    }
  }
  uint32_t pos = block_excl_scan(n, scan_sh);  // its barriers also publish the LDS initialisation
  if (tid == kPlanThreads - 1) info_sh[0] = (int32_t)(pos + n);
  if (last_i >= 0) atomicMax(&info_sh[1], last_i);
  __syncthreads();
  const int count = info_sh[0];
  const int last = info_sh[1];

  if (tid == 0) count_out[b] = count;
  for (int i = beg; i < end; ++i) {
    const bool kept = (bits >> (i - beg)) & 1u;
    if (keep) keep[(int64_t)b * P + i] = kept ? 1 : 0;
    if (!kept) continue;
    const int r = (int)pos;
    ++pos;
    if (r >= W) continue;
    const int slot = npre + r;
    const int64_t tok = d[npre + i];
    const int64_t row = row0 + slot;
    upd[row] = tok;
    abat[row] = b;
    apos[row] = slot;
    atok[row] = tok;
    pmask[row] = tok >= npre ? 1 : 0;
    ridx[row] = tok > npre ? tok - npre : 0;
    qvalid[row] = 1;
    if (slot_map && tok >= 0 && tok < ntok) atomicMin(&lmap[tok], (int32_t)row);
  }
  const int nfill = W - min(count, W);
  if (nfill > 0) {
    int64_t ctok, vtok;
    if (fill == 0) {
      ctok = d[npre + last];
      vtok = ctok;
    } else {
      ctok = count > 0 ? d[npre + last] : (npre > 0 ? d[npre - 1] : 0);
      vtok = 0;
    }
    for (int j = tid; j < nfill; j += kPlanThreads) {
      const int slot = npre + (W - nfill) + j;
      const int64_t row = row0 + slot;
      upd[row] = vtok;
      abat[row] = b;
      apos[row] = slot;
      atok[row] = ctok;
      pmask[row] = ctok >= npre ? 1 : 0;
      ridx[row] = ctok > npre ? ctok - npre : 0;
      qvalid[row] = fill == 0 ? 1 : 0;
      // A fixed-width fill slot is a query (candidate 0 of an image that keeps nothing is corrected
      // only through these slots); a padded fill slot is not.
      if (fill == 0 && j == 0 && slot_map && ctok >= 0 && ctok < ntok) atomicMin(&lmap[ctok], (int32_t)row);
    }
  }
  for (int j = tid; j < npre; j += kPlanThreads) {
    const int64_t tok = d[j];
    const int64_t row = row0 + j;
    upd[row] = tok;
    abat[row] = b;
    apos[row] = j;
    atok[row] = tok;
    pmask[row] = tok >= npre ? 1 : 0;
    ridx[row] = tok > npre ? tok - npre : 0;
    qvalid[row] = 1;
    if (slot_map && tok >= 0 && tok < ntok) atomicMin(&lmap[tok], (int32_t)row);
  }
  if (slot_map) {
    __syncthreads();
    for (int i = tid; i < ntok; i += kPlanThreads) {
      const int32_t v = lmap[i];
      slot_map[(int64_t)b * ntok + i] = v == 0x7fffffff ? -1 : v;
    }
  }
}

// Running statistics of one plan (one 1024-thread workgroup, a fixed summation order, so the values
// do not depend on timing): out = {sum(scores * keep), sum(scores), sum(keep), B * P, B}. The
// product takes keep as 0.0 / 1.0 exactly like (scores * keep.float()).sum(), so a -inf score that
// is not kept makes the first sum NaN, as it does there.
__global__ __launch_bounds__(kPlanThreads) void plan_stats_kernel(const float* __restrict__ scores, int B, int P,
                                                                  int64_t ssb, const uint8_t* __restrict__ keep,
                                                                  float* __restrict__ out) {
  __shared__ float part[3][kPlanWaves];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  float kept_mass = 0.0f, full_mass = 0.0f, kept = 0.0f;
  // Thread t takes columns t, t + 1024, ... of every row, rows in order; four loads in flight.
  for (int b = 0; b < B; ++b) {
    const float* srow = scores + (int64_t)b * ssb;
    const uint8_t* krow = keep + (int64_t)b * P;
    for (int p0 = tid; p0 < P; p0 += 4 * kPlanThreads) {
      float v[4], kf[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int p = p0 + u * kPlanThreads;
        v[u] = p < P ? srow[p] : 0.0f;
        kf[u] = (p < P && krow[p]) ? 1.0f : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (p0 + u * kPlanThreads < P) {
          kept_mass += v[u] * kf[u];
          full_mass += v[u];
          kept += kf[u];
        }
      }
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    kept_mass += __shfl_xor(kept_mass, o, 64);
    full_mass += __shfl_xor(full_mass, o, 64);
    kept += __shfl_xor(kept, o, 64);
  }
  if (lane == 0) {
    part[0][w] = kept_mass;
    part[1][w] = full_mass;
    part[2][w] = kept;
  }
  __syncthreads();
  if (tid < 3) {
    float t = part[tid][0];
    for (int j = 1; j < kPlanWaves; ++j) t += part[tid][j];
    out[tid] = 0.0f + t;  // as the running total 0 + sum after the first plan (-0 becomes +0)
  } else if (tid == 3) {
    out[3] = (float)B * (float)P;
  } else if (tid == 4) {
    out[4] = (float)B;
  }
}

}  // namespace oudjat

using namespace oudjat;

extern "C" int oudjat_plan_stats(const float* scores, int64_t B, int64_t P, int64_t ssb, const uint8_t* keep,
                                 float* out, oudjat_stream_t stream) {
  OUDJAT_REQUIRE(B >= 0 && P >= 0, OUDJAT_ERR_INVALID_ARGUMENT, "plan_stats: negative size");
  OUDJAT_REQUIRE(out && (B * P == 0 || (scores && keep)), OUDJAT_ERR_INVALID_ARGUMENT, "plan_stats: null pointer");
  OUDJAT_REQUIRE(ssb >= P, OUDJAT_ERR_UNSUPPORTED_LAYOUT, "plan_stats: score row stride %lld < P=%lld",
                 (long long)ssb, (long long)P);
  OUDJAT_REQUIRE(B < ((int64_t)1 << 24) && B * P < ((int64_t)1 << 40), OUDJAT_ERR_TOO_LARGE, "plan_stats: too large");
  plan_stats_kernel<<<1, kPlanThreads, 0, as_stream(stream)>>>(scores, (int)B, (int)P, ssb, keep, out);
  return check_launch("plan_stats");
}

extern "C" int oudjat_topk_plan(const float* scores, int64_t B, int64_t P, int64_t ssb, int64_t k,
                                const int64_t* dindice, int64_t dsb, int64_t npre, int64_t ntok, int64_t* upd,
                                int64_t* abat, int64_t* apos, int64_t* atok, uint8_t* pmask, int64_t* ridx,
                                uint8_t* keep, int32_t* slot_map, oudjat_stream_t stream) {
  OUDJAT_REQUIRE(B >= 0 && P >= 0 && npre >= 0 && ntok >= 0, OUDJAT_ERR_INVALID_ARGUMENT, "topk_plan: negative size");
  OUDJAT_REQUIRE(k >= 0 && k <= P, OUDJAT_ERR_INVALID_ARGUMENT, "topk_plan: k=%lld outside [0, P=%lld]", (long long)k,
                 (long long)P);
  if (B == 0) return OUDJAT_OK;
  OUDJAT_REQUIRE(dindice && upd && abat && apos && atok && pmask && ridx && (scores || P == 0),
                 OUDJAT_ERR_INVALID_ARGUMENT, "topk_plan: null pointer");
  OUDJAT_REQUIRE(P <= kMaxCandidates, OUDJAT_ERR_TOO_LARGE, "topk_plan: P=%lld exceeds %lld", (long long)P,
                 (long long)kMaxCandidates);
  OUDJAT_REQUIRE(npre + k < ((int64_t)1 << 30) && B * (npre + k) < ((int64_t)1 << 31), OUDJAT_ERR_TOO_LARGE,
                 "topk_plan: plan too large for int32 slots");
  const int64_t lds = (P + (slot_map ? ntok : 0)) * 4;
  OUDJAT_REQUIRE(lds <= kMaxPlanLds, OUDJAT_ERR_TOO_LARGE, "topk_plan: needs %lld bytes of LDS (max %lld)",
                 (long long)lds, (long long)kMaxPlanLds);
  if (lds > 48 * 1024) {
    // Raised to the maximum once per device (also keeps the call out of captured launch sequences).
    static std::atomic<uint8_t> attr_set[64];
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return set_error(OUDJAT_ERR_HIP, "topk_plan: hipGetDevice: %s", hipGetErrorString(e));
    if (!attr_set[dev & 63].load(std::memory_order_acquire)) {
      e = hipFuncSetAttribute((const void*)topk_plan_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)kMaxPlanLds);
      if (e != hipSuccess) return set_error(OUDJAT_ERR_HIP, "topk_plan: hipFuncSetAttribute: %s", hipGetErrorString(e));
      attr_set[dev & 63].store(1, std::memory_order_release);
    }
  }
  topk_plan_kernel<<<(unsigned)B, kPlanThreads, (size_t)lds, as_stream(stream)>>>(
      scores, (int)P, ssb, (int)k, dindice, dsb, (int)npre, (int)ntok, upd, abat, apos, atok, pmask, ridx, keep,
      slot_map);
  return check_launch("topk_plan");
}

extern "C" int oudjat_threshold_keep(const float* scores, int64_t B, int64_t P, int64_t ssb, float thres,
                                     uint8_t* keep, int32_t* kept_count, oudjat_stream_t stream) {
  OUDJAT_REQUIRE(B >= 0 && P >= 0, OUDJAT_ERR_INVALID_ARGUMENT, "threshold_keep: negative size");
  if (B == 0) return OUDJAT_OK;
  OUDJAT_REQUIRE(kept_count && (scores || P == 0), OUDJAT_ERR_INVALID_ARGUMENT, "threshold_keep: null pointer");
  OUDJAT_REQUIRE(P == 0 || ssb >= P, OUDJAT_ERR_UNSUPPORTED_LAYOUT, "threshold_keep: score row stride %lld < P=%lld",
                 (long long)ssb, (long long)P);
  OUDJAT_REQUIRE(B < ((int64_t)1 << 31) && P < ((int64_t)1 << 30), OUDJAT_ERR_TOO_LARGE, "threshold_keep: too large");
  threshold_keep_kernel<<<(unsigned)B, kKeepThreads, 0, as_stream(stream)>>>(scores, (int)P, ssb, thres, keep,
                                                                            kept_count);
  return check_launch("threshold_keep");
}

extern "C" int oudjat_threshold_plan(const float* scores, int64_t B, int64_t P, int64_t ssb, float thres,
                                     int64_t width, int fill_mode, const int64_t* dindice, int64_t dsb, int64_t npre,
                                     int64_t ntok, int64_t* upd, int64_t* abat, int64_t* apos, int64_t* atok,
                                     uint8_t* pmask, int64_t* ridx, uint8_t* query_valid, uint8_t* keep,
                                     int32_t* kept_count, int32_t* slot_map, oudjat_stream_t stream) {
  OUDJAT_REQUIRE(B >= 0 && P >= 0 && npre >= 0 && ntok >= 0, OUDJAT_ERR_INVALID_ARGUMENT,
                 "threshold_plan: negative size");
  OUDJAT_REQUIRE(width >= 0 && width <= P, OUDJAT_ERR_INVALID_ARGUMENT, "threshold_plan: width=%lld outside [0, P=%lld]",
                 (long long)width, (long long)P);
  OUDJAT_REQUIRE(fill_mode == 0 || fill_mode == 1, OUDJAT_ERR_INVALID_ARGUMENT, "threshold_plan: fill_mode %d",
                 fill_mode);
  if (B == 0) return OUDJAT_OK;
  OUDJAT_REQUIRE(dindice && upd && abat && apos && atok && pmask && ridx && query_valid && kept_count &&
                     (scores || P == 0),
                 OUDJAT_ERR_INVALID_ARGUMENT, "threshold_plan: null pointer");
  OUDJAT_REQUIRE(P == 0 || ssb >= P, OUDJAT_ERR_UNSUPPORTED_LAYOUT, "threshold_plan: score row stride %lld < P=%lld",
                 (long long)ssb, (long long)P);
  OUDJAT_REQUIRE(dsb >= npre + P, OUDJAT_ERR_UNSUPPORTED_LAYOUT, "threshold_plan: dindice row stride %lld < %lld",
                 (long long)dsb, (long long)(npre + P));
  OUDJAT_REQUIRE(P <= kMaxCandidates, OUDJAT_ERR_TOO_LARGE, "threshold_plan: P=%lld exceeds %lld", (long long)P,
                 (long long)kMaxCandidates);
  OUDJAT_REQUIRE(npre + width < ((int64_t)1 << 30) && B * (npre + width) < ((int64_t)1 << 31), OUDJAT_ERR_TOO_LARGE,
                 "threshold_plan: plan too large for int32 slots");
  const int64_t lds = slot_map ? ntok * 4 : 0;
  OUDJAT_REQUIRE(lds <= kMaxPlanLds, OUDJAT_ERR_TOO_LARGE, "threshold_plan: needs %lld bytes of LDS (max %lld)",
                 (long long)lds, (long long)kMaxPlanLds);
  if (lds > 48 * 1024) {
    static std::atomic<uint8_t> attr_set[64];
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return set_error(OUDJAT_ERR_HIP, "threshold_plan: hipGetDevice: %s", hipGetErrorString(e));
    if (!attr_set[dev & 63].load(std::memory_order_acquire)) {
      e = hipFuncSetAttribute((const void*)threshold_plan_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)kMaxPlanLds);
      if (e != hipSuccess)
        return set_error(OUDJAT_ERR_HIP, "threshold_plan: hipFuncSetAttribute: %s", hipGetErrorString(e));
      attr_set[dev & 63].store(1, std::memory_order_release);
    }
  }
  threshold_plan_kernel<<<(unsigned)B, kPlanThreads, (size_t)lds, as_stream(stream)>>>(
      scores, (int)P, ssb, thres, (int)width, fill_mode, dindice, dsb, (int)npre, (int)ntok, upd, abat, apos, atok,
      pmask, ridx, query_valid, keep, kept_count, slot_map);
  return check_launch("threshold_plan");
}
