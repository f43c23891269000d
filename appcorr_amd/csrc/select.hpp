// Block-wide selection helpers of the plan kernels (1024-thread workgroups).
#pragma once

#include "common.hpp"

namespace oudjat {

static constexpr int kPlanThreads = 1024;
static constexpr int kPlanWaves = kPlanThreads / 64;

__device__ __forceinline__ uint32_t order_key(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0xffffffffu;  // NaN ranks above +inf
  if (u == 0x80000000u) u = 0u;                             // -0.0 ties with +0.0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    uint32_t t = __shfl_up(v, o, 64);
    if (lane >= o) v += t;
  }
  return v;
}

// Exclusive prefix sum of one value per thread over the 1024-thread block, in thread order.
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t* sh) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const uint32_t incl = wave_incl_scan(v, lane);
  if (lane == 63) sh[w] = incl;
  __syncthreads();
  if (w == 0) {
    uint32_t t = lane < kPlanWaves ? sh[lane] : 0u;
    uint32_t ti = wave_incl_scan(t, lane);
    if (lane < kPlanWaves) sh[lane] = ti - t;
  }
  __syncthreads();
  const uint32_t r = sh[w] + incl - v;
  __syncthreads();
  return r;
}

// The k-th largest of the P order keys in LDS (0 < k < P): a 4-round radix select, 8-bit digits from
// the top, one LDS histogram per round. Returns the k-th key; *remaining = how many keys equal to it
// are among the k largest. Every thread of the 1024-thread block must call it.
__device__ __forceinline__ uint32_t radix_select_kth(const uint32_t* keys, int P, uint32_t k, uint32_t* hist,
                                                     uint32_t* sel_sh, uint32_t* remaining_out) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  uint32_t remaining = k;
  uint32_t prefix = 0u, pbits = 0u;
  for (int shift = 24; shift >= 0; shift -= 8) {
    if (tid < 256) hist[tid] = 0u;
    __syncthreads();
    for (int i = tid; i < P; i += kPlanThreads) {
      const uint32_t key = keys[i];
      if ((key & pbits) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (tid < 64) {
      // Lane l owns bins 255-4l .. 252-4l, i.e. the histogram read from the top digit down.
      uint32_t c[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) c[j] = hist[255 - 4 * tid - j];
      const uint32_t local = c[0] + c[1] + c[2] + c[3];
      uint32_t run = wave_incl_scan(local, lane) - local;  // elements in higher bins
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (run < remaining && remaining <= run + c[j]) {
          sel_sh[0] = (uint32_t)(255 - 4 * tid - j);
          sel_sh[1] = run;
        }
        run += c[j];
      }
    }
    __syncthreads();
    const uint32_t digit = sel_sh[0];
    remaining -= sel_sh[1];
    prefix |= digit << shift;
    pbits |= 255u << shift;
    __syncthreads();
  }
  *remaining_out = remaining;
  return prefix;
}

}  // namespace oudjat
