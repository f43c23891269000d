// Shared device/host helpers for the gfx950 token-correction kernels.
//
// bf16 values travel as raw uint16_t bit patterns; conversions are written out here so that the
// rounding (round-to-nearest-even, the rounding torch's c10::BFloat16 uses) is explicit.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>

#include "../../include/oudjat.h"

namespace oudjat {

typedef uint16_t bf16_t;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;  // canonical quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

// Two bf16 packed in one dword: low half = element 0.
__device__ __forceinline__ float lo_bf16(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_bf16(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return f32_to_bf16(a) | (f32_to_bf16(b) << 16);
}

__device__ __forceinline__ float round_bf16(float f) { return __uint_as_float(f32_to_bf16(f) << 16); }

// Unpack 8 bf16 (one 16-byte vector) to fp32.
__device__ __forceinline__ void unpack8(const uint4& v, float* f) {
  f[0] = lo_bf16(v.x); f[1] = hi_bf16(v.x);
  f[2] = lo_bf16(v.y); f[3] = hi_bf16(v.y);
  f[4] = lo_bf16(v.z); f[5] = hi_bf16(v.z);
  f[6] = lo_bf16(v.w); f[7] = hi_bf16(v.w);
}
__device__ __forceinline__ uint4 pack8(const float* f) {
  uint4 v;
  v.x = pack_bf16x2(f[0], f[1]);
  v.y = pack_bf16x2(f[2], f[3]);
  v.z = pack_bf16x2(f[4], f[5]);
  v.w = pack_bf16x2(f[6], f[7]);
  return v;
}

__device__ __forceinline__ bf16x8_t as_bf16x8(const uint4& v) { return __builtin_bit_cast(bf16x8_t, v); }

// Rotate-half RoPE on one 8-wide chunk of the left half and its partner chunk of the right half.
// fp32 math with every product and sum rounded separately, matching an eager
// (x * cos) + (rotate_half(x) * sin) evaluated in fp32. Contraction is switched off for this scope
// (plain operators: the __f*_rn helpers are themselves contractable after inlining).
__device__ __forceinline__ void rope8(float* l, float* r, const float* cl, const float* cr, const float* sl,
                                      const float* sr) {
#pragma clang fp contract(off)
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float nl = l[e] * cl[e] - r[e] * sl[e];
    const float nr = r[e] * cr[e] + l[e] * sr[e];
    l[e] = nl;
    r[e] = nr;
  }
}

__device__ __forceinline__ void load8f(const float* p, float* f) {
  const float4 a = reinterpret_cast<const float4*>(p)[0];
  const float4 b = reinterpret_cast<const float4*>(p)[1];
  f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
  f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
}

// Wavefront (64-lane) reductions.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// ---------------------------------------------------------------------------------------------
// Host-side status plumbing. Every exported entry point returns an oudjat status; the message of
// the most recent failure on the calling thread is kept for oudjat_last_error().
// ---------------------------------------------------------------------------------------------
int set_error(int status, const char* fmt, ...);
int check_launch(const char* what);

// Device address of the no-alloc entry point's scratch array on the current device (pscore.hip),
// looked up once per device; `out` may be NULL to only perform the lookup.
int noalloc_scratch(float** out);

inline hipStream_t as_stream(oudjat_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned(const void* p, int64_t a) { return (reinterpret_cast<uintptr_t>(p) % (uintptr_t)a) == 0; }

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---- direct-to-LDS loads and their waits (shared by the GEMM and attention kernels) ----------------

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding: vmcnt in bits 3:0 and
// 15:14, expcnt 6:4 and lgkmcnt 11:8 at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Workgroup barrier without the vmcnt(0) of __syncthreads() (which would drain the loads in flight
// for later tiles): LDS reads are complete (lgkmcnt(0)), then s_barrier. The scheduling barriers
// keep the compiler from moving memory operations across it.
__device__ __forceinline__ void block_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));  // lgkmcnt(0), vmcnt/expcnt unconstrained
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
}

// Buffer descriptor of a raw byte range (stride 0, bounds-checked against `bytes`: loads past it
// return zeros) and the 16-byte-per-lane buffer load into LDS (lane l's bytes land at lds + 16 l).
typedef int i32x4_t __attribute__((ext_vector_type(4)));
__device__ void llvm_raw_buffer_load_lds(i32x4_t rsrc, __attribute__((address_space(3))) void* lds, int size,
                                         int voffset, int soffset, int offset,
                                         int aux) __asm("llvm.amdgcn.raw.buffer.load.lds");
__device__ __forceinline__ i32x4_t make_buffer_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  i32x4_t r;
  r[0] = (int)(uint32_t)a;
  r[1] = (int)((uint32_t)(a >> 32) & 0xffffu);  // base[47:32], stride 0
  r[2] = (int)bytes;
  r[3] = 0x00020000;                            // 32-bit data format, no swizzle
  return r;
}
__device__ __forceinline__ void buffer_load_lds16(i32x4_t rsrc, unsigned char* lds, uint32_t voffset) {
  llvm_raw_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)lds, 16, (int)voffset, 0, 0, 0);
}

}  // namespace oudjat

#define OUDJAT_REQUIRE(cond, status, ...)                 \
  do {                                                    \
    if (!(cond)) return ::oudjat::set_error((status), __VA_ARGS__); \
  } while (0)
