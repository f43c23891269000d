// Row movement kernels: gather, scatter (K/V rewrite, query scatter), active-token update, the fused
// reconstruct + scatter + persist step, LayerScale-add and the per-patch importance reduction.
//
// All of these are HBM-bound byte movers. Layout decisions:
//   * one wavefront per row, so the row's (batch, token) index pair is a wave-uniform scalar load;
//   * each lane moves 16-byte vectors (8 bf16) and issues all of its loads before its stores so a
//     wave keeps up to 4 x 16 B per lane in flight;
//   * four waves (256 threads) per workgroup, thousands of workgroups per launch on the headline
//     shapes (M = 4176 rows -> 1044 workgroups), which spreads the rows over all 8 XCDs.
#include "common.hpp"

namespace oudjat {

static constexpr int kRowThreads = 256;
static constexpr int kRowsPerWg = kRowThreads / 64;
static constexpr int kUnroll = 4;

// Copy `chunks` vectors of type V from s to d, one wave, lanes striding by 64.
template <typename V>
__device__ __forceinline__ void wave_copy(const char* __restrict__ s, char* __restrict__ d, int chunks, int lane) {
  const V* sv = reinterpret_cast<const V*>(s);
  V* dv = reinterpret_cast<V*>(d);
  int c = lane;
  for (; c + 64 * (kUnroll - 1) < chunks; c += 64 * kUnroll) {
    V r[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) r[u] = sv[c + 64 * u];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) dv[c + 64 * u] = r[u];
  }
  for (; c < chunks; c += 64) dv[c] = sv[c];
}

template <typename V>
__global__ __launch_bounds__(kRowThreads) void gather_rows_kernel(
    const char* __restrict__ src, int64_t sb, int64_t sn, int chunks, const int64_t* __restrict__ bi,
    const int64_t* __restrict__ ti, int64_t n, char* __restrict__ dst, int64_t ds) {
  const int64_t row = (int64_t)blockIdx.x * kRowsPerWg + (threadIdx.x >> 6);
  if (row >= n) return;
  const int lane = threadIdx.x & 63;
  const int64_t b = bi[row], t = ti[row];
  wave_copy<V>(src + b * sb + t * sn, dst + row * ds, chunks, lane);
}

template <typename V>
__global__ __launch_bounds__(kRowThreads) void scatter_rows_kernel(
    char* __restrict__ dst, int64_t db, int64_t dn, int chunks, const int64_t* __restrict__ bi,
    const int64_t* __restrict__ ti, int64_t n, const char* __restrict__ src, int64_t ss) {
  const int64_t row = (int64_t)blockIdx.x * kRowsPerWg + (threadIdx.x >> 6);
  if (row >= n) return;
  const int lane = threadIdx.x & 63;
  const int64_t b = bi[row], t = ti[row];
  wave_copy<V>(src + row * ss, dst + b * db + t * dn, chunks, lane);
}

// Largest power-of-two vector width (<= 16 bytes) that divides every byte quantity given.
static int pick_width(std::initializer_list<int64_t> vals) {
  int w = 16;
  for (int64_t v : vals) {
    while (w > 1 && (v % w) != 0) w >>= 1;
  }
  return w;
}

template <bool kGather>
static int launch_rows(char* dst, int64_t d0, int64_t d1, const char* src, int64_t s0, int64_t s1, int64_t row_bytes,
                       const int64_t* bi, const int64_t* ti, int64_t n, hipStream_t st) {
  // kGather: src is indexed by (bi, ti) with strides (s0, s1); dst rows stride d0.
  // scatter: dst is indexed by (bi, ti) with strides (d0, d1); src rows stride s0.
  int w = pick_width({(int64_t)(uintptr_t)dst, (int64_t)(uintptr_t)src, d0, d1, s0, s1, row_bytes});
  int chunks = (int)(row_bytes / w);
  dim3 grid((unsigned)cdiv(n, kRowsPerWg));
#define OUDJAT_ROWS_CASE(W, T)                                                                          \
  case W:                                                                                               \
    if (kGather)                                                                                        \
      gather_rows_kernel<T><<<grid, kRowThreads, 0, st>>>(src, s0, s1, chunks, bi, ti, n, dst, d0);     \
    else                                                                                                \
      scatter_rows_kernel<T><<<grid, kRowThreads, 0, st>>>(dst, d0, d1, chunks, bi, ti, n, src, s0);    \
    break;
  switch (w) {
    OUDJAT_ROWS_CASE(16, uint4)
    OUDJAT_ROWS_CASE(8, uint2)
    OUDJAT_ROWS_CASE(4, uint32_t)
    OUDJAT_ROWS_CASE(2, uint16_t)
    OUDJAT_ROWS_CASE(1, uint8_t)
  }
#undef OUDJAT_ROWS_CASE
  return check_launch(kGather ? "gather_rows" : "scatter_rows");
}

// x_out[b, t] = bf16(a[i] + d[i]) for C bf16 columns.
__global__ __launch_bounds__(kRowThreads) void active_token_update_kernel(
    uint16_t* __restrict__ xo, int64_t sb, int64_t sn, const int64_t* __restrict__ bi, const int64_t* __restrict__ ti,
    int64_t n, const uint16_t* __restrict__ a, int64_t as, const uint16_t* __restrict__ d, int64_t ds, int chunks) {
  const int64_t row = (int64_t)blockIdx.x * kRowsPerWg + (threadIdx.x >> 6);
  if (row >= n) return;
  const int lane = threadIdx.x & 63;
  const int64_t b = bi[row], t = ti[row];
  const uint4* av = reinterpret_cast<const uint4*>(a + row * as);
  const uint4* dv = reinterpret_cast<const uint4*>(d + row * ds);
  uint4* ov = reinterpret_cast<uint4*>(xo + b * sb + t * sn);
  for (int c = lane; c < chunks; c += 64) {
    float fa[8], fd[8];
    unpack8(av[c], fa);
    unpack8(dv[c], fd);
#pragma unroll
    for (int e = 0; e < 8; ++e) fa[e] = fa[e] + fd[e];
    ov[c] = pack8(fa);
  }
}

// The fused residual step of one correction block. One wave per row of [rows, C].
__global__ __launch_bounds__(kRowThreads) void reconstruct_scatter_persist_kernel(
    const uint16_t* x, uint16_t* __restrict__ bos, const int32_t* __restrict__ row_slot,
    const uint16_t* __restrict__ xa, const uint16_t* __restrict__ xt, const uint16_t* __restrict__ mlp,
    int64_t rows, int64_t C, uint16_t* xo) {
  const int64_t row = (int64_t)blockIdx.x * kRowsPerWg + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const int chunks = (int)(C >> 3);
  const int32_t slot = row_slot[row];
  uint4* ov = reinterpret_cast<uint4*>(xo + row * C);
  uint4* bv = reinterpret_cast<uint4*>(bos + row * C);
  if (slot < 0) {
    const uint4* xv = reinterpret_cast<const uint4*>(x + row * C);
    for (int c = lane; c < chunks; c += 64) {
      float fx[8], fb[8];
      unpack8(xv[c], fx);
      unpack8(bv[c], fb);
#pragma unroll
      for (int e = 0; e < 8; ++e) fx[e] = fx[e] + fb[e];
      ov[c] = pack8(fx);
    }
  } else {
    const int64_t s = slot;
    const uint4* av = reinterpret_cast<const uint4*>(xa + s * C);
    const uint4* tv = reinterpret_cast<const uint4*>(xt + s * C);
    const uint4* mv = reinterpret_cast<const uint4*>(mlp + s * C);
    for (int c = lane; c < chunks; c += 64) {
      float fa[8], ft[8], fm[8], fo[8], fb[8];
      unpack8(av[c], fa);
      unpack8(tv[c], ft);
      unpack8(mv[c], fm);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        fo[e] = ft[e] + fm[e];
        fb[e] = round_bf16(ft[e] - fa[e]) + fm[e];
      }
      ov[c] = pack8(fo);
      bv[c] = pack8(fb);
    }
  }
}

// Selected-row half of the residual step when the selected rows stay packed between blocks:
// x_new[i] = bf16(x_attn + mlp) and blocks_out_sum[b_i, t_i] = bf16(bf16(x_attn - x_act) + mlp).
// One wave per packed row.
__global__ __launch_bounds__(kRowThreads) void packed_residual_persist_kernel(
    const uint16_t* __restrict__ xa, const uint16_t* __restrict__ xt, const uint16_t* __restrict__ mlp, int64_t rows,
    int64_t C, const int64_t* __restrict__ bi, const int64_t* __restrict__ ti, uint16_t* __restrict__ bos,
    int64_t bsb, int64_t bsn, uint16_t* xn) {
  const int64_t row = (int64_t)blockIdx.x * kRowsPerWg + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const int chunks = (int)(C >> 3);
  const uint4* av = reinterpret_cast<const uint4*>(xa + row * C);
  const uint4* tv = reinterpret_cast<const uint4*>(xt + row * C);
  const uint4* mv = reinterpret_cast<const uint4*>(mlp + row * C);
  uint4* ov = reinterpret_cast<uint4*>(xn + row * C);
  uint4* bv = reinterpret_cast<uint4*>(bos + bi[row] * bsb + ti[row] * bsn);
  for (int c = lane; c < chunks; c += 64) {
    float fa[8], ft[8], fm[8], fo[8], fb[8];
    unpack8(av[c], fa);
    unpack8(tv[c], ft);
    unpack8(mv[c], fm);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      fo[e] = ft[e] + fm[e];
      fb[e] = round_bf16(ft[e] - fa[e]) + fm[e];
    }
    ov[c] = pack8(fo);
    bv[c] = pack8(fb);
  }
}

// Rows of [rows, C] after a run of L correction blocks whose selected rows stayed packed: a selected
// row (row_slot >= 0) takes its packed row; an unselected row takes x + bos_0 + ... + bos_{L-1}
// with a bf16 rounding after every addition, i.e. the per-block x + blocks_out_sum sequence. One
// thread per 8 columns, the L row loads issued four at a time.
__global__ __launch_bounds__(256) void fold_residual_rows_kernel(const uint16_t* x, int64_t rows, int64_t C,
                                                                 const int32_t* __restrict__ row_slot,
                                                                 const uint16_t* __restrict__ xp,
                                                                 const uint16_t* const* __restrict__ bos, int L,
                                                                 uint16_t* xo) {
  const int64_t chunks = C >> 3;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t row = gid / chunks;
  if (row >= rows) return;
  const int64_t off = row * C + (gid - row * chunks) * 8;
  const int32_t slot = row_slot[row];
  if (slot >= 0) {
    *reinterpret_cast<uint4*>(xo + off) =
        *reinterpret_cast<const uint4*>(xp + (int64_t)slot * C + (gid - row * chunks) * 8);
    return;
  }
  float v[8];
  unpack8(*reinterpret_cast<const uint4*>(x + off), v);
  int l = 0;
  for (; l + 4 <= L; l += 4) {
    uint4 b[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) b[u] = *reinterpret_cast<const uint4*>(bos[l + u] + off);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      float f[8];
      unpack8(b[u], f);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = round_bf16(v[e] + f[e]);
    }
  }
  for (; l < L; ++l) {
    float f[8];
    unpack8(*reinterpret_cast<const uint4*>(bos[l] + off), f);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = round_bf16(v[e] + f[e]);
  }
  *reinterpret_cast<uint4*>(xo + off) = pack8(v);
}

__global__ __launch_bounds__(kRowThreads) void layerscale_add_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ a, const uint16_t* __restrict__ g, int64_t rows,
    int64_t C, uint16_t* __restrict__ o) {
  const int64_t row = (int64_t)blockIdx.x * kRowsPerWg + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const int chunks = (int)(C >> 3);
  const uint4* xv = reinterpret_cast<const uint4*>(x + row * C);
  const uint4* av = reinterpret_cast<const uint4*>(a + row * C);
  const uint4* gv = reinterpret_cast<const uint4*>(g);
  uint4* ov = reinterpret_cast<uint4*>(o + row * C);
  for (int c = lane; c < chunks; c += 64) {
    float fx[8], fa[8], fg[8];
    unpack8(xv[c], fx);
    unpack8(av[c], fa);
    unpack8(gv[c], fg);
#pragma unroll
    for (int e = 0; e < 8; ++e) fx[e] = fmaf(fa[e], fg[e], fx[e]);
    ov[c] = pack8(fx);
  }
}

// The approximate block's two residual sums in one pass (block.py:336-347): the cached
// blocks_out_sum = bf16(inc + mlp) (inc = ls1(attn)) and the block output bf16(x_attn + mlp). One wave
// per row, every load of the row issued before the first store.
template <int CH>
__global__ __launch_bounds__(kRowThreads) void residual_pair_kernel(const uint16_t* __restrict__ inc,
                                                                   const uint16_t* __restrict__ xa,
                                                                   const uint16_t* __restrict__ mlp, int64_t rows,
                                                                   int64_t C, uint16_t* __restrict__ bos,
                                                                   uint16_t* __restrict__ out) {
  const int64_t row = (int64_t)blockIdx.x * kRowsPerWg + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const int chunks = (int)(C >> 3);
  const uint4* iv = reinterpret_cast<const uint4*>(inc + row * C);
  const uint4* av = reinterpret_cast<const uint4*>(xa + row * C);
  const uint4* mv = reinterpret_cast<const uint4*>(mlp + row * C);
  uint4 ri[CH], ra[CH], rm[CH];
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    const int c = lane + 64 * j;
    if (c < chunks) {
      ri[j] = iv[c];
      ra[j] = av[c];
      rm[j] = mv[c];
    }
  }
  uint4* bv = reinterpret_cast<uint4*>(bos + row * C);
  uint4* ov = reinterpret_cast<uint4*>(out + row * C);
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    const int c = lane + 64 * j;
    if (c < chunks) {
      float fi[8], fa[8], fm[8], fb[8], fo[8];
      unpack8(ri[j], fi);
      unpack8(ra[j], fa);
      unpack8(rm[j], fm);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        fb[e] = fi[e] + fm[e];
        fo[e] = fa[e] + fm[e];
      }
      bv[c] = pack8(fb);
      ov[c] = pack8(fo);
    }
  }
}

// vec: rows are 16-byte aligned with dim % 4 == 0, so a lane reads 16-byte vectors, four in flight
// (a 1024-wide row is one round of four loads per lane).
__global__ __launch_bounds__(kRowThreads) void patch_importance_kernel(
    const float* __restrict__ d, int64_t rows, int64_t dim, int64_t rs, int mode, bool vec, float* __restrict__ out) {
  const int64_t row = (int64_t)blockIdx.x * kRowsPerWg + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const float* p = d + row * rs;
  float acc = 0.0f;
  if (vec) {
    const float4* p4 = reinterpret_cast<const float4*>(p);
    const int64_t n4 = dim >> 2;
    int64_t c = lane;
    for (; c + 192 < n4; c += 256) {
      float4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = p4[c + 64 * u];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        acc = fmaf(v[u].x, v[u].x, acc);
        acc = fmaf(v[u].y, v[u].y, acc);
        acc = fmaf(v[u].z, v[u].z, acc);
        acc = fmaf(v[u].w, v[u].w, acc);
      }
    }
    for (; c < n4; c += 64) {
      const float4 v = p4[c];
      acc = fmaf(v.x, v.x, acc);
      acc = fmaf(v.y, v.y, acc);
      acc = fmaf(v.z, v.z, acc);
      acc = fmaf(v.w, v.w, acc);
    }
  } else {
    for (int64_t c = lane; c < dim; c += 64) {
      float v = p[c];
      acc = fmaf(v, v, acc);
    }
  }
  acc = wave_sum(acc);
  if (lane == 0) {
    float r;
    if (mode == OUDJAT_IMPORTANCE_ENERGY) r = acc;
    else if (mode == OUDJAT_IMPORTANCE_RMS) r = sqrtf(acc / (float)dim);
    else r = sqrtf(acc);
    out[row] = r;
  }
}

}  // namespace oudjat

using namespace oudjat;

extern "C" int oudjat_gather_rows(const void* src, int64_t sb, int64_t sn, int64_t row_bytes, const int64_t* bi,
                                  const int64_t* ti, int64_t n, void* dst, int64_t ds, oudjat_stream_t stream) {
  OUDJAT_REQUIRE(n >= 0 && row_bytes >= 0, OUDJAT_ERR_INVALID_ARGUMENT, "gather_rows: negative size");
  if (n == 0 || row_bytes == 0) return OUDJAT_OK;
  OUDJAT_REQUIRE(src && dst && bi && ti, OUDJAT_ERR_INVALID_ARGUMENT, "gather_rows: null pointer");
  OUDJAT_REQUIRE(ds >= row_bytes, OUDJAT_ERR_UNSUPPORTED_LAYOUT, "gather_rows: dst rows overlap (stride %lld < row %lld)",
                 (long long)ds, (long long)row_bytes);
  OUDJAT_REQUIRE(row_bytes <= (int64_t)1 << 30 && n < ((int64_t)1 << 40), OUDJAT_ERR_TOO_LARGE, "gather_rows: too large");
  return launch_rows<true>((char*)dst, ds, 0, (const char*)src, sb, sn, row_bytes, bi, ti, n, as_stream(stream));
}

extern "C" int oudjat_scatter_rows(void* dst, int64_t db, int64_t dn, int64_t row_bytes, const int64_t* bi,
                                   const int64_t* ti, int64_t n, const void* src, int64_t ss, oudjat_stream_t stream) {
  OUDJAT_REQUIRE(n >= 0 && row_bytes >= 0, OUDJAT_ERR_INVALID_ARGUMENT, "scatter_rows: negative size");
  if (n == 0 || row_bytes == 0) return OUDJAT_OK;
  OUDJAT_REQUIRE(src && dst && bi && ti, OUDJAT_ERR_INVALID_ARGUMENT, "scatter_rows: null pointer");
  OUDJAT_REQUIRE(row_bytes <= (int64_t)1 << 30 && n < ((int64_t)1 << 40), OUDJAT_ERR_TOO_LARGE, "scatter_rows: too large");
  return launch_rows<false>((char*)dst, db, dn, (const char*)src, ss, 0, row_bytes, bi, ti, n, as_stream(stream));
}

extern "C" int oudjat_active_token_update(uint16_t* xo, int64_t sb, int64_t sn, const int64_t* bi, const int64_t* ti,
                                          int64_t n, const uint16_t* a, int64_t as, const uint16_t* d, int64_t ds,
                                          int64_t C, oudjat_stream_t stream) {
  OUDJAT_REQUIRE(n >= 0 && C >= 0, OUDJAT_ERR_INVALID_ARGUMENT, "active_token_update: negative size");
  if (n == 0 || C == 0) return OUDJAT_OK;
  OUDJAT_REQUIRE(xo && bi && ti && a && d, OUDJAT_ERR_INVALID_ARGUMENT, "active_token_update: null pointer");
  OUDJAT_REQUIRE(C % 8 == 0 && sb % 8 == 0 && sn % 8 == 0 && as % 8 == 0 && ds % 8 == 0 && aligned(xo, 16) &&
                     aligned(a, 16) && aligned(d, 16),
                 OUDJAT_ERR_UNSUPPORTED_LAYOUT, "active_token_update: rows must be 16-byte aligned with C %% 8 == 0");
  active_token_update_kernel<<<(unsigned)cdiv(n, kRowsPerWg), kRowThreads, 0, as_stream(stream)>>>(
      xo, sb, sn, bi, ti, n, a, as, d, ds, (int)(C / 8));
  return check_launch("active_token_update");
}

extern "C" int oudjat_reconstruct_scatter_persist(const uint16_t* x, uint16_t* bos, const int32_t* row_slot,
                                                  const uint16_t* xa, const uint16_t* xt, const uint16_t* mlp,
                                                  int64_t rows, int64_t C, uint16_t* xo, oudjat_stream_t stream) {
  OUDJAT_REQUIRE(rows >= 0 && C >= 0, OUDJAT_ERR_INVALID_ARGUMENT, "reconstruct_scatter_persist: negative size");
  if (rows == 0 || C == 0) return OUDJAT_OK;
  OUDJAT_REQUIRE(x && bos && row_slot && xo, OUDJAT_ERR_INVALID_ARGUMENT, "reconstruct_scatter_persist: null pointer");
  OUDJAT_REQUIRE(C % 8 == 0 && aligned(x, 16) && aligned(bos, 16) && aligned(xo, 16) && (!xa || aligned(xa, 16)) &&
                     (!xt || aligned(xt, 16)) && (!mlp || aligned(mlp, 16)),
                 OUDJAT_ERR_UNSUPPORTED_LAYOUT, "reconstruct_scatter_persist: rows must be 16-byte aligned, C %% 8 == 0");
  reconstruct_scatter_persist_kernel<<<(unsigned)cdiv(rows, kRowsPerWg), kRowThreads, 0, as_stream(stream)>>>(
      x, bos, row_slot, xa, xt, mlp, rows, C, xo);
  return check_launch("reconstruct_scatter_persist");
}

extern "C" int oudjat_packed_residual_persist(const uint16_t* x_act, const uint16_t* x_attn, const uint16_t* mlp,
                                              int64_t rows, int64_t C, const int64_t* batch_idx,
                                              const int64_t* token_idx, uint16_t* bos, int64_t bos_stride_b,
                                              int64_t bos_stride_n, uint16_t* x_new, oudjat_stream_t stream) {
  OUDJAT_REQUIRE(rows >= 0 && C >= 0, OUDJAT_ERR_INVALID_ARGUMENT, "packed_residual_persist: negative size");
  if (rows == 0 || C == 0) return OUDJAT_OK;
  OUDJAT_REQUIRE(x_act && x_attn && mlp && batch_idx && token_idx && bos && x_new, OUDJAT_ERR_INVALID_ARGUMENT,
                 "packed_residual_persist: null pointer");
  OUDJAT_REQUIRE(C % 8 == 0 && aligned(x_act, 16) && aligned(x_attn, 16) && aligned(mlp, 16) && aligned(bos, 16) &&
                     aligned(x_new, 16) && bos_stride_b % 8 == 0 && bos_stride_n % 8 == 0,
                 OUDJAT_ERR_UNSUPPORTED_LAYOUT, "packed_residual_persist: 16-byte aligned rows, C %% 8 == 0");
  packed_residual_persist_kernel<<<(unsigned)cdiv(rows, kRowsPerWg), kRowThreads, 0, as_stream(stream)>>>(
      x_act, x_attn, mlp, rows, C, batch_idx, token_idx, bos, bos_stride_b, bos_stride_n, x_new);
  return check_launch("packed_residual_persist");
}

extern "C" int oudjat_fold_residual_rows(const uint16_t* x, int64_t rows, int64_t C, const int32_t* row_slot,
                                         const uint16_t* x_packed, const uint16_t* const* bos_rows, int64_t n_blocks,
                                         uint16_t* out, oudjat_stream_t stream) {
  OUDJAT_REQUIRE(rows >= 0 && C >= 0 && n_blocks >= 0, OUDJAT_ERR_INVALID_ARGUMENT, "fold_residual_rows: negative size");
  if (rows == 0 || C == 0) return OUDJAT_OK;
  OUDJAT_REQUIRE(x && row_slot && out && (n_blocks == 0 || bos_rows), OUDJAT_ERR_INVALID_ARGUMENT,
                 "fold_residual_rows: null pointer");
  OUDJAT_REQUIRE(C % 8 == 0 && aligned(x, 16) && aligned(out, 16) && (!x_packed || aligned(x_packed, 16)),
                 OUDJAT_ERR_UNSUPPORTED_LAYOUT, "fold_residual_rows: 16-byte aligned rows, C %% 8 == 0");
  OUDJAT_REQUIRE(n_blocks < 4096 && rows * (C / 8) < ((int64_t)1 << 40), OUDJAT_ERR_TOO_LARGE,
                 "fold_residual_rows: too large");
  const int64_t threads = rows * (C / 8);
  fold_residual_rows_kernel<<<(unsigned)cdiv(threads, 256), 256, 0, as_stream(stream)>>>(
      x, rows, C, row_slot, x_packed, bos_rows, (int)n_blocks, out);
  return check_launch("fold_residual_rows");
}

extern "C" int oudjat_fused_layerscale_add(const uint16_t* x, const uint16_t* a, const uint16_t* g, int64_t rows,
                                           int64_t C, uint16_t* o, oudjat_stream_t stream) {
  OUDJAT_REQUIRE(rows >= 0 && C >= 0, OUDJAT_ERR_INVALID_ARGUMENT, "fused_layerscale_add: negative size");
  if (rows == 0 || C == 0) return OUDJAT_OK;
  OUDJAT_REQUIRE(x && a && g && o, OUDJAT_ERR_INVALID_ARGUMENT, "fused_layerscale_add: null pointer");
  OUDJAT_REQUIRE(C % 8 == 0 && aligned(x, 16) && aligned(a, 16) && aligned(g, 16) && aligned(o, 16),
                 OUDJAT_ERR_UNSUPPORTED_LAYOUT, "fused_layerscale_add: 16-byte aligned rows with C %% 8 == 0 required");
  layerscale_add_kernel<<<(unsigned)cdiv(rows, kRowsPerWg), kRowThreads, 0, as_stream(stream)>>>(x, a, g, rows, C, o);
  return check_launch("fused_layerscale_add");
}

extern "C" int oudjat_residual_pair(const uint16_t* inc, const uint16_t* x_attn, const uint16_t* mlp, int64_t rows,
                                    int64_t C, uint16_t* bos, uint16_t* out, oudjat_stream_t stream) {
  OUDJAT_REQUIRE(rows >= 0 && C >= 0, OUDJAT_ERR_INVALID_ARGUMENT, "residual_pair: negative size");
  if (rows == 0 || C == 0) return OUDJAT_OK;
  OUDJAT_REQUIRE(inc && x_attn && mlp && bos && out, OUDJAT_ERR_INVALID_ARGUMENT, "residual_pair: null pointer");
  OUDJAT_REQUIRE(C % 8 == 0 && aligned(inc, 16) && aligned(x_attn, 16) && aligned(mlp, 16) && aligned(bos, 16) &&
                     aligned(out, 16),
                 OUDJAT_ERR_UNSUPPORTED_LAYOUT, "residual_pair: 16-byte aligned rows with C %% 8 == 0 required");
  OUDJAT_REQUIRE(C <= 8192, OUDJAT_ERR_TOO_LARGE, "residual_pair: C=%lld > 8192", (long long)C);
  const unsigned grid = (unsigned)cdiv(rows, kRowsPerWg);
  const hipStream_t st = as_stream(stream);
  if (C <= 512) residual_pair_kernel<1><<<grid, kRowThreads, 0, st>>>(inc, x_attn, mlp, rows, C, bos, out);
  else if (C <= 1024) residual_pair_kernel<2><<<grid, kRowThreads, 0, st>>>(inc, x_attn, mlp, rows, C, bos, out);
  else if (C <= 2048) residual_pair_kernel<4><<<grid, kRowThreads, 0, st>>>(inc, x_attn, mlp, rows, C, bos, out);
  else if (C <= 4096) residual_pair_kernel<8><<<grid, kRowThreads, 0, st>>>(inc, x_attn, mlp, rows, C, bos, out);
  else residual_pair_kernel<16><<<grid, kRowThreads, 0, st>>>(inc, x_attn, mlp, rows, C, bos, out);
  return check_launch("residual_pair");
}

extern "C" int oudjat_patch_importance(const float* d, int64_t rows, int64_t dim, int64_t rs, int mode, float* out,
                                       oudjat_stream_t stream) {
  OUDJAT_REQUIRE(rows >= 0 && dim >= 0, OUDJAT_ERR_INVALID_ARGUMENT, "patch_importance: negative size");
  OUDJAT_REQUIRE(mode >= 0 && mode <= 2, OUDJAT_ERR_INVALID_ARGUMENT, "patch_importance: bad mode %d", mode);
  if (rows == 0) return OUDJAT_OK;
  OUDJAT_REQUIRE(out && (d || dim == 0), OUDJAT_ERR_INVALID_ARGUMENT, "patch_importance: null pointer");
  const bool vec = dim % 4 == 0 && rs % 4 == 0 && aligned(d, 16);
  patch_importance_kernel<<<(unsigned)cdiv(rows, kRowsPerWg), kRowThreads, 0, as_stream(stream)>>>(d, rows, dim, rs,
                                                                                                    mode, vec, out);
  return check_launch("patch_importance");
}
