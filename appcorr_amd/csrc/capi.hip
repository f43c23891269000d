// Status plumbing, ABI version and the runtime self-test.
#include "common.hpp"

#define OUDJAT_ABI_VERSION 18

namespace oudjat {

static thread_local char g_last_error[1024] = "";

int set_error(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return status;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(OUDJAT_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return OUDJAT_OK;
}

__global__ void selftest_kernel(const float* x, float* y, int n) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = 2.0f * x[i];
}

}  // namespace oudjat

using namespace oudjat;

extern "C" int oudjat_abi_version(void) { return OUDJAT_ABI_VERSION; }

extern "C" const char* oudjat_status_string(int status) {
  switch (status) {
    case OUDJAT_OK: return "ok";
    case OUDJAT_ERR_INVALID_ARGUMENT: return "invalid argument";
    case OUDJAT_ERR_UNSUPPORTED_SHAPE: return "unsupported shape";
    case OUDJAT_ERR_UNSUPPORTED_LAYOUT: return "unsupported layout";
    case OUDJAT_ERR_TOO_LARGE: return "too large";
    case OUDJAT_ERR_LAUNCH: return "kernel launch failed";
    case OUDJAT_ERR_HIP: return "HIP runtime error";
    default: return "unknown status";
  }
}

extern "C" const char* oudjat_last_error(void) { return g_last_error; }

extern "C" int oudjat_selftest(oudjat_stream_t stream) {
  const int n = 8;
  float hx[n], hy[n];
  for (int i = 0; i < n; ++i) hx[i] = (float)i - 3.5f;
  float* d = nullptr;
  hipError_t e = hipMalloc(&d, 2 * n * sizeof(float));
  if (e != hipSuccess) return set_error(OUDJAT_ERR_HIP, "selftest: hipMalloc: %s", hipGetErrorString(e));
  hipStream_t s = as_stream(stream);
  int status = OUDJAT_OK;
  e = hipMemcpyAsync(d, hx, n * sizeof(float), hipMemcpyHostToDevice, s);
  if (e == hipSuccess) {
    selftest_kernel<<<1, 64, 0, s>>>(d, d + n, n);
    status = check_launch("selftest");
    if (status == OUDJAT_OK) {
      e = hipMemcpyAsync(hy, d + n, n * sizeof(float), hipMemcpyDeviceToHost, s);
      if (e == hipSuccess) e = hipStreamSynchronize(s);
    }
  }
  if (status == OUDJAT_OK && e != hipSuccess)
    status = set_error(OUDJAT_ERR_HIP, "selftest: %s", hipGetErrorString(e));
  (void)hipFree(d);
  if (status != OUDJAT_OK) return status;
  for (int i = 0; i < n; ++i)
    if (hy[i] != 2.0f * hx[i]) return set_error(OUDJAT_ERR_HIP, "selftest: wrong result at %d: %f", i, hy[i]);
  // Library set-up on this device: the address of the no-alloc entry point's scratch array.
  return noalloc_scratch(nullptr);
}
