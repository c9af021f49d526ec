// Error state, build info, the probe op and layout transposes.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "gwa_common.h"

#ifndef GWA_BUILD_DESC
#define GWA_BUILD_DESC "archs=gfx950"
#endif

static thread_local char g_last_error[512] = "";

int gwa_set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int gwa_check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return gwa_set_error(GWA_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return GWA_OK;
}

extern "C" int gwa_version(void) { return 1; }

extern "C" const char* gwa_build_info(void) {
  static char buf[256];
  snprintf(buf, sizeof(buf), "gen_worker_amd %s hip=%d.%d", GWA_BUILD_DESC, HIP_VERSION_MAJOR,
           HIP_VERSION_MINOR);
  return buf;
}

extern "C" const char* gwa_last_error(void) { return g_last_error; }

// ---------------------------------------------------------------------------
// debug build: every translation unit's violation word (gwa_common.h)
// ---------------------------------------------------------------------------
#ifdef GWA_DEBUG
namespace {
constexpr int kDbgMaxTus = 32;
int (*g_dbg_readers[kDbgMaxTus])(uint32_t*, uint64_t*, int);
int g_dbg_count = 0;
}  // namespace

// called from static initialisers (one per translation unit, before any entry point runs)
int gwa_dbg_register(int (*reader)(uint32_t*, uint64_t*, int)) {
  if (g_dbg_count < kDbgMaxTus) g_dbg_readers[g_dbg_count++] = reader;
  return g_dbg_count;
}
#endif

extern "C" int gwa_debug_violations(uint32_t* bits, uint64_t* first, int clear) {
#ifdef GWA_DEBUG
  GWA_REQUIRE(bits && first, "debug_violations: null pointer");
  *bits = 0;
  *first = 0;
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return gwa_set_error(GWA_ERR_HIP, "debug_violations: %s", hipGetErrorString(e));
  for (int i = 0; i < g_dbg_count; ++i) {
    const int rc = g_dbg_readers[i](bits, first, clear);
    if (rc != GWA_OK) return gwa_set_error(rc, "debug_violations: reading a violation word failed");
  }
  return GWA_OK;
#else
  (void)bits;
  (void)first;
  (void)clear;
  return gwa_set_error(GWA_ERR_INVALID, "debug_violations: not a debug build (compile with GWA_DEBUG)");
#endif
}

// ---------------------------------------------------------------------------
// probe: out = in + 1
// ---------------------------------------------------------------------------
__global__ void gwa_add_one_kernel(const float* __restrict__ in, float* __restrict__ out, int64_t n) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = in[i] + 1.0f;
}

extern "C" int gwa_probe_add_one(const float* in, float* out, int64_t n, void* stream) {
  GWA_REQUIRE(n >= 0, "probe_add_one: negative size %lld", (long long)n);
  if (n == 0) return GWA_OK;
  GWA_REQUIRE(in && out, "probe_add_one: null pointer");
  GWA_REQUIRE(GWA_ALIGNED(in, 4) && GWA_ALIGNED(out, 4), "probe_add_one: misaligned pointer");
  const int threads = 256;
  const int64_t blocks = (n + threads - 1) / threads;
  GWA_REQUIRE(blocks < (1ll << 31), "probe_add_one: n=%lld too large", (long long)n);
  hipLaunchKernelGGL(gwa_add_one_kernel, dim3((unsigned)blocks), dim3(threads), 0,
                     (hipStream_t)stream, in, out, n);
  return gwa_check_launch("probe_add_one");
}

// ---------------------------------------------------------------------------
// 2-D transpose through a 32x32 LDS tile
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void gwa_transpose_kernel(const T* __restrict__ src, T* __restrict__ dst,
                                                            int64_t rows, int64_t cols) {
  __shared__ T tile[32][33];
  const int64_t c0 = (int64_t)blockIdx.x * 32, r0 = (int64_t)blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
  for (int j = ty; j < 32; j += 8) {
    int64_t r = r0 + j, c = c0 + tx;
    if (r < rows && c < cols) tile[j][tx] = src[r * cols + c];
  }
  __syncthreads();
  for (int j = ty; j < 32; j += 8) {
    int64_t c = c0 + j, r = r0 + tx;
    if (r < rows && c < cols) dst[c * rows + r] = tile[tx][j];
  }
}

extern "C" int gwa_transpose_2d(const void* src, void* dst, int64_t rows, int64_t cols,
                                int64_t elem_size, void* stream) {
  GWA_REQUIRE(rows >= 0 && cols >= 0, "transpose_2d: negative shape");
  if (rows == 0 || cols == 0) return GWA_OK;
  GWA_REQUIRE(src && dst, "transpose_2d: null pointer");
  GWA_REQUIRE(GWA_ALIGNED(src, elem_size) && GWA_ALIGNED(dst, elem_size), "transpose_2d: misaligned pointer");
  GWA_REQUIRE((cols + 31) / 32 < (1ll << 31) && (rows + 31) / 32 < 65536,
              "transpose_2d: shape [%lld, %lld] too large", (long long)rows, (long long)cols);
  dim3 grid((unsigned)((cols + 31) / 32), (unsigned)((rows + 31) / 32));
  hipStream_t s = (hipStream_t)stream;
  switch (elem_size) {
    case 1: hipLaunchKernelGGL(gwa_transpose_kernel<uint8_t>, grid, dim3(256), 0, s,
                               (const uint8_t*)src, (uint8_t*)dst, rows, cols); break;
    case 2: hipLaunchKernelGGL(gwa_transpose_kernel<uint16_t>, grid, dim3(256), 0, s,
                               (const uint16_t*)src, (uint16_t*)dst, rows, cols); break;
    case 4: hipLaunchKernelGGL(gwa_transpose_kernel<uint32_t>, grid, dim3(256), 0, s,
                               (const uint32_t*)src, (uint32_t*)dst, rows, cols); break;
    default: return gwa_set_error(GWA_ERR_INVALID, "transpose_2d: elem_size %lld not in {1,2,4}",
                                  (long long)elem_size);
  }
  return gwa_check_launch("transpose_2d");
}
