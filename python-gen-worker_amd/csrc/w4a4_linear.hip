// One SVDQuant W4A4 linear per call on the fp6 lane: kernel 1 (smoothing, int4 group-64 act-quant written
// as fp6 operand records, la = x @ proj_down as fp32 partial slots and their fixed-order reduction to
// bf16) and the W4A4 GEMM with its fused epilogue, enqueued on one stream. The intermediates (records,
// partial slots, bf16 la) live in a workspace the caller passes in; gwa_svdq_w4a4_linear_fp6_workspace gives
// its size.
//
// gwa_svdq_w4a4_linear_fp6_noalloc is the same call for callers that cannot allocate device memory: its
// intermediates live in `scratch`, a fixed-size array of this library's code object (one copy per GPU, held
// until the process ends). Host code never passes the array's name to a kernel: on the host that name is a
// stand-in, not a device address. The device address of each GPU's copy is looked up once per device with
// hipGetSymbolAddress (with that device current) and only that address is used.
#include <mutex>

#include "gwa_common.h"

namespace {

constexpr int64_t kAlign = 256;
constexpr int64_t kRecordSlack = GWA_FP6_RECORD_SLACK;  // the GEMM may read this far past the records

int64_t align_up(int64_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

// workspace layout: [records + slack | la partial slots fp32 (kernel 1's la workspace) | la bf16 [M, R]]
struct Scratch {
  int64_t partials = 0, partial_bytes = 0, la = 0, total = 0;
};

Scratch scratch_layout(int64_t M, int64_t K, int64_t R) {
  Scratch s;
  s.partial_bytes = R ? gwa_svdq_quant_fp6_la_workspace(M, K, R) : 0;
  s.partials = align_up(M * ((K + 127) / 128) * GWA_FP6_REC + kRecordSlack);
  s.la = align_up(s.partials + s.partial_bytes);
  s.total = align_up(s.la + M * R * 2);
  return s;
}

// the weight records' readable bytes, checked before anything is enqueued (the GEMM checks them again)
int check_weight_records(const char* what, const uint8_t* qw6, int64_t qw6_bytes, int64_t N, int64_t K) {
  const int64_t S = (K + 127) / 128;  // K % 128 == 64: a half stage
  GWA_REQUIRE(qw6 != nullptr && qw6_bytes >= S * N * GWA_FP6_REC + kRecordSlack,
              "%s: qw6 has %lld readable bytes, the weight's records need %lld plus %d of slack", what,
              (long long)qw6_bytes, (long long)(S * N * GWA_FP6_REC), GWA_FP6_RECORD_SLACK);
  return GWA_OK;
}

int linear_fp6_run(const char* what, const void* x, int64_t ldx, const void* smooth, const float* s2,
                   const void* proj_down_op6, int64_t rank, const uint8_t* qw6, int64_t qw6_bytes, const float* second,
                   int64_t second_numel, const void* proj_up, const void* bias, void* out, int out_dtype,
                   int epilogue_flags, int64_t M, int64_t N, int64_t K, uint8_t* ws, int64_t ws_bytes, void* stream) {
  GWA_REQUIRE(M >= 0 && N > 0 && K > 0 && K % 64 == 0, "%s: bad shape M=%lld N=%lld K=%lld (K %% 64 == 0)", what,
              (long long)M, (long long)N, (long long)K);
  GWA_REQUIRE((proj_down_op6 == nullptr) == (proj_up == nullptr),
              "%s: proj_down_op6 and proj_up must both be given or both be NULL", what);
  GWA_REQUIRE((epilogue_flags & ~GWA_EPI_GELU_TANH) == 0, "%s: epilogue flags 0x%x (only GWA_EPI_GELU_TANH)", what,
              epilogue_flags);
  const int64_t R = proj_down_op6 ? rank : 0;
  GWA_REQUIRE(R == 0 || R == 16 || R == 32 || R == 64 || R == 128, "%s: rank %lld not in {0,16,32,64,128}", what,
              (long long)R);
  GWA_REQUIRE(M < (1ll << 31) && K < (1ll << 24), "%s: shape too large", what);
  if (M == 0) return GWA_OK;
  const int wrc = check_weight_records(what, qw6, qw6_bytes, N, K);  // before kernel 1 is enqueued
  if (wrc != GWA_OK) return wrc;
  const Scratch s = scratch_layout(M, K, R);
  GWA_REQUIRE(ws != nullptr && ws_bytes >= s.total, "%s: workspace of %lld bytes, this shape needs %lld", what,
              (long long)ws_bytes, (long long)s.total);
  GWA_REQUIRE(GWA_ALIGNED(ws, 256), "%s: workspace must be 256-byte aligned", what);
  uint8_t* la = R ? ws + s.la : nullptr;
  const int rc = R ? gwa_svdq_quant_fp6_la(x, ldx, smooth, s2, proj_down_op6, R, ws, la, (float*)(ws + s.partials),
                                           s.partial_bytes, M, K, stream)
                   : gwa_svdq_quant_fp6(x, ldx, smooth, s2, nullptr, 0, ws, nullptr, M, K, stream);
  if (rc != GWA_OK) return rc;
  // the records' region of the workspace holds the slack the GEMM reads past them
  return gwa_svdq_gemm_w4a4_fp6(ws, s.partials, qw6, qw6_bytes, s2, second, second_numel, la, R ? proj_up : nullptr,
                                R, bias, out, out_dtype, epilogue_flags, M, N, K, stream);
}

}  // namespace

// ---------------------------------------------------------------------------
// zero-allocation variant
// ---------------------------------------------------------------------------
namespace {

constexpr int64_t kScratchBytes = GWA_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint8_t* g_scratch_ptr[kMaxDevices] = {};

// the device address of the current device's copy of `scratch` (looked up on the first call per device)
int current_scratch(const char* what, uint8_t** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return gwa_set_error(GWA_ERR_HIP, "%s: hipGetDevice failed: %s", what, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return gwa_set_error(GWA_ERR_INVALID, "%s: device %d is beyond the %d devices this library tracks", what, dev,
                         kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return gwa_set_error(GWA_ERR_HIP, "%s: hipGetSymbolAddress(scratch) on device %d failed: %s", what, dev,
                           hipGetErrorString(e));
    if (!GWA_ALIGNED(p, 256))
      return gwa_set_error(GWA_ERR_HIP, "%s: scratch on device %d is not 256-byte aligned", what, dev);
    g_scratch_ptr[dev] = (uint8_t*)p;
  }
  *out = g_scratch_ptr[dev];
  return GWA_OK;
}

}  // namespace

extern "C" int gwa_svdq_w4a4_linear_fp6_noalloc(const void* x, int64_t ldx, const void* smooth, const float* s2,
                                                const void* proj_down_op6, int64_t rank, const uint8_t* qw6,
                                                int64_t qw6_bytes, const float* second, int64_t second_numel, const void* proj_up,
                                                const void* bias, void* out, int out_dtype, int epilogue_flags,
                                                int64_t M, int64_t N, int64_t K, void* stream) {
  const char* what = "svdq_w4a4_linear_fp6_noalloc";
  const int64_t need = gwa_svdq_w4a4_linear_fp6_workspace(M, K, proj_down_op6 ? rank : 0);
  GWA_REQUIRE(need <= kScratchBytes,
              "%s: M=%lld K=%lld rank=%lld needs %lld bytes of scratch; the library's static scratch holds %lld "
              "(use gwa_svdq_w4a4_linear_fp6 with a workspace, or split the rows)",
              what, (long long)M, (long long)K, (long long)rank, (long long)need, (long long)kScratchBytes);
  uint8_t* ws = nullptr;
  if (M > 0 && N > 0 && K > 0 && K % 64 == 0) {
    const int wrc = check_weight_records(what, qw6, qw6_bytes, N, K);  // before the scratch lookup's HIP calls
    if (wrc != GWA_OK) return wrc;
  }
  if (M > 0) {
    const int rc = current_scratch(what, &ws);
    if (rc != GWA_OK) return rc;
  }
  return linear_fp6_run(what, x, ldx, smooth, s2, proj_down_op6, rank, qw6, qw6_bytes, second, second_numel, proj_up,
                        bias, out, out_dtype, epilogue_flags, M, N, K, ws, kScratchBytes, stream);
}

extern "C" int64_t gwa_svdq_w4a4_linear_fp6_noalloc_scratch_bytes(void) { return kScratchBytes; }

extern "C" int64_t gwa_svdq_w4a4_linear_fp6_workspace(int64_t M, int64_t K, int64_t rank) {
  if (M <= 0 || K <= 0 || K % 64 || M >= (1ll << 31) || K >= (1ll << 24)) return 0;
  if (rank != 0 && rank != 16 && rank != 32 && rank != 64 && rank != 128) return 0;
  return scratch_layout(M, K, rank).total;
}

extern "C" int gwa_svdq_w4a4_linear_fp6(const void* x, int64_t ldx, const void* smooth, const float* s2,
                                        const void* proj_down_op6, int64_t rank, const uint8_t* qw6,
                                        int64_t qw6_bytes, const float* second, int64_t second_numel, const void* proj_up,
                                        const void* bias, void* out, int out_dtype, int epilogue_flags, int64_t M,
                                        int64_t N, int64_t K, void* workspace, int64_t workspace_bytes,
                                        void* stream) {
  return linear_fp6_run("svdq_w4a4_linear_fp6", x, ldx, smooth, s2, proj_down_op6, rank, qw6, qw6_bytes, second,
                        second_numel, proj_up, bias, out, out_dtype, epilogue_flags, M, N, K, (uint8_t*)workspace,
                        workspace_bytes, stream);
}
