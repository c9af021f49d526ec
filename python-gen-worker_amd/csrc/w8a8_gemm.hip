// W8A8 GEMM: int8 MFMA 32x32x32 with int32 accumulation over the whole K and
// the fp32 epilogue acc * sa * sw[n] + bias[n] of torch._scaled_mm: per-token
// activation scales in the rowwise mode (models/w8a8.py:374-378), one scalar in
// the pertensor mode (:366-372, whose weight scale and bias the reference
// applies as two further bf16 ops; here they are fused in fp32).
//
// Same orientation as the W4A4 kernel: A operand = weight rows (n), B operand
// = activation rows (m); accumulator block D[n][m], lane l holds m = l % 32
// and n = 8*(v/4) + 4*(l/32) + (v%4).
#include "gwa_common.h"

namespace {

constexpr int TILE = 128;
constexpr int KT = 128;                 // int8 bytes (= K elements) per row per stage
constexpr int LDS_STRIDE = KT + 16;
constexpr int LDS_TILE = TILE * LDS_STRIDE;
constexpr int LOADS = TILE * KT / 16 / 256;

template <int BIAS_DT, bool OUT_F16>  // BIAS_DT: -1 none, else GWA_DT_*
__global__ __launch_bounds__(256) void w8a8_gemm_kernel(const int8_t* __restrict__ qa,
                                                        const int8_t* __restrict__ qw,
                                                        const float* __restrict__ sa,
                                                        const float* __restrict__ sw,
                                                        const void* __restrict__ bias,
                                                        uint16_t* __restrict__ out, int M, int N, int K,
                                                        int sa_row) {
  __shared__ __attribute__((aligned(16))) uint8_t lds_w[2][LDS_TILE];
  __shared__ __attribute__((aligned(16))) uint8_t lds_x[2][LDS_TILE];

  const int tiles_n = (N + TILE - 1) / TILE;
  const int tn = blockIdx.x % tiles_n, tm = blockIdx.x / tiles_n;
  const int n0 = tn * TILE, m0 = tm * TILE;
  const int nstages = (K + KT - 1) / KT;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int wn = wave & 1, wm = wave >> 1;
  const int r32 = lane & 31, h = lane >> 5;
  const int t = threadIdx.x;

  v16i acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) acc[a][b] = (v16i){};

  v4i rw[LOADS], rx[LOADS];
  auto load = [&](int stage) {
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
      const int idx = t + j * 256;
      const int row = idx / (KT / 16), c = idx % (KT / 16);
      const int kb = stage * KT + c * 16;
      const bool kin = kb < K;
      rw[j] = (n0 + row < N && kin) ? *(const v4i*)(qw + (int64_t)(n0 + row) * K + kb) : (v4i){0, 0, 0, 0};
      rx[j] = (m0 + row < M && kin) ? *(const v4i*)(qa + (int64_t)(m0 + row) * K + kb) : (v4i){0, 0, 0, 0};
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
      const int idx = t + j * 256;
      const int row = idx / (KT / 16), c = idx % (KT / 16);
      *(v4i*)(lds_w[buf] + row * LDS_STRIDE + c * 16) = rw[j];
      *(v4i*)(lds_x[buf] + row * LDS_STRIDE + c * 16) = rx[j];
    }
  };

  load(0);
  store(0);
  __syncthreads();
  for (int st = 0; st < nstages; ++st) {
    const int buf = st & 1;
    if (st + 1 < nstages) load(st + 1);
    const uint8_t* lw = lds_w[buf];
    const uint8_t* lx = lds_x[buf];
#pragma unroll
    for (int ks = 0; ks < KT / 32; ++ks) {
      v4i a[2], b[2];
#pragma unroll
      for (int bn = 0; bn < 2; ++bn)
        a[bn] = *(const v4i*)(lw + (64 * wn + 32 * bn + r32) * LDS_STRIDE + ks * 32 + 16 * h);
#pragma unroll
      for (int bm = 0; bm < 2; ++bm)
        b[bm] = *(const v4i*)(lx + (64 * wm + 32 * bm + r32) * LDS_STRIDE + ks * 32 + 16 * h);
#pragma unroll
      for (int bn = 0; bn < 2; ++bn)
#pragma unroll
        for (int bm = 0; bm < 2; ++bm)
          acc[bn][bm] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[bn], b[bm], acc[bn][bm], 0, 0, 0);
    }
    if (st + 1 < nstages) store(buf ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int bn = 0; bn < 2; ++bn) {
    const int nb = n0 + 64 * wn + 32 * bn;
#pragma unroll
    for (int bm = 0; bm < 2; ++bm) {
      const int m = m0 + 64 * wm + 32 * bm + r32;
      if (m >= M) continue;
      const float am = sa[sa_row ? m : 0];
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        const int n = nb + 8 * qd + 4 * h;
        if (n >= N) continue;
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float y = (float)acc[bn][bm][4 * qd + e] * am * sw[n + e];
          if (BIAS_DT == GWA_DT_F32) y += ((const float*)bias)[n + e];
          if (BIAS_DT == GWA_DT_BF16) y += bf16_to_f32(((const uint16_t*)bias)[n + e]);
          if (BIAS_DT == GWA_DT_F16) y += f16_bits_to_f32(((const uint16_t*)bias)[n + e]);
          o[e] = y;
        }
        uint2 pk;
        if (OUT_F16) {
          pk.x = pack_f16x2(o[0], o[1]);
          pk.y = pack_f16x2(o[2], o[3]);
        } else {
          pk.x = pack_bf16x2(o[0], o[1]);
          pk.y = pack_bf16x2(o[2], o[3]);
        }
        *(uint2*)(out + (int64_t)m * N + n) = pk;
      }
    }
  }
}

}  // namespace

extern "C" int gwa_w8a8_gemm(const int8_t* qa, const int8_t* qw, const float* sa, int64_t sa_numel,
                             const float* sw, const void* bias, int bias_dtype, void* out, int out_dtype, int64_t M,
                             int64_t N, int64_t K, void* stream) {
  GWA_REQUIRE(M >= 0 && N > 0 && K > 0, "w8a8_gemm: bad shape M=%lld N=%lld K=%lld", (long long)M, (long long)N,
              (long long)K);
  GWA_REQUIRE(K % 64 == 0, "w8a8_gemm: K=%lld is not a multiple of 64", (long long)K);
  GWA_REQUIRE(N % 16 == 0, "w8a8_gemm: N=%lld is not a multiple of 16", (long long)N);
  GWA_REQUIRE(out_dtype == GWA_DT_BF16 || out_dtype == GWA_DT_F16, "w8a8_gemm: out_dtype %d not bf16/f16",
              out_dtype);
  GWA_REQUIRE(bias == nullptr || bias_dtype == GWA_DT_BF16 || bias_dtype == GWA_DT_F16 || bias_dtype == GWA_DT_F32,
              "w8a8_gemm: bias_dtype %d", bias_dtype);
  GWA_REQUIRE(M < (1ll << 31) && N < (1ll << 30) && K < (1ll << 30), "w8a8_gemm: shape too large");
  if (M == 0) return GWA_OK;
  GWA_REQUIRE(sa_numel == 1 || sa_numel == M, "w8a8_gemm: sa has %lld values for M=%lld (1 or M)",
              (long long)sa_numel, (long long)M);
  GWA_REQUIRE(qa && qw && sa && sw && out, "w8a8_gemm: null pointer");
  GWA_REQUIRE(GWA_ALIGNED(qa, 16) && GWA_ALIGNED(qw, 16) && GWA_ALIGNED(out, 8) && GWA_ALIGNED(sa, 4) &&
                  GWA_ALIGNED(sw, 4) && GWA_ALIGNED(bias, 2),
              "w8a8_gemm: qa/qw must be 16-byte and out 8-byte aligned");
  const int64_t tiles = ((M + TILE - 1) / TILE) * ((N + TILE - 1) / TILE);
  GWA_REQUIRE(tiles < (1ll << 31), "w8a8_gemm: too many tiles");
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)tiles), block(256);
  const bool f16 = out_dtype == GWA_DT_F16;
  uint16_t* op = (uint16_t*)out;
  const int m = (int)M, n = (int)N, k = (int)K, sr = sa_numel == M && M > 1 ? 1 : 0;
#define GWA_W8A8_LAUNCH(BD)                                                                                   \
  do {                                                                                                        \
    if (f16) hipLaunchKernelGGL((w8a8_gemm_kernel<BD, true>), grid, block, 0, s, qa, qw, sa, sw, bias, op, m, n, k, sr); \
    else hipLaunchKernelGGL((w8a8_gemm_kernel<BD, false>), grid, block, 0, s, qa, qw, sa, sw, bias, op, m, n, k, sr);    \
  } while (0)
  if (!bias) GWA_W8A8_LAUNCH(-1);
  else if (bias_dtype == GWA_DT_F32) GWA_W8A8_LAUNCH(GWA_DT_F32);
  else if (bias_dtype == GWA_DT_BF16) GWA_W8A8_LAUNCH(GWA_DT_BF16);
  else GWA_W8A8_LAUNCH(GWA_DT_F16);
#undef GWA_W8A8_LAUNCH
  return gwa_check_launch("w8a8_gemm");
}
