// AWQ W4A16 linear for the M = 1 (or few-token) modulation layers: bf16
// activations times group-64 asymmetric uint4 weights.
//
// Weight layout (the reference's packed-resident buffers,
// models/svdq_awq_packed.py:181-196 and :240-243): weight uint8 [N, K/2],
// code of column 2j in the LOW nibble of byte j, codes 0..15; wscales and
// wzeros bf16 [N, K/64] (zeros pre-scaled and pre-negated on disk, so the
// dequantized weight is an ADD: w = code * s + z).
//
// Arithmetic = the reference's (models/svdq_awq_packed.py:70-93, and the
// decode path models/svdq_awq.py:74-82): w = RN_bf16(code * s + z) with the
// product exact in fp32 (4-bit code times 8-bit significand) and the sum
// rounded once in fp32, so one fma gives the same value as the reference's
// multiply-then-add; y[m, n] = sum_k w[n, k] * x[m, k] in fp32, + bias in
// fp32, rounded to bf16.
//
// The layer is bound by the weight read (N * K / 2 bytes + the two scale
// grids); every weight byte is read once per MT activation rows:
//  * a workgroup stages MT activation rows in LDS (bf16) and owns 16 output
//    rows, one per 16-lane team; lane t of a team takes the 32 codes
//    [512 s + 32 t, +32) of span s (16 weight bytes, one coalesced 256-byte
//    segment per team and span: half a group) and that group's scale and zero;
//  * each 8 codes become four bf16 pairs (nibble split, byte-to-float
//    conversion, one fma each, one v_cvt_pk_bf16_f32 per pair) and each pair
//    meets the matching activation pair in one v_dot2c_f32_bf16 per
//    activation row (fp32 accumulation), the activations read as 16 bytes
//    per lane from LDS, swizzled so the 16 lanes of a team hit distinct banks;
//  * the first batch of 4 spans is requested before the activations are
//    staged, later batches as the previous one is consumed; the team's 16
//    partial sums are reduced by lane exchanges, and lane 0 adds the bias and
//    stores the bf16 result.
// A second kernel dequantizes the whole weight to bf16 [N, K] (the same
// values) for callers with many activation rows, which then run a library
// GEMM.
#include "gwa_common.h"

namespace {

constexpr int AWQ_THREADS = 256, AWQ_TEAMS = AWQ_THREADS / 16;  // 16 output rows per workgroup
constexpr int AWQ_SPAN = 512;                                    // codes of a row per team step (16 lanes x 32)
constexpr int AWQ_BATCH = 4;                                     // spans per load batch
constexpr int AWQ_LDS_MAX = 64 * 1024;                           // activation rows staged in LDS

typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

// eight codes (one dword: code 2b in the low nibble of byte b) of one group -> four bf16 pairs (w_2b, w_2b+1)
__device__ __forceinline__ void dequant8(uint32_t d, float s, float z, uint32_t (&w)[4]) {
  uint32_t lo = d & 0x0F0F0F0Fu, hi = (d >> 4) & 0x0F0F0F0Fu;
  // (float)(byte b) compiles to one v_cvt_f32_ubyte<b> (the empty asm hides the nibble masks, which would
  // otherwise turn each byte into a 4-bit field extract plus a conversion)
  asm("" : "+v"(lo), "+v"(hi));
  const float l0 = (float)(lo & 0xFFu), h0 = (float)(hi & 0xFFu);
  const float l1 = (float)((lo >> 8) & 0xFFu), h1 = (float)((hi >> 8) & 0xFFu);
  const float l2 = (float)((lo >> 16) & 0xFFu), h2 = (float)((hi >> 16) & 0xFFu);
  const float l3 = (float)(lo >> 24), h3 = (float)(hi >> 24);
  w[0] = pack_bf16x2_rn(fmaf(l0, s, z), fmaf(h0, s, z));
  w[1] = pack_bf16x2_rn(fmaf(l1, s, z), fmaf(h1, s, z));
  w[2] = pack_bf16x2_rn(fmaf(l2, s, z), fmaf(h2, s, z));
  w[3] = pack_bf16x2_rn(fmaf(l3, s, z), fmaf(h3, s, z));
}

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2bf, a), __builtin_bit_cast(v2bf, b), c, false);
}

// 16-byte unit u of a staged activation row lives at unit u ^ ((u >> 4) & 3): the four 16-byte reads
// of a lane's 64 bytes (units 4t + i of a span, lanes t = 0..15) then hit 16 distinct bank groups
__device__ __forceinline__ int x_unit(int u) { return u ^ ((u >> 4) & 3); }

template <int MT>
__global__ __launch_bounds__(AWQ_THREADS) void awq_w4a16_gemv_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const uint8_t* __restrict__ weight,
    const uint16_t* __restrict__ wscales, const uint16_t* __restrict__ wzeros, const uint16_t* __restrict__ bias,
    uint16_t* __restrict__ out, int M, int N, int K) {
  extern __shared__ __attribute__((aligned(16))) uint8_t awq_lds[];
  const int tid = threadIdx.x;
  const int m0 = blockIdx.y * MT;
  const int ku = K >> 3;  // 16-byte units of one activation row

  // team (16 lanes) -> output row n; lane t -> codes [512 s + 32 t, +32) of every span s (half a group)
  const int team = tid >> 4, t = tid & 15;
  const int n = blockIdx.x * AWQ_TEAMS + team;
  const bool row_ok = n < N;
  const int spans = (K + AWQ_SPAN - 1) / AWQ_SPAN, ng = K >> 6;
  const rsrc_t wbuf = make_rsrc(weight, (uint32_t)((int64_t)N * (K >> 1)));
  const rsrc_t sbuf = make_rsrc(wscales, (uint32_t)((int64_t)N * ng * 2));
  const rsrc_t zbuf = make_rsrc(wzeros, (uint32_t)((int64_t)N * ng * 2));
  const uint32_t wrow = (uint32_t)((int64_t)n * (K >> 1)) + 16u * (uint32_t)t;
  const uint32_t grow = (uint32_t)((int64_t)n * ng + (t >> 1)) * 2u;

  v4i wd[AWQ_BATCH];
  uint16_t sc[AWQ_BATCH], ze[AWQ_BATCH];
  auto load_batch = [&](int s0) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < AWQ_BATCH; ++j) {
      const bool ok = row_ok && (s0 + j) * AWQ_SPAN + 32 * t < K;
      wd[j] = buf_load16(wbuf, ok ? wrow + (uint32_t)(AWQ_SPAN / 2) * (uint32_t)(s0 + j) : kOOB);
      sc[j] = buf_load2(sbuf, ok ? grow + 16u * (uint32_t)(s0 + j) : kOOB);
      ze[j] = buf_load2(zbuf, ok ? grow + 16u * (uint32_t)(s0 + j) : kOOB);
    }
  };
  // 1. the first batch of weights goes out before the activations are staged (its latency covers theirs)
  load_batch(0);

  // 2. the MT activation rows into LDS (rows past M: zeros), units swizzled by x_unit
  {
    const rsrc_t xbuf = make_rsrc(x, (uint32_t)(((int64_t)(M - 1) * ldx + K) * 2));
    for (int u = tid; u < MT * ku; u += AWQ_THREADS) {
      const int r = u / ku, c = u - r * ku;
      const v4i v = buf_load16(xbuf, m0 + r < M ? (uint32_t)(((int64_t)(m0 + r) * ldx + 8 * c) * 2) : kOOB);
      *(v4i*)(awq_lds + 16 * (r * ku + x_unit(c))) = v;
    }
  }
  __syncthreads();

  // 3. batches of spans: dequantize 32 codes, dot them with every activation row
  float acc[MT];
#pragma unroll
  for (int r = 0; r < MT; ++r) acc[r] = 0.0f;
  for (int s0 = 0; s0 < spans; s0 += AWQ_BATCH) {
    if (s0) load_batch(s0);
#pragma unroll
    for (int j = 0; j < AWQ_BATCH; ++j) {
      if ((s0 + j) * AWQ_SPAN + 32 * t >= K) continue;  // past the row (K % 512 != 0)
      const float sv = bf16_to_f32(sc[j]), zv = bf16_to_f32(ze[j]);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint32_t w[4];
        dequant8((uint32_t)wd[j][q], sv, zv, w);
        const int unit = x_unit(64 * (s0 + j) + 4 * t + q);  // activation columns 512 s + 32 t + 8 q .. +8
#pragma unroll
        for (int r = 0; r < MT; ++r) {
          const v4i xv = *(const v4i*)(awq_lds + 16 * (r * ku + unit));
#pragma unroll
          for (int b = 0; b < 4; ++b) acc[r] = dot2_bf16(w[b], (uint32_t)xv[b], acc[r]);
        }
      }
    }
  }
  // 4. team sum (lanes t ^ 8, 4, 2, 1), bias, bf16
  const float bv = (bias && row_ok) ? bf16_to_f32(bias[n]) : 0.0f;
#pragma unroll
  for (int r = 0; r < MT; ++r) {
    float v = acc[r];
    v += __shfl_xor(v, 8, 16);
    v += __shfl_xor(v, 4, 16);
    v += __shfl_xor(v, 2, 16);
    v += __shfl_xor(v, 1, 16);
    if (t == 0 && row_ok && m0 + r < M) out[(int64_t)(m0 + r) * N + n] = f32_to_bf16(v + bv);
  }
}

// weight [N, K/2] + scales / zeros [N, K/64] -> bf16 [N, K]: one dword of codes (8 columns) per thread
__global__ __launch_bounds__(256) void awq_w4a16_dequant_kernel(const uint32_t* __restrict__ weight,
                                                                 const uint16_t* __restrict__ wscales,
                                                                 const uint16_t* __restrict__ wzeros,
                                                                 uint16_t* __restrict__ out, int64_t N, int K) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // dword index
  const int per_row = K >> 3;
  if (i >= N * per_row) return;
  const int64_t n = i / per_row;
  const int c = (int)(i - n * per_row);
  const int64_t g = n * (K >> 6) + (c >> 3);
  uint32_t w[4];
  dequant8(weight[i], bf16_to_f32(wscales[g]), bf16_to_f32(wzeros[g]), w);
  *(v4i*)(out + 8 * i) = (v4i){(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
}

template <int MT>
int launch_gemv(const void* x, int64_t ldx, const void* weight, const void* ws, const void* wz, const void* bias,
                void* out, int64_t M, int64_t N, int64_t K, hipStream_t st) {
  const size_t lds = (size_t)MT * (size_t)K * 2;
  const dim3 grid((unsigned)((N + AWQ_TEAMS - 1) / AWQ_TEAMS), (unsigned)((M + MT - 1) / MT));
  hipLaunchKernelGGL((awq_w4a16_gemv_kernel<MT>), grid, dim3(AWQ_THREADS), lds, st, (const uint16_t*)x, ldx,
                     (const uint8_t*)weight, (const uint16_t*)ws, (const uint16_t*)wz, (const uint16_t*)bias,
                     (uint16_t*)out, (int)M, (int)N, (int)K);
  return gwa_check_launch("awq_w4a16_mm");
}

}  // namespace

extern "C" int gwa_awq_w4a16_mm(const void* x, int64_t ldx, const void* weight, const void* wscales,
                                const void* wzeros, const void* bias, void* out, int64_t M, int64_t N, int64_t K,
                                void* stream) {
  const char* what = "awq_w4a16_mm";
  GWA_REQUIRE(M >= 0 && N > 0 && K > 0 && N % 16 == 0 && K % 128 == 0,
              "%s: [N=%lld, K=%lld] breaks the packed contract (N %% 16, K %% 128)", what, (long long)N,
              (long long)K);
  GWA_REQUIRE(ldx >= K && ldx % 8 == 0, "%s: row stride %lld must be >= K and a multiple of 8", what,
              (long long)ldx);
  GWA_REQUIRE(K * 2 <= AWQ_LDS_MAX, "%s: K=%lld exceeds %d (one activation row staged in LDS)", what,
              (long long)K, AWQ_LDS_MAX / 2);
  GWA_REQUIRE(M < (1ll << 31) && N * K / 2 < (1ll << 31) && M * ldx * 2 < (1ll << 31) && M * N < (1ll << 31),
              "%s: operands must stay below 2 GiB (buffer addressing)", what);
  if (M == 0) return GWA_OK;
  GWA_REQUIRE(x && weight && wscales && wzeros && out, "%s: null pointer", what);
  GWA_REQUIRE(GWA_ALIGNED(x, 16) && GWA_ALIGNED(weight, 4) && GWA_ALIGNED(wscales, 2) && GWA_ALIGNED(wzeros, 2) &&
                  GWA_ALIGNED(bias, 2) && GWA_ALIGNED(out, 2),
              "%s: x must be 16-byte and weight 4-byte aligned", what);
  hipStream_t st = (hipStream_t)stream;
  // activation rows per workgroup: up to 4, as many as fit the LDS budget
  int mt = M == 1 ? 1 : (M == 2 ? 2 : 4);
  while (mt > 1 && (int64_t)mt * K * 2 > AWQ_LDS_MAX) mt /= 2;
  if (mt == 1) return launch_gemv<1>(x, ldx, weight, wscales, wzeros, bias, out, M, N, K, st);
  if (mt == 2) return launch_gemv<2>(x, ldx, weight, wscales, wzeros, bias, out, M, N, K, st);
  return launch_gemv<4>(x, ldx, weight, wscales, wzeros, bias, out, M, N, K, st);
}

extern "C" int gwa_awq_w4a16_dequant(const void* weight, const void* wscales, const void* wzeros, void* out,
                                     int64_t N, int64_t K, void* stream) {
  const char* what = "awq_w4a16_dequant";
  GWA_REQUIRE(N > 0 && K > 0 && K % 64 == 0 && N * K < (1ll << 40), "%s: bad shape [N=%lld, K=%lld]", what,
              (long long)N, (long long)K);
  GWA_REQUIRE(weight && wscales && wzeros && out, "%s: null pointer", what);
  GWA_REQUIRE(GWA_ALIGNED(weight, 4) && GWA_ALIGNED(wscales, 2) && GWA_ALIGNED(wzeros, 2) && GWA_ALIGNED(out, 16),
              "%s: weight must be 4-byte and out 16-byte aligned", what);
  const int64_t dwords = N * (K / 8);
  hipLaunchKernelGGL(awq_w4a16_dequant_kernel, dim3((unsigned)((dwords + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, (const uint32_t*)weight, (const uint16_t*)wscales,
                     (const uint16_t*)wzeros, (uint16_t*)out, N, (int)K);
  return gwa_check_launch(what);
}
