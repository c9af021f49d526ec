// Activation-side kernels: int4 group-64 quantization (+ fused x @ proj_down),
// int8 per-token quantization, and the standalone SVDQuant epilogue.
#include "gwa_common.h"

// ---------------------------------------------------------------------------
// Kernel 1: smoothing divide -> group-64 absmax -> fp16 scale -> int4 codes,
// packed two per byte; plus la = x @ proj_down on the RAW activations via
// bf16 MFMA 16x16x32.
//
// One wave owns 16 rows. Lane (i = lane % 16, kq = lane / 16) holds, per
// group of 64, the 16 elements of row i at K offsets kq*8 + [0,8) and
// 32 + kq*8 + [0,8): each is one 16-byte load, and the same registers are
// the MFMA A operand for the two 32-wide K halves of the group. The row's
// group absmax is a max over the 4 lanes {i, i+16, i+32, i+48}.
//
// Arithmetic follows the reference order (models/svdq_fused.py:88-103,
// models/nvfp4_quant.py:96-102): xs = bf16(x / smooth) (IEEE fp32 divide,
// RNE); scale = fp16(clamp(amax / (7 * s2), 2^-24, 65504)); codes =
// clamp(rne(xs / (float(scale) * s2)), -8, 7).
// ---------------------------------------------------------------------------
namespace {

constexpr float kScaleMin = 5.9604644775390625e-08f;  // 2^-24, smallest positive fp16
constexpr float kFp16Max = 65504.0f;

__device__ __forceinline__ void unpack8_bf16(v4i w, float* v) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t u = (uint32_t)w[j];
    v[2 * j] = bf16_lo(u);
    v[2 * j + 1] = bf16_hi(u);
  }
}

__device__ __forceinline__ float bf16_round(float f) { return bf16_to_f32(f32_to_bf16(f)); }

__device__ __forceinline__ uint32_t int4_code(float v, float d) {
  float q = __builtin_rintf(v / d);
  q = fminf(fmaxf(q, -8.0f), 7.0f);
  return (uint32_t)((int)q) & 0xFu;
}

template <int RB>
__global__ __launch_bounds__(64) void svdq_quant_int4_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const uint16_t* __restrict__ smooth,
    const float* __restrict__ s2p, const uint16_t* __restrict__ pdt, uint8_t* __restrict__ q,
    uint16_t* __restrict__ sc, uint16_t* __restrict__ la, int M, int K) {
  const int lane = threadIdx.x;
  const int i = lane & 15, kq = lane >> 4;
  const int row0 = blockIdx.x * 16;
  const int row = row0 + i;
  const bool valid = row < M;
  const float s2 = s2p ? *s2p : 1.0f;
  const float den7 = 7.0f * s2;
  const int G = K >> 6;
  const uint16_t* xr = x + (int64_t)(valid ? row : 0) * ldx;
  uint8_t* qr = q + (int64_t)(valid ? row : 0) * (K >> 1);

  v4f acc[RB > 0 ? RB : 1];
#pragma unroll
  for (int rb = 0; rb < (RB > 0 ? RB : 1); ++rb) acc[rb] = (v4f){0.f, 0.f, 0.f, 0.f};

  for (int g = 0; g < G; ++g) {
    const int k0 = g * 64 + kq * 8;
    v4i xa = {0, 0, 0, 0}, xb = {0, 0, 0, 0};
    if (valid) {
      xa = *(const v4i*)(xr + k0);
      xb = *(const v4i*)(xr + k0 + 32);
    }
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const uint16_t* pr = pdt + (int64_t)(rb * 16 + i) * K;
      v4i ba = *(const v4i*)(pr + k0);
      v4i bb = *(const v4i*)(pr + k0 + 32);
      acc[rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, xa),
                                                        __builtin_bit_cast(v8bf, ba), acc[rb], 0, 0, 0);
      acc[rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, xb),
                                                        __builtin_bit_cast(v8bf, bb), acc[rb], 0, 0, 0);
    }

    float v[16];
    unpack8_bf16(xa, v);
    unpack8_bf16(xb, v + 8);
    if (smooth) {
      float sm[16];
      unpack8_bf16(*(const v4i*)(smooth + k0), sm);
      unpack8_bf16(*(const v4i*)(smooth + k0 + 32), sm + 8);
#pragma unroll
      for (int j = 0; j < 16; ++j) v[j] = bf16_round(v[j] / sm[j]);
    }
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) amax = fmaxf(amax, fabsf(v[j]));
    amax = fmaxf(amax, __shfl_xor(amax, 16));
    amax = fmaxf(amax, __shfl_xor(amax, 32));

    float scl = amax / den7;
    scl = fminf(fmaxf(scl, kScaleMin), kFp16Max);
    const uint16_t sh = f32_to_f16_bits(scl);
    const float d = f16_bits_to_f32(sh) * s2;

    uint32_t w0 = 0, w1 = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      w0 |= int4_code(v[j], d) << (4 * j);
      w1 |= int4_code(v[8 + j], d) << (4 * j);
    }
    if (valid) {
      *(uint32_t*)(qr + (k0 >> 1)) = w0;
      *(uint32_t*)(qr + ((k0 + 32) >> 1)) = w1;
      if (kq == 0) sc[(int64_t)row * G + g] = sh;
    }
  }

  if (RB > 0) {
    const int R = RB * 16;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int r = row0 + 4 * kq + t;
        if (r < M) la[(int64_t)r * R + rb * 16 + i] = f32_to_bf16(acc[rb][t]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// int8 per-token quantization: one 256-thread block per row.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void w8a8_quant_int8_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                              int8_t* __restrict__ q, float* __restrict__ sa,
                                                              int M, int K) {
  __shared__ float red[4];
  const int row = blockIdx.x;
  const uint16_t* xr = x + (int64_t)row * ldx;
  int8_t* qr = q + (int64_t)row * K;
  const int nchunk = K >> 3;
  float am = 0.0f;
  for (int c = threadIdx.x; c < nchunk; c += 256) {
    float v[8];
    unpack8_bf16(*(const v4i*)(xr + c * 8), v);
#pragma unroll
    for (int j = 0; j < 8; ++j) am = fmaxf(am, fabsf(v[j]));
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) am = fmaxf(am, __shfl_xor(am, off));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = am;
  __syncthreads();
  am = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float s = fmaxf(am / 127.0f, 1e-12f);
  for (int c = threadIdx.x; c < nchunk; c += 256) {
    float v[8];
    unpack8_bf16(*(const v4i*)(xr + c * 8), v);
    uint32_t w[2] = {0, 0};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float t = __builtin_rintf(v[j] / s);
      t = fminf(fmaxf(t, -127.0f), 127.0f);
      w[j >> 2] |= ((uint32_t)((int)t) & 0xFFu) << (8 * (j & 3));
    }
    *(uint2*)(qr + c * 8) = make_uint2(w[0], w[1]);
  }
  if (threadIdx.x == 0) sa[row] = s;
}

// ---------------------------------------------------------------------------
// standalone epilogue: out = y0 * (s2 * second) + la @ up^T + bias, bf16 out
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void svdq_epilogue_kernel(const uint16_t* __restrict__ y0,
                                                            const uint16_t* __restrict__ la,
                                                            const uint16_t* __restrict__ up, int R,
                                                            const float* __restrict__ s2p,
                                                            const float* __restrict__ second, int per_channel,
                                                            const uint16_t* __restrict__ bias,
                                                            uint16_t* __restrict__ out, int M, int N) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)M * N) return;
  const int m = (int)(idx / N), n = (int)(idx % N);
  const float s2 = s2p ? *s2p : 1.0f;
  const float sec = second ? second[per_channel ? n : 0] : 1.0f;
  float y = bf16_to_f32(y0[idx]) * (s2 * sec);
  float lr = 0.0f;
  for (int r = 0; r < R; ++r) lr = fmaf(bf16_to_f32(la[(int64_t)m * R + r]), bf16_to_f32(up[(int64_t)n * R + r]), lr);
  y += lr;
  if (bias) y += bf16_to_f32(bias[n]);
  out[idx] = f32_to_bf16(y);
}

}  // namespace

extern "C" int gwa_svdq_quant_int4(const void* x, int64_t ldx, const void* smooth, const float* s2,
                                   const void* proj_down_t, int64_t rank, uint8_t* q, void* scales,
                                   void* la, int64_t M, int64_t K, void* stream) {
  GWA_REQUIRE(M >= 0 && K > 0, "svdq_quant_int4: bad shape M=%lld K=%lld", (long long)M, (long long)K);
  GWA_REQUIRE(K % 64 == 0, "svdq_quant_int4: K=%lld is not a multiple of 64", (long long)K);
  GWA_REQUIRE(ldx >= K && ldx % 8 == 0, "svdq_quant_int4: row stride %lld must be >= K and a multiple of 8",
              (long long)ldx);
  GWA_REQUIRE((proj_down_t == nullptr) == (la == nullptr),
              "svdq_quant_int4: proj_down_t and la must both be given or both be NULL");
  const int64_t R = proj_down_t ? rank : 0;
  GWA_REQUIRE(R % 16 == 0 && R <= 128, "svdq_quant_int4: rank %lld must be a multiple of 16 and <= 128",
              (long long)R);
  GWA_REQUIRE(M < (1ll << 31) && K < (1ll << 30), "svdq_quant_int4: shape too large");
  if (M == 0) return GWA_OK;
  GWA_REQUIRE(x && q && scales, "svdq_quant_int4: null pointer");
  GWA_REQUIRE(GWA_ALIGNED(x, 16) && GWA_ALIGNED(q, 16) && GWA_ALIGNED(scales, 2) &&
                  GWA_ALIGNED(smooth, 16) && GWA_ALIGNED(proj_down_t, 16) && GWA_ALIGNED(la, 2),
              "svdq_quant_int4: x, q, smooth and proj_down_t must be 16-byte aligned");
  const dim3 grid((unsigned)((M + 15) / 16)), block(64);
  hipStream_t s = (hipStream_t)stream;
  const uint16_t* xp = (const uint16_t*)x;
  const uint16_t* sm = (const uint16_t*)smooth;
  const uint16_t* pd = (const uint16_t*)proj_down_t;
  uint16_t* sc = (uint16_t*)scales;
  uint16_t* lp = (uint16_t*)la;
  const int m = (int)M, k = (int)K;
#define GWA_QUANT_CASE(RBV)                                                                              \
  case RBV:                                                                                              \
    hipLaunchKernelGGL(svdq_quant_int4_kernel<RBV>, grid, block, 0, s, xp, ldx, sm, s2, pd, q, sc, lp, m, k); \
    break;
  switch (R / 16) {
    GWA_QUANT_CASE(0)
    GWA_QUANT_CASE(1)
    GWA_QUANT_CASE(2)
    GWA_QUANT_CASE(3)
    GWA_QUANT_CASE(4)
    GWA_QUANT_CASE(5)
    GWA_QUANT_CASE(6)
    GWA_QUANT_CASE(7)
    GWA_QUANT_CASE(8)
    default: return gwa_set_error(GWA_ERR_INVALID, "svdq_quant_int4: unsupported rank %lld", (long long)R);
  }
#undef GWA_QUANT_CASE
  return gwa_check_launch("svdq_quant_int4");
}

extern "C" int gwa_w8a8_quant_int8(const void* x, int64_t ldx, int8_t* q, float* sa, int64_t M, int64_t K,
                                   void* stream) {
  GWA_REQUIRE(M >= 0 && K > 0 && K % 8 == 0, "w8a8_quant_int8: bad shape M=%lld K=%lld (K %% 8 == 0)",
              (long long)M, (long long)K);
  GWA_REQUIRE(ldx >= K && ldx % 8 == 0, "w8a8_quant_int8: bad row stride %lld", (long long)ldx);
  GWA_REQUIRE(M < (1ll << 31) && K < (1ll << 30), "w8a8_quant_int8: shape too large");
  if (M == 0) return GWA_OK;
  GWA_REQUIRE(x && q && sa, "w8a8_quant_int8: null pointer");
  GWA_REQUIRE(GWA_ALIGNED(x, 16) && GWA_ALIGNED(q, 8) && GWA_ALIGNED(sa, 4),
              "w8a8_quant_int8: x must be 16-byte and q 8-byte aligned");
  hipLaunchKernelGGL(w8a8_quant_int8_kernel, dim3((unsigned)M), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)x, ldx, q, sa, (int)M, (int)K);
  return gwa_check_launch("w8a8_quant_int8");
}

extern "C" int gwa_svdq_epilogue_lora(const void* y0, const void* la, const void* up, int64_t rank,
                                      const float* s2, const float* second, int64_t second_numel,
                                      const void* bias, void* out, int64_t M, int64_t N, void* stream) {
  GWA_REQUIRE(M >= 0 && N >= 0 && rank >= 0, "svdq_epilogue_lora: bad shape");
  GWA_REQUIRE(second == nullptr || second_numel == 1 || second_numel == N,
              "svdq_epilogue_lora: second has %lld values for N=%lld", (long long)second_numel, (long long)N);
  GWA_REQUIRE(M * N < (1ll << 40), "svdq_epilogue_lora: shape too large");
  if (M == 0 || N == 0) return GWA_OK;
  GWA_REQUIRE(y0 && out && (rank == 0 || (la && up)), "svdq_epilogue_lora: null pointer");
  GWA_REQUIRE(GWA_ALIGNED(y0, 2) && GWA_ALIGNED(out, 2) && GWA_ALIGNED(la, 2) && GWA_ALIGNED(up, 2) &&
                  GWA_ALIGNED(second, 4) && GWA_ALIGNED(s2, 4) && GWA_ALIGNED(bias, 2),
              "svdq_epilogue_lora: misaligned pointer");
  const int64_t total = M * N;
  hipLaunchKernelGGL(svdq_epilogue_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)y0, (const uint16_t*)la, (const uint16_t*)up,
                     (int)rank, s2, second, (int)(second_numel > 1), (const uint16_t*)bias, (uint16_t*)out,
                     (int)M, (int)N);
  return gwa_check_launch("svdq_epilogue_lora");
}
