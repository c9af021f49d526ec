// nvfp4 compatibility lane: the reference's modelopt nvfp4 W4A4 contract
// (e2m1 codes, e4m3 scales per block of 16 along K, a second-level fp32
// scale) on MI355X. CDNA4's block-scaled MFMA takes E8M0 scales per 32
// elements, not e4m3 per 16, and a dequantized value code * scale has up to
// 6 significant bits, more than any MX element format holds; it is exact in
// bf16. So the lane quantizes activations exactly as the reference does and
// runs the product on the exact bf16 values (a plain library GEMM).
//
// Activation quantization = quantize_activation_torch
// (models/nvfp4_quant.py:92-103), per 16-element block of a row, in fp32:
//   bmax  = max |x|                                   (exact)
//   sa    = e4m3_rne(clamp(bmax / RN(6 * s2), 2^-9, 448))
//   q_i   = x_i / RN(sa * s2)                         (IEEE division)
//   code  = cast_e2m1(q_i) (:41-51): sign bit 8 when q < 0; magnitude = the
//           number of bounds {0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0} below |q|,
//           plus one at the ties |q| in {0.75, 1.75, 2.5}
//   packed: element 2j in the low nibble of byte j (pack_e2m1, :54-56)
// Scales are written flat [M, K/16] or in the cuBLAS 128 x 4 blocked order of
// to_blocked_scales (:72-84): entry (r, c) at
//   ((r / 128) * ncb + c / 4) * 512 + (r % 32) * 16 + ((r % 128) / 32) * 4 + c % 4,
// ncb = ceil((K/16) / 4); padding entries are the caller's (zeros).
// The same pass may also write the dequantized activations code * sa as bf16
// (exact), the operand of the bf16 GEMM.
//
// Two lanes per block: 16 bytes of x in per lane, 4 bytes of codes and 16 of
// bf16 values out, one scale byte per pair: HBM-bound.
#include <algorithm>

#include "gwa_common.h"

namespace {

constexpr int NV_THREADS = 256;

// e2m1 code (sign bit 3) -> its value: magnitude m = code & 7 is 0 or 0.5 (m < 2), else
// 2^((m >> 1) - 1) * (1 + (m & 1) / 2), built from its fp32 exponent and top mantissa bit
__device__ __forceinline__ float e2m1_value(uint32_t code) {
  const uint32_t m = code & 7u;
  const uint32_t mag = m < 2u ? (m ? 0x3F000000u : 0u) : ((((m >> 1) + 126u) << 23) | ((m & 1u) << 22));
  return __uint_as_float(mag | ((code & 8u) << 28));
}

// fp32 in [2^-9, 448] -> e4m3fn bits (bias 7, 3 mantissa bits), round to nearest, ties to even
__device__ __forceinline__ uint32_t e4m3_rne(float v) {
  const uint32_t u = __float_as_uint(v);
  const int e = (int)(u >> 23) - 127;
  if (e < -6) return (uint32_t)rintf(v * 512.0f);  // subnormal grid 2^-9 (8 = the smallest normal, code 8)
  const uint32_t m = u & 0x7FFFFFu;
  uint32_t r = m >> 20;
  const uint32_t rem = m & 0xFFFFFu;
  if (rem > 0x80000u || (rem == 0x80000u && (r & 1u))) ++r;
  return ((uint32_t)(e + 7) << 3) + r;  // r == 8 carries into the exponent
}

constexpr uint32_t kE4m3Nan = 0x7Fu;  // e4m3fn has no infinity: S.1111.111 is NaN

__device__ __forceinline__ float e4m3_value(uint32_t c) {
  if ((c & 0x7Fu) == kE4m3Nan) return __uint_as_float(0x7FC00000u);
  const uint32_t ex = (c >> 3) & 15u, m = c & 7u;
  return ex == 0 ? (float)m * (1.0f / 512.0f) : __uint_as_float(((ex + 120u) << 23) | (m << 20));
}

// a NaN sorts past every bound (code 7, sign clear), as the reference's searchsorted places it
__device__ __forceinline__ uint32_t e2m1_code(float q) {
  const float a = fabsf(q);
  if (a != a) return 7u;
  uint32_t c = (a > 0.25f) + (a > 0.75f) + (a > 1.25f) + (a > 1.75f) + (a > 2.5f) + (a > 3.5f) + (a > 5.0f);
  c += (a == 0.75f) | (a == 1.75f) | (a == 2.5f);
  return c | (q < 0.0f ? 8u : 0u);
}

// max of |x| over a set as the bit pattern of a non-negative float: unsigned order is value order, and a NaN
// (any payload, sign cleared) sits above infinity, so it propagates like the reference's amax
__device__ __forceinline__ uint32_t abs_bits(float v) { return __float_as_uint(v) & 0x7FFFFFFFu; }

__device__ __forceinline__ int64_t blocked_index(int64_t r, int64_t c, int64_t ncb) {
  return ((r >> 7) * ncb + (c >> 2)) * 512 + (r & 31) * 16 + ((r & 127) >> 5) * 4 + (c & 3);
}

// Dynamic second-level scale (the forward without a static input_scale, models/w4a4.py:342-343):
// s2 = max(max|x| / 2688, 1e-12) in fp32. Pass 1 writes one partial max |x| per workgroup (no
// initialised accumulator, no atomics); the quantizer's workgroups each fold the partials again.
constexpr int NV_MAX_PARTS = 1024;

__global__ __launch_bounds__(NV_THREADS) void nvfp4_absmax_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                                  int64_t M, int K, float* __restrict__ part) {
  __shared__ uint32_t red[NV_THREADS / 64];
  const int64_t chunks = M * (K / 8);
  uint32_t mx = 0u;
  for (int64_t i = (int64_t)blockIdx.x * NV_THREADS + threadIdx.x; i < chunks; i += (int64_t)gridDim.x * NV_THREADS) {
    const int64_t row = i / (K / 8);
    const int col = (int)(i - row * (K / 8)) * 8;
    const v4i w = *(const v4i*)(x + row * ldx + col);
#pragma unroll
    for (int j = 0; j < 4; ++j) mx = max(mx, max(abs_bits(bf16_lo((uint32_t)w[j])), abs_bits(bf16_hi((uint32_t)w[j]))));
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = max(mx, (uint32_t)__shfl_xor((int)mx, o));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t m = red[0];
    for (int w = 1; w < NV_THREADS / 64; ++w) m = max(m, red[w]);
    part[blockIdx.x] = __uint_as_float(m);
  }
}

// s2 from the parts (every thread of the workgroup gets it)
__device__ __forceinline__ float nvfp4_dynamic_s2(const float* __restrict__ part, int nparts) {
  __shared__ uint32_t red[NV_THREADS / 64];
  uint32_t mx = 0u;
  for (int i = threadIdx.x; i < nparts; i += NV_THREADS) mx = max(mx, abs_bits(part[i]));
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = max(mx, (uint32_t)__shfl_xor((int)mx, o));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
  __syncthreads();
  uint32_t m = red[0];
#pragma unroll
  for (int w = 1; w < NV_THREADS / 64; ++w) m = max(m, red[w]);
  const float s = __uint_as_float(m) / 2688.0f;
  return s != s ? s : fmaxf(s, 1e-12f);  // the reference's clamp keeps a NaN
}

// Two lanes per block (lane pair 2p, 2p + 1 holds its elements 0-7 and 8-15), so every load and store of a
// wave covers one contiguous run; the block maximum is one exchange within the pair.
__global__ __launch_bounds__(NV_THREADS) void nvfp4_quant_act_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                                     const float* __restrict__ s2p,
                                                                     uint8_t* __restrict__ q,
                                                                     uint8_t* __restrict__ scales, int blocked,
                                                                     uint16_t* __restrict__ xdq, int64_t M, int KB,
                                                                     const float* __restrict__ parts, int nparts,
                                                                     float* __restrict__ s2_out) {
  // dynamic s2: every workgroup folds the partial maxima (before any thread leaves)
  const float s2 = parts ? nvfp4_dynamic_s2(parts, nparts) : *s2p;
  if (parts && blockIdx.x == 0 && threadIdx.x == 0) *s2_out = s2;
  const int64_t t = (int64_t)blockIdx.x * NV_THREADS + threadIdx.x;  // half-block index over [M, KB, 2]
  if (t >= 2 * M * KB) return;  // the total is even: a pair is active together
  const int64_t b = t >> 1;
  const int h = (int)(t & 1);
  const int64_t row = b / KB;
  const int c = (int)(b - row * KB);
  const v4i w = *(const v4i*)(x + row * ldx + 16 * c + 8 * h);
  float v[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[2 * j] = bf16_lo((uint32_t)w[j]);
    v[2 * j + 1] = bf16_hi((uint32_t)w[j]);
  }
  uint32_t mb = 0u;
#pragma unroll
  for (int i = 0; i < 8; ++i) mb = max(mb, abs_bits(v[i]));
  mb = max(mb, (uint32_t)__shfl_xor((int)mb, 1));
  const float tq = __uint_as_float(mb) / (6.0f * s2);
  // a NaN block maximum (or s2) stays NaN through the reference's clamp and casts to the NaN code
  const uint32_t sc = tq != tq ? kE4m3Nan : e4m3_rne(fminf(fmaxf(tq, 1.0f / 512.0f), 448.0f));
  const float sa = e4m3_value(sc);
  const float den = sa * s2;
  uint32_t codes = 0;
  uint32_t dq[4];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t code = e2m1_code(v[i] / den);
    codes |= code << (4 * i);
    if (xdq) {
      const float d = e2m1_value(code) * sa;  // exact in bf16
      const uint32_t bits = __float_as_uint(d) >> 16;
      if (i & 1) dq[i >> 1] |= bits << 16;
      else dq[i >> 1] = bits;
    }
  }
  *(uint32_t*)(q + b * 8 + 4 * h) = codes;
  if (h == 0) {
    const int64_t ncb = (KB + 3) / 4;
    scales[blocked ? blocked_index(row, c, ncb) : b] = (uint8_t)sc;
  }
  if (xdq) *(v4i*)(xdq + b * 16 + 8 * h) = (v4i){(int)dq[0], (int)dq[1], (int)dq[2], (int)dq[3]};
}

// codes [rows, K/2] + e4m3 scales (flat or blocked) -> bf16 [rows, K] = code * scale (exact)
__global__ __launch_bounds__(NV_THREADS) void nvfp4_dequant_kernel(const uint8_t* __restrict__ q,
                                                                   const uint8_t* __restrict__ scales, int blocked,
                                                                   uint16_t* __restrict__ out, int64_t rows, int KB) {
  const int64_t b = (int64_t)blockIdx.x * NV_THREADS + threadIdx.x;
  if (b >= rows * KB) return;
  const int64_t row = b / KB;
  const int c = (int)(b - row * KB);
  const int64_t ncb = (KB + 3) / 4;
  const float sa = e4m3_value(scales[blocked ? blocked_index(row, c, ncb) : b]);
  const uint2 w = *(const uint2*)(q + b * 8);
  uint32_t dq[8];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint32_t code = ((i < 8 ? w.x : w.y) >> (4 * (i & 7))) & 15u;
    const float d = e2m1_value(code) * sa;
    const uint32_t bits = __float_as_uint(d) >> 16;
    if (i & 1) dq[i >> 1] |= bits << 16;
    else dq[i >> 1] = bits;
  }
  uint16_t* dst = out + b * 16;
  *(v4i*)dst = (v4i){(int)dq[0], (int)dq[1], (int)dq[2], (int)dq[3]};
  *(v4i*)(dst + 8) = (v4i){(int)dq[4], (int)dq[5], (int)dq[6], (int)dq[7]};
}

// y (bf16 [M, N], in place) = RN_bf16(RN_bf16(y * c) + bias), c = RN_bf16(s2 * ws2): the module's
// `y * (s2 * weight_scale_2).to(y.dtype)` then `+ bias` (models/w4a4.py:349-351), each rounded to bf16 as
// torch's bf16 ops round; 8 elements per thread
__global__ __launch_bounds__(NV_THREADS) void nvfp4_scale_bias_kernel(uint16_t* __restrict__ y,
                                                                      const float* __restrict__ s2,
                                                                      const float* __restrict__ ws2,
                                                                      const uint16_t* __restrict__ bias, int64_t M,
                                                                      int N) {
  const int64_t i = ((int64_t)blockIdx.x * NV_THREADS + threadIdx.x) * 8;
  if (i >= M * N) return;
  const float c = bf16_to_f32(f32_to_bf16(*s2 * *ws2));
  const int n0 = (int)(i % N);
  v4i w = *(const v4i*)(y + i);
  v4i b = bias ? *(const v4i*)(bias + n0) : (v4i){0, 0, 0, 0};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float lo = bf16_to_f32(f32_to_bf16(bf16_lo((uint32_t)w[j]) * c));
    float hi = bf16_to_f32(f32_to_bf16(bf16_hi((uint32_t)w[j]) * c));
    if (bias) {
      lo += bf16_lo((uint32_t)b[j]);
      hi += bf16_hi((uint32_t)b[j]);
    }
    w[j] = (int)pack_bf16x2_rn(lo, hi);
  }
  *(v4i*)(y + i) = w;
}

}  // namespace

extern "C" int gwa_nvfp4_scale_bias(void* y, const float* s2, const float* ws2, const void* bias, int64_t M,
                                    int64_t N, void* stream) {
  const char* what = "nvfp4_scale_bias";
  GWA_REQUIRE(M >= 0 && N > 0 && N % 8 == 0 && M * N < (1ll << 40), "%s: bad shape [%lld, %lld] (N %% 8)", what,
              (long long)M, (long long)N);
  if (M == 0) return GWA_OK;
  GWA_REQUIRE(y && s2 && ws2, "%s: null pointer", what);
  GWA_REQUIRE(GWA_ALIGNED(y, 16) && GWA_ALIGNED(bias, 16) && GWA_ALIGNED(s2, 4) && GWA_ALIGNED(ws2, 4),
              "%s: y and bias must be 16-byte aligned", what);
  const int64_t threads = M * N / 8;
  hipLaunchKernelGGL(nvfp4_scale_bias_kernel, dim3((unsigned)((threads + NV_THREADS - 1) / NV_THREADS)),
                     dim3(NV_THREADS), 0, (hipStream_t)stream, (uint16_t*)y, s2, ws2, (const uint16_t*)bias, M,
                     (int)N);
  return gwa_check_launch(what);
}

extern "C" int64_t gwa_nvfp4_blocked_scale_numel(int64_t rows, int64_t kblocks) {
  if (rows <= 0 || kblocks <= 0) return 0;
  return (rows + 127) / 128 * 128 * ((kblocks + 3) / 4) * 4;
}

static int nvfp4_quant(const char* what, const void* x, int64_t ldx, const float* s2, float* s2_out, float* parts,
                       uint8_t* q, uint8_t* scales, int scale_layout, void* xdq, int64_t M, int64_t K,
                       void* stream) {
  GWA_REQUIRE(M >= 0 && K > 0 && K % 16 == 0, "%s: K=%lld is not a multiple of 16", what, (long long)K);
  GWA_REQUIRE(ldx >= K && ldx % 8 == 0, "%s: row stride %lld must be >= K and a multiple of 8", what,
              (long long)ldx);
  GWA_REQUIRE(scale_layout == GWA_NVFP4_SCALES_FLAT || scale_layout == GWA_NVFP4_SCALES_BLOCKED,
              "%s: scale_layout %d", what, scale_layout);
  GWA_REQUIRE(M * K < (1ll << 40), "%s: shape too large", what);
  if (M == 0) return GWA_OK;
  GWA_REQUIRE(x && (s2 || (s2_out && parts)) && q && scales, "%s: null pointer", what);
  GWA_REQUIRE(GWA_ALIGNED(x, 16) && GWA_ALIGNED(q, 8) && GWA_ALIGNED(s2, 4) && GWA_ALIGNED(s2_out, 4) &&
                  GWA_ALIGNED(parts, 4) && GWA_ALIGNED(xdq, 16),
              "%s: x and xdq must be 16-byte, q 8-byte aligned", what);
  hipStream_t st = (hipStream_t)stream;
  int nparts = 0;
  if (parts) {
    const int64_t chunks = M * (K / 8);
    nparts = (int)std::min<int64_t>(NV_MAX_PARTS, (chunks + NV_THREADS * 8 - 1) / (NV_THREADS * 8));
    hipLaunchKernelGGL(nvfp4_absmax_kernel, dim3((unsigned)nparts), dim3(NV_THREADS), 0, st, (const uint16_t*)x,
                       ldx, M, (int)K, parts);
    const int rc = gwa_check_launch(what);
    if (rc != GWA_OK) return rc;
  }
  const int64_t halves = 2 * M * (K / 16);
  hipLaunchKernelGGL(nvfp4_quant_act_kernel, dim3((unsigned)((halves + NV_THREADS - 1) / NV_THREADS)),
                     dim3(NV_THREADS), 0, st, (const uint16_t*)x, ldx, s2, q, scales,
                     scale_layout == GWA_NVFP4_SCALES_BLOCKED ? 1 : 0, (uint16_t*)xdq, M, (int)(K / 16), parts,
                     nparts, s2_out);
  return gwa_check_launch(what);
}

extern "C" int gwa_nvfp4_quant_act(const void* x, int64_t ldx, const float* s2, uint8_t* q, uint8_t* scales,
                                   int scale_layout, void* xdq, int64_t M, int64_t K, void* stream) {
  return nvfp4_quant("nvfp4_quant_act", x, ldx, s2, nullptr, nullptr, q, scales, scale_layout, xdq, M, K, stream);
}

extern "C" int gwa_nvfp4_quant_act_dyn(const void* x, int64_t ldx, float* s2_out, float* parts, uint8_t* q,
                                       uint8_t* scales, int scale_layout, void* xdq, int64_t M, int64_t K,
                                       void* stream) {
  return nvfp4_quant("nvfp4_quant_act_dyn", x, ldx, nullptr, s2_out, parts, q, scales, scale_layout, xdq, M, K,
                     stream);
}

extern "C" int gwa_nvfp4_dequant(const uint8_t* q, const uint8_t* scales, int scale_layout, void* out, int64_t rows,
                                 int64_t K, void* stream) {
  const char* what = "nvfp4_dequant";
  GWA_REQUIRE(rows >= 0 && K > 0 && K % 16 == 0 && rows * K < (1ll << 40), "%s: bad shape [%lld, %lld]", what,
              (long long)rows, (long long)K);
  GWA_REQUIRE(scale_layout == GWA_NVFP4_SCALES_FLAT || scale_layout == GWA_NVFP4_SCALES_BLOCKED,
              "%s: scale_layout %d", what, scale_layout);
  if (rows == 0) return GWA_OK;
  GWA_REQUIRE(q && scales && out, "%s: null pointer", what);
  GWA_REQUIRE(GWA_ALIGNED(q, 8) && GWA_ALIGNED(out, 16), "%s: q must be 8-byte, out 16-byte aligned", what);
  const int64_t blocks = rows * (K / 16);
  hipLaunchKernelGGL(nvfp4_dequant_kernel, dim3((unsigned)((blocks + NV_THREADS - 1) / NV_THREADS)),
                     dim3(NV_THREADS), 0, (hipStream_t)stream, q, scales,
                     scale_layout == GWA_NVFP4_SCALES_BLOCKED ? 1 : 0, (uint16_t*)out, rows, (int)(K / 16));
  return gwa_check_launch(what);
}
