// Activation-side kernels: int4 group-64 quantization (+ fused x @ proj_down),
// int8 per-token quantization, and the standalone SVDQuant epilogue.
#include "gwa_common.h"

// ---------------------------------------------------------------------------
// Kernel 1: smoothing divide -> group-64 absmax -> fp16 scale -> int4 codes,
// packed two per byte; plus la = x @ proj_down on the RAW activations via
// bf16 MFMA 16x16x32.
//
// Work split: a workgroup owns 16 rows; its NW waves split the K groups of
// those rows evenly, and their partial la blocks are summed through LDS. Lane
// (i = lane % 16, kq = lane / 16) holds, per group of 64, the 16 elements of
// row i at K offsets kq*8 + [0,8) and 32 + kq*8 + [0,8): each is one 16-byte
// load, and the same registers are the MFMA A operand of the group's two
// 32-wide K halves. The row's group absmax is a max over lanes {i, i+16,
// i+32, i+48}.
//
// Arithmetic = the reference order (models/svdq_fused.py:88-103,
// models/nvfp4_quant.py:96-102): xs = RN_bf16(RN_f32(x / smooth));
// scale = fp16(clamp(RN_f32(amax / (7 * s2)), 2^-24, 65504));
// code = clamp(rne(RN_f32(xs / (float(scale) * s2))), -8, 7).
//
// Fast path (bit-identical, no per-element division):
//  * smoothing: xs = RN_bf16(x * r), r = RN_f32(1 / smooth). For bf16 x and a
//    normal bf16 smooth, x/s lies at least 2^-17 (relative) from any bf16
//    rounding tie unless it is exact, and |x*r - x/s| <= 2^-23 |x/s|, so both
//    round to the same bf16.
//  * codes (s2 == 1, scale a normal fp16 below the clamp): q = xs / d with an
//    8-bit-significand xs and an 11-bit d is either an exact half-integer or
//    more than 2^-12 from one; p = xs * rcp(d) is within 2^-19 of q. Adding
//    3072 rounds p onto a 2^-12 grid, which lands exact ties exactly on k+1/2
//    and leaves every other value on its own side; adding (1.5*2^23 - 3072)
//    then rounds that grid value to an integer with ties-to-even, exactly the
//    RNE of q. |q| <= 7*(1 + 2^-11) < 7.5 here, so no clamp is needed, and
//    the code is the low nibble of the float's bits.
//  Anything else (s2 != 1, non-normal smooth, clamped or subnormal scales)
//  takes the IEEE-division path.
// ---------------------------------------------------------------------------
namespace {

constexpr float kScaleMin = 5.9604644775390625e-08f;  // 2^-24, smallest positive fp16
constexpr float kFp16Max = 65504.0f;
constexpr float kFp16MinNormal = 6.103515625e-05f;     // 2^-14
constexpr float kSnap = 3072.0f;                       // 1.5 * 2^11: spacing 2^-12 on [2048, 4096)
constexpr float kRound = 12582912.0f - 3072.0f;        // 1.5 * 2^23 - 3072

typedef float v2f __attribute__((ext_vector_type(2)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef unsigned short v2u16 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ void unpack8_bf16(v4i w, float* v) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t u = (uint32_t)w[j];
    v[2 * j] = bf16_lo(u);
    v[2 * j + 1] = bf16_hi(u);
  }
}

__device__ __forceinline__ uint32_t int4_code_exact(float v, float d) {
  float q = __builtin_rintf(v / d);
  q = fminf(fmaxf(q, -8.0f), 7.0f);
  return (uint32_t)((int)q) & 0xFu;
}

// Pack 8 codes held as the low nibbles of h[0..7] (element 2j in the low nibble).
// Each pair becomes one byte (bits 8+ of the pair word are don't-care), and
// two byte permutes gather the four bytes.
__device__ __forceinline__ uint32_t pack_nibbles(const uint32_t* h) {
  uint32_t p[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) p[j] = (h[2 * j] & 0xFu) | (h[2 * j + 1] << 4);
  const uint32_t lo = __builtin_amdgcn_perm(p[1], p[0], 0x0c0c0400u);  // bytes 0,1: p0.b0, p1.b0
  const uint32_t hi = __builtin_amdgcn_perm(p[3], p[2], 0x04000c0cu);  // bytes 2,3: p2.b0, p3.b0
  return lo | hi;
}

// smoothing factor usable by the multiply path: 1/s is a normal float
__device__ __forceinline__ bool smooth_ok(float s) {
  const float a = fabsf(s);
  return a >= 1.1754943508222875e-38f && a < 8.507059173023462e37f;
}

// ---------------------------------------------------------------------------
// Kernel 1. A workgroup owns 16 rows and walks K in rounds of NW groups:
// in round r wave w quantizes group r * NW + w. Each round's low-rank operand
// slice (proj_down^T, NW * 64 columns) and smoothing factors are staged
// once per workgroup into a double-buffered LDS area by all threads, so the
// waves' registers only hold their own activation prefetch ring (PF rounds
// deep). Staging loads for round r+2 are issued in round r, into the second
// of two register sets, and written to LDS at the end of round r+1; they are
// issued before the activation loads of round r+PF, and vector memory
// operations complete in order, so waiting for the staging never waits for
// activations still in flight.
//
// LDS per buffer: [NW][RB][2][64 lanes][8 bf16] operand slice, then
// [NW * 64] reciprocals and [NW * 64] factors (fp32), then one flag word
// holding the last round whose factors the multiply path cannot use.
// ---------------------------------------------------------------------------
template <int RB, int NW>
struct QuantLds {
  static constexpr int kOpBytes = NW * RB * 2 * 64 * 16;
  static constexpr int kBufBytes = kOpBytes + NW * 64 * 4 * 2 + 16;
  static constexpr int kChunks = (NW * RB * 2 * 64) / (NW * 64);  // 16-byte operand loads per thread per round
};

template <int RB, int NW, int PF>
__global__ __launch_bounds__(NW * 64) void svdq_quant_int4_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const uint16_t* __restrict__ smooth,
    const float* __restrict__ s2p, const uint16_t* __restrict__ pdt, uint8_t* __restrict__ q,
    uint16_t* __restrict__ sc, uint16_t* __restrict__ la, int M, int K) {
  using L = QuantLds<RB, NW>;
  constexpr int NCH = RB > 0 ? L::kChunks : 1;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int i = lane & 15, kq = lane >> 4;
  const int row0 = blockIdx.x * 16;
  const int row = row0 + i;
  const int G = K >> 6;
  const int rounds = (G + NW - 1) / NW;

  // buffers: every access is unconditional; rows >= M and groups >= G read 0 / store nothing
  const rsrc_t xbuf = make_rsrc(x, (uint32_t)(((int64_t)(M - 1) * ldx + K) * 2));
  const rsrc_t qbuf = make_rsrc(q, (uint32_t)((int64_t)M * (K >> 1)));
  const rsrc_t sbuf = make_rsrc(sc, (uint32_t)((int64_t)M * G * 2));
  const rsrc_t pbuf = make_rsrc(pdt, (uint32_t)(RB * 16 * K * 2));
  const rsrc_t smbuf = make_rsrc(smooth, smooth ? (uint32_t)(K * 2) : 0u);
  const uint32_t xrow = (uint32_t)((int64_t)row * ldx * 2) + (uint32_t)(kq * 16);
  const uint32_t qrow = (uint32_t)((int64_t)row * (K >> 1)) + (uint32_t)(kq * 4);
  const uint32_t srow = kq == 0 ? (uint32_t)((int64_t)row * G * 2) : kOOB;

  // staging roles: operand chunk c = tid + j * NW * 64 -> (slot, rb, half, lane c % 64)
  uint32_t poff[NCH];
  int pslot[NCH];
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int c = tid + j * NW * 64;
    const int cl = c & 63, half = (c >> 6) & 1, rb = (c >> 7) % (RB > 0 ? RB : 1);
    pslot[j] = (c >> 7) / (RB > 0 ? RB : 1);
    poff[j] = (uint32_t)(((rb * 16 + (cl & 15)) * K + half * 32 + (cl >> 4) * 8) * 2);
  }
  // smoothing: threads 0 .. NW*32-1 stage two factors each
  const bool sm_role = smooth && tid < NW * 32;

  auto stage_load = [&](v4i* pv, uint32_t& sv, int r) {
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int g = r * NW + pslot[j];
      pv[j] = RB > 0 ? buf_load16(pbuf, g < G ? poff[j] + (uint32_t)(g * 128) : kOOB) : (v4i){0, 0, 0, 0};
    }
    const int k = r * NW * 64 + tid * 2;
    sv = sm_role ? buf_load4(smbuf, k < K ? (uint32_t)(k * 2) : kOOB) : 0u;
  };
  // writes the staged round r into LDS buffer b; a factor the multiply path
  // cannot use marks the buffer's flag word with r (stale marks hold older
  // rounds, so the flag never needs clearing)
  auto stage_store = [&](const v4i* pv, uint32_t sv, int r, int b) {
    uint8_t* base = lds + b * L::kBufBytes;
#pragma unroll
    for (int j = 0; j < NCH; ++j)
      if (RB > 0) *(v4i*)(base + (tid + j * NW * 64) * 16) = pv[j];
    if (sm_role) {
      const float s0 = bf16_lo(sv), s1 = bf16_hi(sv);
      const int k = tid * 2;
      float* rs = (float*)(base + L::kOpBytes);
      float* fs = rs + NW * 64;
      rs[k] = 1.0f / s0;
      rs[k + 1] = 1.0f / s1;
      fs[k] = s0;
      fs[k + 1] = s1;
      const bool live = (r * NW * 64 + k < K);  // factors past K are padding
      if (live && (!smooth_ok(s0) || !smooth_ok(s1))) *(int*)(fs + NW * 64) = r;
    }
  };
  auto round_bad = [&](int r, int b) -> bool {
    return *(const int*)(lds + b * L::kBufBytes + L::kOpBytes + NW * 64 * 8) == r;
  };

  const float s2 = s2p ? *s2p : 1.0f;
  const bool s2_one = (s2 == 1.0f);
  const float den7 = 7.0f * s2;

  // prologue: stage round 0 (and issue round 1), prime the activation ring with rounds 0 .. PF-1
  v4i pv[2][NCH];
  uint32_t sv[2];
  stage_load(pv[0], sv[0], 0);
  stage_load(pv[1], sv[1], 1);
  v4i xa[PF], xb[PF];
#pragma unroll
  for (int j = 0; j < PF; ++j) {
    const int g = j * NW + wave;
    const uint32_t off = g < G ? xrow + (uint32_t)(g * 128) : kOOB;
    xa[j] = buf_load16(xbuf, off);
    xb[j] = buf_load16(xbuf, g < G ? off + 64 : kOOB);
  }
  if (tid < 2) *(int*)(lds + tid * L::kBufBytes + L::kOpBytes + NW * 64 * 8) = -1;
  __syncthreads();
  stage_store(pv[0], sv[0], 0, 0);
  __syncthreads();

  v4f acc[RB > 0 ? RB : 1];
#pragma unroll
  for (int rb = 0; rb < (RB > 0 ? RB : 1); ++rb) acc[rb] = (v4f){0.f, 0.f, 0.f, 0.f};

  static_assert(PF % 2 == 0, "the staging register set alternates with the round");
  for (int rr = 0; rr < rounds; rr += PF) {
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      const int r = rr + j;
      const int b = r & 1;
      // staging loads for round r+2 (set r & 1 was published at the end of
      // round r-1), then the activation loads for round r+PF
      stage_load(pv[j & 1], sv[j & 1], r + 2);
      const v4i ca = xa[j], cb = xb[j];
      {
        const int gn = (r + PF) * NW + wave;
        const uint32_t off = gn < G ? xrow + (uint32_t)(gn * 128) : kOOB;
        xa[j] = buf_load16(xbuf, off);
        xb[j] = buf_load16(xbuf, gn < G ? off + 64 : kOOB);
      }
      const int g = r * NW + wave;
      const bool valid = g < G;
      const uint8_t* base = lds + b * L::kBufBytes;
      const bool bad = smooth && round_bad(r, b);

      // xs as packed bf16 words (8 per lane)
      uint32_t w[8];
      if (!smooth) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          w[t] = (uint32_t)ca[t];
          w[4 + t] = (uint32_t)cb[t];
        }
      } else {
        float v[16], f[16];
        unpack8_bf16(ca, v);
        unpack8_bf16(cb, v + 8);
        // bad == 0: multiply by RN(1/s), bit-identical to dividing (|x*r - x/s| <= 2^-23 |x/s|,
        // while x/s is 2^-18 or more (relative) from every bf16 rounding tie); else divide.
        const float* src = (const float*)(base + L::kOpBytes) + (bad ? NW * 64 : 0) + wave * 64 + kq * 8;
        *(v4f*)(f) = *(const v4f*)(src);
        *(v4f*)(f + 4) = *(const v4f*)(src + 4);
        *(v4f*)(f + 8) = *(const v4f*)(src + 32);
        *(v4f*)(f + 12) = *(const v4f*)(src + 36);
        if (!bad) {
#pragma unroll
          for (int t = 0; t < 16; ++t) v[t] *= f[t];
        } else {
#pragma unroll
          for (int t = 0; t < 16; ++t) v[t] /= f[t];
        }
#pragma unroll
        for (int t = 0; t < 8; ++t)
          w[t] = __builtin_bit_cast(uint32_t, __builtin_convertvector((v2f){v[2 * t], v[2 * t + 1]}, v2bf));
      }
      // group absmax on the bf16 bit patterns (|x| orders like its bits)
      v2u16 mx = {0, 0};
#pragma unroll
      for (int t = 0; t < 8; ++t)
        mx = __builtin_elementwise_max(mx, __builtin_bit_cast(v2u16, w[t] & 0x7fff7fffu));
      uint32_t mb = mx[0] > mx[1] ? mx[0] : mx[1];
      mb = max(mb, (uint32_t)__shfl_xor((int)mb, 16));
      mb = max(mb, (uint32_t)__shfl_xor((int)mb, 32));
      const float amax = __uint_as_float(mb << 16);

      float scl = amax / den7;
      const bool fast = !valid || (s2_one && scl >= kFp16MinNormal && scl < kFp16Max);
      scl = fminf(fmaxf(scl, kScaleMin), kFp16Max);
      const uint16_t sh = f32_to_f16_bits(scl);
      const float d = f16_bits_to_f32(sh) * s2;

      float v[16];
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        v[2 * t] = bf16_lo(w[t]);
        v[2 * t + 1] = bf16_hi(w[t]);
      }
      uint32_t w0, w1;
      // wave-uniform choice; neither side touches memory
      if (__builtin_amdgcn_ballot_w64(!fast) == 0) {
        const float rd = __builtin_amdgcn_rcpf(d);
        uint32_t h[16];
#pragma unroll
        for (int t = 0; t < 16; ++t) h[t] = __float_as_uint(((v[t] * rd) + kSnap) + kRound);
        w0 = pack_nibbles(h);
        w1 = pack_nibbles(h + 8);
      } else {
        w0 = w1 = 0;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          w0 |= int4_code_exact(v[t], d) << (4 * t);
          w1 |= int4_code_exact(v[8 + t], d) << (4 * t);
        }
      }
      const uint32_t qo = valid ? qrow + (uint32_t)(g * 32) : kOOB;
      buf_store4(w0, qbuf, qo);
      buf_store4(w1, qbuf, valid ? qo + 16 : kOOB);
      buf_store2(sh, sbuf, valid ? srow + (uint32_t)(g * 2) : kOOB);

      // la += x[:, group] @ proj_down[group, :] (raw activations)
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        const uint8_t* op = base + ((wave * RB + rb) * 2) * 1024 + lane * 16;
        const v4i b0 = *(const v4i*)(op);
        const v4i b1 = *(const v4i*)(op + 1024);
        acc[rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, ca), __builtin_bit_cast(v8bf, b0),
                                                          acc[rb], 0, 0, 0);
        acc[rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, cb), __builtin_bit_cast(v8bf, b1),
                                                          acc[rb], 0, 0, 0);
      }
      // publish round r+1 (its buffer was last read in round r-1, before the previous barrier)
      stage_store(pv[(j + 1) & 1], sv[(j + 1) & 1], r + 1, b ^ 1);
      __syncthreads();
    }
  }

  if (RB > 0) {
    // sum the NW partial la blocks through LDS (buffer 0 is free after the last barrier); wave 0 writes bf16
    float* lap = (float*)lds;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) *(v4f*)(lap + ((wave * RB + rb) * 64 + lane) * 4) = acc[rb];
    __syncthreads();
    if (wave == 0) {
      const int R = RB * 16;
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        v4f s = acc[rb];
        for (int w = 1; w < NW; ++w) {
          const v4f o = *(const v4f*)(lap + ((w * RB + rb) * 64 + lane) * 4);
          s += o;
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int r = row0 + 4 * kq + t;
          if (r < M) la[(int64_t)r * R + rb * 16 + i] = f32_to_bf16(s[t]);
        }
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
  GWA_REQUIRE(R == 0 || R == 16 || R == 32 || R == 64 || R == 128,
              "svdq_quant_int4: rank %lld not in {0,16,32,64,128}", (long long)R);
  GWA_REQUIRE(M < (1ll << 31) && K < (1ll << 24) && (M * ldx * 2) < (1ll << 31),
              "svdq_quant_int4: x must stay below 2 GiB (buffer addressing)");
  if (M == 0) return GWA_OK;
  GWA_REQUIRE(x && q && scales, "svdq_quant_int4: null pointer");
  GWA_REQUIRE(GWA_ALIGNED(x, 16) && GWA_ALIGNED(q, 16) && GWA_ALIGNED(scales, 2) &&
                  GWA_ALIGNED(smooth, 16) && GWA_ALIGNED(proj_down_t, 16) && GWA_ALIGNED(la, 2),
              "svdq_quant_int4: x, q, smooth and proj_down_t must be 16-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  const uint16_t* xp = (const uint16_t*)x;
  const uint16_t* sm = (const uint16_t*)smooth;
  const uint16_t* pd = (const uint16_t*)proj_down_t;
  uint16_t* sc = (uint16_t*)scales;
  uint16_t* lp = (uint16_t*)la;
  const int m = (int)M, k = (int)K;
  const int rb = (int)(R / 16);
  // K is walked in rounds of NW groups per 16-row block: more waves when
  // there are few row blocks, so that small-M calls still fill the GPU, as
  // long as the double-buffered operand staging fits in LDS.
  const int64_t blocks = (M + 15) / 16;
  int nw = blocks >= 512 ? 4 : (blocks >= 128 ? 8 : 16);
  auto lds_bytes = [&](int w) { return (size_t)2 * ((size_t)w * rb * 2048 + (size_t)w * 512); };
  while (nw > 4 && lds_bytes(nw) > 160 * 1024) nw >>= 1;
  const size_t lds = lds_bytes(nw);
  GWA_REQUIRE(lds <= 160 * 1024, "svdq_quant_int4: rank %lld needs too much LDS", (long long)R);
  // activation prefetch depth (even: the staging registers alternate by round)
  const int64_t rounds = (K / 64 + nw - 1) / nw;
  const int pf = (rounds % 4 == 0) ? 4 : 2;
  const dim3 grid((unsigned)blocks);
#define GWA_QUANT_LAUNCH(RBV, NWV, PFV)                                                                  \
  hipLaunchKernelGGL((svdq_quant_int4_kernel<RBV, NWV, PFV>), grid, dim3(NWV * 64), lds, s, xp, ldx, sm, s2, pd, \
                     q, sc, lp, m, k)
#define GWA_QUANT_NW(RBV, NWV)                                   \
  if (pf == 4) GWA_QUANT_LAUNCH(RBV, NWV, 4);                    \
  else GWA_QUANT_LAUNCH(RBV, NWV, 2);
#define GWA_QUANT_RB(RBV)                    \
  case RBV:                                  \
    if (nw == 16) { GWA_QUANT_NW(RBV, 16) }  \
    else if (nw == 8) { GWA_QUANT_NW(RBV, 8) } \
    else { GWA_QUANT_NW(RBV, 4) }            \
    break;
  switch (rb) {
    GWA_QUANT_RB(0)
    GWA_QUANT_RB(1)
    GWA_QUANT_RB(2)
    case 4:
      if (nw == 8) { GWA_QUANT_NW(4, 8) }
      else { GWA_QUANT_NW(4, 4) }
      break;
    case 8: GWA_QUANT_NW(8, 4) break;
    default: return gwa_set_error(GWA_ERR_INVALID, "svdq_quant_int4: rank %lld not in {0,16,32,64,128}", (long long)R);
  }
#undef GWA_QUANT_NW
#undef GWA_QUANT_RB
#undef GWA_QUANT_LAUNCH
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
