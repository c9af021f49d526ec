// Group-64 int4 activation quantization of one lane's 8 consecutive
// elements, shared by the act-quant kernel and the GEMM epilogue that
// quantizes the next layer's input, so both produce the same codes and
// scales bit for bit.
//
// Lane layout: a 64-element group is held by 8 consecutive lanes 8j .. 8j+7
// of a wave, each lane 8 consecutive elements (lane 8j + e holds elements
// 8e .. 8e+7 of the group).
//
// Arithmetic = the reference order (models/svdq_fused.py:88-103,
// models/nvfp4_quant.py:96-102): xs = RN_bf16(RN_f32(x / smooth));
// scale = fp16(clamp(RN_f32(amax / (7 * s2)), 2^-24, 65504));
// code = clamp(rne(RN_f32(xs / (float(scale) * s2))), -8, 7).
//
// Fast path (bit-identical, no per-element division):
//  * smoothing: xs = RN_bf16(x * r), r = RN_f32(1 / smooth). For bf16 x and a
//    normal bf16 smooth, x/s lies at least 2^-18 (relative) from any bf16
//    rounding tie unless it is exact, and |x*r - x/s| <= 2^-23 |x/s|, so both
//    round to the same bf16.
//  * scale: RN(amax / 7) = fma(fma(-7, q1, amax), RN(1/7), q1) with
//    q1 = amax * RN(1/7), for every finite bf16 amax (checked exhaustively
//    with rational arithmetic).
//  * codes (s2 == 1, scale a normal fp16 below the clamp): q = xs / d with an
//    8-bit-significand xs and an 11-bit d is either an exact half-integer or
//    more than 2^-12 from one; p = xs * rcp(d) is within 2^-19 of q. Adding
//    3072 rounds p onto a 2^-12 grid, which lands exact ties exactly on k+1/2
//    and leaves every other value on its own side; adding (1.5*2^23 - 3072)
//    then rounds that grid value to an integer with ties-to-even, exactly the
//    RNE of q. |q| <= 7*(1 + 2^-11) < 7.5 here, so no clamp is needed, and
//    the code is the low nibble of the float's bits.
//  Anything else (s2 != 1, non-normal smooth, clamped or subnormal scales)
//  takes the IEEE-division path (a wave-uniform branch).
#pragma once

#include "gwa_common.h"

namespace g64 {

constexpr float kScaleMin = 5.9604644775390625e-08f;  // 2^-24, smallest positive fp16
constexpr float kFp16Max = 65504.0f;
constexpr float kFp16MinNormal = 6.103515625e-05f;     // 2^-14
constexpr float kSnap = 3072.0f;                       // 1.5 * 2^11: spacing 2^-12 on [2048, 4096)
constexpr float kRound = 12582912.0f - 3072.0f;        // 1.5 * 2^23 - 3072

typedef float v2f __attribute__((ext_vector_type(2)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef unsigned short v2u16 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t code_exact(float v, float d) {
  float q = __builtin_rintf(v / d);
  q = fminf(fmaxf(q, -8.0f), 7.0f);
  return (uint32_t)((int)q) & 0xFu;
}

// smoothing factor usable by the multiply path: 1/s is a normal float
__device__ __forceinline__ bool smooth_ok(float s) {
  const float a = fabsf(s);
  return a >= 1.1754943508222875e-38f && a < 8.507059173023462e37f;
}

// max over the 8-lane group (lanes 8j .. 8j+7) of a 32-bit value
__device__ __forceinline__ uint32_t oct_max(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));   // quad_perm 1,0,3,2
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));   // quad_perm 2,3,0,1
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));  // row_half_mirror
  return v;
}

// xs = RN_bf16(x / smooth) of 8 bf16 values (4 dwords of pairs): multiplied
// by the reciprocals f, or divided by the factors f when `divide` is set
__device__ __forceinline__ void smooth8(v4i c, const float* f, bool divide, uint32_t w[4]) {
  float v[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[2 * j] = bf16_lo((uint32_t)c[j]);
    v[2 * j + 1] = bf16_hi((uint32_t)c[j]);
  }
  if (!divide) {
#pragma unroll
    for (int t = 0; t < 8; ++t) v[t] *= f[t];
  } else {
#pragma unroll
    for (int t = 0; t < 8; ++t) v[t] /= f[t];
  }
#pragma unroll
  for (int t = 0; t < 4; ++t)
    w[t] = __builtin_bit_cast(uint32_t, __builtin_convertvector((v2f){v[2 * t], v[2 * t + 1]}, v2bf));
}

// codes and scale of the lane's 8 smoothed bf16 values w[4] (pairs, element
// 2t in the low half of w[t]): nb[j] holds the codes of elements 4j .. 4j+3,
// one two's-complement nibble per byte; sh = the group's fp16 scale bits.
// Lanes with !valid take part in the group max (their values must be 0) and
// never force the slow path. Every lane of the wave must call this together.
__device__ __forceinline__ void quant8(const uint32_t w[4], bool valid, bool s2_one, float s2, uint32_t nb[2],
                                       uint16_t& sh) {
  // group absmax on the bf16 bit patterns (|x| orders like its bits), over the 8 lanes of the group
  v2u16 mx = {0, 0};
#pragma unroll
  for (int t = 0; t < 4; ++t) mx = __builtin_elementwise_max(mx, __builtin_bit_cast(v2u16, w[t] & 0x7fff7fffu));
  const uint32_t mb = oct_max(mx[0] > mx[1] ? mx[0] : mx[1]);
  const float amax = __uint_as_float(mb << 16);

  float scl;
  const float r7 = 1.0f / 7.0f;
  const bool easy = s2_one && (mb & 0x7F80u) != 0x7F80u;
  if (__builtin_amdgcn_ballot_w64(!easy) == 0) {
    const float q1 = amax * r7;
    scl = fmaf(fmaf(-7.0f, q1, amax), r7, q1);
  } else {
    scl = amax / (7.0f * s2);
  }
  const bool fast = !valid || (s2_one && scl >= kFp16MinNormal && scl < kFp16Max);
  scl = fminf(fmaxf(scl, kScaleMin), kFp16Max);
  sh = f32_to_f16_bits(scl);
  const float d = f16_bits_to_f32(sh) * s2;

  float v[8];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    v[2 * t] = bf16_lo(w[t]);
    v[2 * t + 1] = bf16_hi(w[t]);
  }
  if (__builtin_amdgcn_ballot_w64(!fast) == 0) {  // wave-uniform; neither side touches memory
    const float rd = __builtin_amdgcn_rcpf(d);
#pragma unroll
    for (int j4 = 0; j4 < 2; ++j4) {
      uint32_t hb[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) hb[e] = __float_as_uint(((v[4 * j4 + e] * rd) + kSnap) + kRound);
      nb[j4] = __builtin_amdgcn_perm(__builtin_amdgcn_perm(hb[3], hb[2], 0x0c0c0400u),
                                     __builtin_amdgcn_perm(hb[1], hb[0], 0x0c0c0400u), 0x05040100u) &
               0x0F0F0F0Fu;
    }
  } else {
#pragma unroll
    for (int j4 = 0; j4 < 2; ++j4) {
      nb[j4] = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) nb[j4] |= code_exact(v[4 * j4 + e], d) << (8 * e);
    }
  }
}

// The lane's 8 codes and the group's scale into an fp6 operand record (the
// record of 128-column stage s and row m starts at byte (s * M + m) * 104;
// group `godd` = the group's index within the stage). 8 codes = 48 bits per
// lane; lane pairs share three dwords (the even lane stores the first two);
// the group's first lane stores the scale. Stores of lanes with !valid go
// out of range (dropped). Every lane of the wave must call this together.
__device__ __forceinline__ void store_fp6(rsrc_t qbuf, uint32_t rec, int godd, int lane, const uint32_t nb[2],
                                          uint16_t sh, bool valid) {
  const uint32_t t0 = pack6_x4(e3m2_x4(nb[0])), t1 = pack6_x4(e3m2_x4(nb[1]));
  const uint32_t lo32 = t0 | (t1 << 24), hi16 = t1 >> 8;  // this lane's 48 bits
  const uint32_t nlo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)lo32, 0xB1, 0xF, 0xF, false);
  const bool even = (lane & 1) == 0;
  const uint32_t base6 = valid ? rec + (uint32_t)(godd * 48 + (lane & 6) * 6) : kOOB;
  // branch-free: each lane issues both stores, the one that is not its own goes out of range
  buf_store8(make_uint2(lo32, hi16 | (nlo << 16)), qbuf, even ? base6 : kOOB);
  buf_store4((lo32 >> 16) | (hi16 << 16), qbuf, (!even && valid) ? base6 + 8 : kOOB);
  buf_store2(sh, qbuf, (valid && (lane & 7) == 0) ? rec + 96u + (uint32_t)(godd * 2) : kOOB);
}

// ---------------------------------------------------------------------------
// 32 consecutive elements per lane (half a group; the group's other half in a
// partner lane): the fp6-record path. Same arithmetic and exactness as
// quant8, codes packed to e3m2 by the hardware converter.
// ---------------------------------------------------------------------------
typedef unsigned int v6u __attribute__((ext_vector_type(6)));
typedef float v16f_ __attribute__((ext_vector_type(16)));

// v[i] = RN_bf16(v[i] * f[i]) (f = RN(1/smooth)) or RN_bf16(v[i] / f[i]) (f = smooth) when `divide`
// (wave-uniform; both give the same bf16 for a normal smooth)
__device__ __forceinline__ void smooth32(float* v, const float* f, bool divide) {
  if (!divide) {
#pragma unroll
    for (int i = 0; i < 32; ++i) v[i] *= f[i];
  } else {
#pragma unroll
    for (int i = 0; i < 32; ++i) v[i] /= f[i];
  }
#pragma unroll
  for (int i = 0; i < 32; i += 2) {
    const uint32_t pk = pack_bf16x2_rn(v[i], v[i + 1]);
    v[i] = bf16_lo(pk);
    v[i + 1] = bf16_hi(pk);
  }
}

// the lane's absmax as bit patterns of bf16-exact floats (|x| orders like its bits; NaN above inf)
__device__ __forceinline__ uint32_t absmax_bits32(const float* v) {
  uint32_t mu = 0;
#pragma unroll
  for (int i = 0; i < 32; ++i) mu = max(mu, __float_as_uint(v[i]) & 0x7fffffffu);
  return mu;
}

// codes of v[32] given the group's absmax bits mu: pk = the 32 e3m2 codes (element t at bits [6t, 6t+6)
// of the 24 bytes), sh = the group's fp16 scale. !valid lanes never force the slow paths. Every lane of
// the wave must call this together.
__device__ __forceinline__ void quant32(const float* v, uint32_t mu, bool valid, bool s2_one, float s2, v6u& pk,
                                        uint16_t& sh) {
  const float amax = __uint_as_float(mu);
  const uint32_t mb = mu >> 16;  // the bf16 bits of amax
  float scl;
  const float r7 = 1.0f / 7.0f;
  const bool easy = s2_one && (mb & 0x7F80u) != 0x7F80u;
  if (__builtin_amdgcn_ballot_w64(!easy) == 0) {
    const float q1 = amax * r7;
    scl = fmaf(fmaf(-7.0f, q1, amax), r7, q1);
  } else {
    scl = amax / (7.0f * s2);
  }
  const bool fast = !valid || (s2_one && scl >= kFp16MinNormal && scl < kFp16Max);
  scl = fminf(fmaxf(scl, kScaleMin), kFp16Max);
  sh = f32_to_f16_bits(scl);
  const float d = f16_bits_to_f32(sh) * s2;
  v16f_ qa, qb;  // codes 2i / 2i + 1, as floats
  if (__builtin_amdgcn_ballot_w64(!fast) == 0) {
    const float rd = __builtin_amdgcn_rcpf(d);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      qa[i] = (((v[2 * i] * rd) + kSnap) + kRound) - 12582912.0f;
      qb[i] = (((v[2 * i + 1] * rd) + kSnap) + kRound) - 12582912.0f;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      // + 0.0f: a -0 code is stored as +0 (e3m2 0x00), as the nibble path does
      qa[i] = fminf(fmaxf(__builtin_rintf(v[2 * i] / d), -8.0f), 7.0f) + 0.0f;
      qb[i] = fminf(fmaxf(__builtin_rintf(v[2 * i + 1] / d), -8.0f), 7.0f) + 0.0f;
    }
  }
  // v_cvt_scalef32_2xpk16_bf6_f32: element 2i from the first source's i, 2i+1 from the second's, divided
  // by the scale (1: exact for the integers -8 .. 8). Written as asm with an early-clobber result: the
  // builtin let the compiler give the 6 result registers a partial overlap with the 32 source registers
  // (v[2:7] <- v[0:15], v[16:31]), and the instruction then read a source it had already overwritten
  // (element 4 of a lane's 32 came out as a non-integer e3m2 code).
  asm("v_cvt_scalef32_2xpk16_bf6_f32 %0, %1, %2, 1.0" : "=&v"(pk) : "v"(qa), "v"(qb));
}

}  // namespace g64
