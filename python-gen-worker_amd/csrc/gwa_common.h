// Shared device/host helpers for the gen_worker_amd C-ABI library (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gen_worker_amd.h"

// ---------------------------------------------------------------------------
// vector types used as MFMA operands
// ---------------------------------------------------------------------------
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

// ---------------------------------------------------------------------------
// host-side error state (defined in gwa_runtime.hip)
// ---------------------------------------------------------------------------
int gwa_set_error(int code, const char* fmt, ...);
int gwa_check_launch(const char* what);

#define GWA_ALIGNED(p, n) ((((uintptr_t)(p)) & ((n) - 1)) == 0)

#define GWA_REQUIRE(cond, ...)                                   \
  do {                                                           \
    if (!(cond)) return gwa_set_error(GWA_ERR_INVALID, __VA_ARGS__); \
  } while (0)

// ---------------------------------------------------------------------------
// scalar conversions (exact, RNE where rounding happens)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float(((uint32_t)b) << 16); }

// float -> bf16 bits, round to nearest even; NaN stays NaN (quiet bit set).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  _Float16 h = (_Float16)f;
  return __builtin_bit_cast(uint16_t, h);
}
__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
  return (float)__builtin_bit_cast(_Float16, b);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return (uint32_t)f32_to_bf16(a) | ((uint32_t)f32_to_bf16(b) << 16);
}
// RN-even bf16 pair with the hardware conversion (v_cvt_pk_bf16_f32); a NaN stays a NaN.
__device__ __forceinline__ uint32_t pack_bf16x2_rn(float a, float b) {
  typedef float v2f_ __attribute__((ext_vector_type(2)));
  typedef __bf16 v2bf_ __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((v2f_){a, b}, v2bf_));
}
__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
  return (uint32_t)f32_to_f16_bits(a) | ((uint32_t)f32_to_f16_bits(b) << 16);
}

// GELU, tanh approximation, fp32: 0.5 y (1 + tanh u) with u = sqrt(2/pi) (y + 0.044715 y^3) equals
// y * sigmoid(2u) = y / (1 + 2^(-2u log2 e)): one native exp2 and one native reciprocal (each ~1 ulp), a
// relative error of a few 1e-6 against the exact form (large |y| saturate to y and -0; NaN stays NaN).
__device__ __forceinline__ float gelu_tanh_f32(float y) {
  constexpr float k0 = -2.0f * 0.7978845608028654f * 1.4426950408889634f;  // -2 sqrt(2/pi) log2(e)
  constexpr float k1 = k0 * 0.044715f;
  const float e = __builtin_amdgcn_exp2f(y * fmaf(y * y, k1, k0));
  return y * __builtin_amdgcn_rcpf(1.0f + e);
}

// ---------------------------------------------------------------------------
// int4 helpers
// ---------------------------------------------------------------------------
// Two's-complement nibbles, element 2j in the low nibble of byte j.
// To int8 operand bytes holding 16*q (the nibble in the high half of the
// byte): a signed int8 MFMA on these computes 256 * sum(qx * qw), exactly.
__device__ __forceinline__ uint32_t int4_lo_x16(uint32_t w) { return (w << 4) & 0xF0F0F0F0u; }
__device__ __forceinline__ uint32_t int4_hi_x16(uint32_t w) { return w & 0xF0F0F0F0u; }

// e3m2 ("bf6") codes: every int4 code -8..7 is an exact e3m2 value, so fp6
// MFMAs on these codes compute integer dot products exactly.
// four nibble codes held as bytes (two's-complement nibble in the low 4 bits) -> four e3m2 bytes
__device__ __forceinline__ uint32_t e3m2_x4(uint32_t nib) {
  // q = 0..7 and q = -8..-1 (nibble 8..15) tables, byte j = code of nibble j / j + 8
  const uint32_t sel = nib & 0x07070707u;
  const uint32_t pos = __builtin_amdgcn_perm(0x17161514u, 0x12100C00u, sel);
  const uint32_t neg = __builtin_amdgcn_perm(0x2C303234u, 0x35363738u, sel);
  const uint32_t m = ((nib >> 3) & 0x01010101u) * 0xFFu;
  return (neg & m) | (pos & ~m);
}

// four 6-bit codes in the low bits of four bytes -> 24 contiguous bits
__device__ __forceinline__ uint32_t pack6_x4(uint32_t b) {
  return (b & 0x3Fu) | ((b >> 2) & 0xFC0u) | ((b >> 4) & 0x3F000u) | ((b >> 6) & 0xFC0000u);
}

__device__ __forceinline__ int ceil_div(int a, int b) { return (a + b - 1) / b; }

// ---------------------------------------------------------------------------
// raw buffer access: loads outside [0, bytes) return 0 and stores there are
// dropped by the hardware, so row/column tails need no branches (and the
// compiler can count outstanding memory operations exactly)
// ---------------------------------------------------------------------------
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ v4i buf_load16(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}
__device__ __forceinline__ uint32_t buf_load4(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
__device__ __forceinline__ uint16_t buf_load2(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}
__device__ __forceinline__ void buf_store16(v4i v, rsrc_t r, uint32_t off) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, 0);
}
__device__ __forceinline__ void buf_store8(uint2 v, rsrc_t r, uint32_t off) {
  typedef unsigned int v2u __attribute__((ext_vector_type(2)));
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(v2u, v), r, off, 0, 0);
}
__device__ __forceinline__ void buf_store4(uint32_t v, rsrc_t r, uint32_t off) {
  __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, 0);
}
__device__ __forceinline__ void buf_store2(uint16_t v, rsrc_t r, uint32_t off) {
  __builtin_amdgcn_raw_buffer_store_b16(v, r, off, 0, 0);
}
constexpr uint32_t kOOB = 0x80000000u;  // an offset past every buffer this library builds (all < 2 GiB)

// ---------------------------------------------------------------------------
// Debug build (GWA_DEBUG): bounds checks on the global accesses whose range no hardware check covers or
// whose silent drop would hide a mistake (direct-to-LDS copies at scalar offsets; record and output
// stores at computed offsets). A failed check sets its site's bit in this translation unit's violation word,
// keeps the first failure's site, workgroup and offset, and the access is redirected or skipped: nothing
// traps and no access leaves its buffer. gwa_debug_violations (gwa_runtime.hip) ORs every translation
// unit's word. Release builds compile the checks to nothing.
// ---------------------------------------------------------------------------
enum GwaDbgSite {
  kDbgFp6CopyA = 0,   // fp6 GEMM: an activation-record copy run past its buffer + slack
  kDbgFp6CopyW = 1,   // fp6 GEMM: a weight-record copy run past its buffer + slack
  kDbgFp6Out = 2,     // fp6 GEMM: an output store past the [M, N] output
  kDbgQuantRec = 3,   // kernel 1: a record store past the record buffer
  kDbgW8Copy = 4,     // W8A8 GEMM: a copy run past the operand rows' K bytes
  kDbgW8Out = 5,      // W8A8 GEMM: an output store past the [M, N] output
};
#ifdef GWA_DEBUG
int gwa_dbg_register(int (*reader)(uint32_t* bits, uint64_t* first, int clear));
namespace {
__device__ uint32_t g_gwa_dbg_bits;   // bit s: site s failed
__device__ uint64_t g_gwa_dbg_first;  // site << 56 | workgroup << 32 | offset of the first failure seen
int gwa_dbg_read_tu(uint32_t* bits, uint64_t* first, int clear) {
  uint32_t b = 0;
  uint64_t f = 0;
  if (hipMemcpyFromSymbol(&b, HIP_SYMBOL(g_gwa_dbg_bits), sizeof b) != hipSuccess) return GWA_ERR_HIP;
  if (hipMemcpyFromSymbol(&f, HIP_SYMBOL(g_gwa_dbg_first), sizeof f) != hipSuccess) return GWA_ERR_HIP;
  *bits |= b;
  if (*first == 0) *first = f;
  if (clear) {
    const uint32_t zb = 0;
    const uint64_t zf = 0;
    if (hipMemcpyToSymbol(HIP_SYMBOL(g_gwa_dbg_bits), &zb, sizeof zb) != hipSuccess) return GWA_ERR_HIP;
    if (hipMemcpyToSymbol(HIP_SYMBOL(g_gwa_dbg_first), &zf, sizeof zf) != hipSuccess) return GWA_ERR_HIP;
  }
  return GWA_OK;
}
[[maybe_unused]] const int g_gwa_dbg_registered = gwa_dbg_register(gwa_dbg_read_tu);
}  // namespace
__device__ __forceinline__ bool gwa_dcheck(bool ok, int site, uint32_t off) {
  if (!ok) {
    const uint64_t rec = ((uint64_t)site << 56) | ((uint64_t)(blockIdx.x & 0xFFFFFFu) << 32) | off;
    if (atomicOr(&g_gwa_dbg_bits, 1u << site) == 0u) atomicCAS((unsigned long long*)&g_gwa_dbg_first, 0ull, rec);
  }
  return ok;
}
#define GWA_DCHECK(ok, site, off) gwa_dcheck((ok), (site), (uint32_t)(off))
#else
#define GWA_DCHECK(ok, site, off) true
#endif

// ---------------------------------------------------------------------------
// GEMM tile order
// ---------------------------------------------------------------------------
constexpr int kXcds = 8;  // MI355X: workgroup i runs on XCD i % 8

// workgroup id -> (tile_m, tile_n): a contiguous run of tiles per XCD, in an
// order that walks GM tile rows before moving to the next tile column
__device__ __forceinline__ bool xcd_tile_of(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int T = tiles_m * tiles_n;
  const int per = (T + kXcds - 1) / kXcds;
  const int t = (bid % kXcds) * per + bid / kXcds;
  if (t >= T) return false;
  constexpr int GM = 8;
  const int band = t / (GM * tiles_n);
  const int gm = min(GM, tiles_m - band * GM);
  const int rem = t - band * GM * tiles_n;
  tm = band * GM + rem % gm;
  tn = rem / gm;
  return true;
}
