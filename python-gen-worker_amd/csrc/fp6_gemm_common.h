// Shared pieces of the fp6-record W4A4 GEMM kernels: record geometry, the direct-to-LDS copy, wait-count
// helpers, the exact fp6 group MFMA and the operand reads.
#pragma once

#include "gwa_common.h"

// Arguments of one fp6 GEMM launch (checked by the entry point before any kernel sees them).
struct GwaFp6Args {
  const uint8_t* qa6;
  const uint8_t* qw6;
  const float* s2;
  const float* second;
  int per_channel;
  const void* la;
  int la_f32;
  const uint16_t* up;
  const uint16_t* bias;
  uint16_t* out;
  int M, N, K;
};

// The software-pipelined kernel (w4a4_gemm_fp6_pipe.hip) for tm x 192 tiles, tm in {256, 288}, rank / 16 in
// {0, 1, 2, 4, 8}; returns -1 for a configuration it does not have.
int gwa_fp6_pipe_launch(int tm, int rb, bool gelu, bool f16, dim3 grid, hipStream_t s, const GwaFp6Args& a);

namespace {

constexpr int NWAVES = 8, NTHREADS = 64 * NWAVES;  // 512
constexpr int GS = 2;                      // groups per stage (one record)
constexpr int GB = 48;                     // bytes of one row's group (64 e3m2 codes)
constexpr int REC = GWA_FP6_REC;           // 104: record = LDS row stride
constexpr int OFF_SC = GS * GB;            // 96: the record's scales
constexpr int kLdsBytes = 160 * 1024;      // gfx950 LDS per workgroup
constexpr int kFmtE3M2 = 3;                // cbsz / blgp code of e3m2 operands
constexpr int kUnitE8M0 = 127;             // 2^0

// Direct-to-LDS copy of 16 bytes per lane: LDS [m0 + 16 lane, +16) <- buffer
// [voff + soff, +16). The hardware range check covers voff only (not the
// SGPR offset): a copy whose SGPR offset may point past the buffer must keep
// its real address inside readable memory, or put its offset in voff (where
// kOOB makes the lane read zeros without touching memory). Issued as asm so
// the compiler's wait-count pass (which
// tracks only a few LDS-DMA writes and then waits for all of them before any
// LDS read) leaves the waits to the kernel: every LDS read of a stage buffer
// comes after an s_waitcnt that covers this wave's copies into it and a
// barrier that covers everyone else's. The "memory" clobber keeps the copy
// in program order with the surrounding LDS accesses.
__device__ __forceinline__ void dma16(v4i rsrc, uint32_t lds_addr, uint32_t voff, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(lds_addr), "v"(voff), "s"(rsrc), "s"(soff)
               : "memory", "m0");
}

// raw buffer descriptor as an SGPR quad (base, stride 0, num_records, 32-bit data format)
__device__ __forceinline__ v4i raw_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = (uint64_t)base;
  return (v4i){(int)(uint32_t)a, (int)(uint32_t)((a >> 32) & 0xFFFFu), (int)bytes, 0x00020000};
}

// compiler-only fence: keeps LDS reads and writes on their side of a barrier
__device__ __forceinline__ void barrier_lds() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// s_waitcnt vmcnt(n) lgkmcnt(0) (gfx9 encoding; expcnt left at its maximum)
template <int n>
__device__ __forceinline__ void wait_vm_lgkm0() {
  static_assert(n >= 0 && n < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | (7 << 4));
}

// wait until at most `newer` stages of `slots` copies each are still in flight
template <int slots, int maxnewer>
__device__ __forceinline__ void wait_stages(int newer) {
  if constexpr (maxnewer >= 3) {
    if (newer >= 3) { wait_vm_lgkm0<3 * slots>(); return; }
  }
  if constexpr (maxnewer >= 2) {
    if (newer == 2) { wait_vm_lgkm0<2 * slots>(); return; }
  }
  if constexpr (maxnewer >= 1) {
    if (newer == 1) { wait_vm_lgkm0<slots>(); return; }
  }
  wait_vm_lgkm0<0>();
}

__device__ __forceinline__ v16f group_mfma_fp6(v8i a, v8i b) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, (v16f){}, kFmtE3M2, kFmtE3M2, 0, kUnitE8M0, 0,
                                                         kUnitE8M0);
}

// one lane's 32 codes of a group half: 24 bytes, three 8-byte LDS reads. An e3m2 operand of the scaled MFMA is
// six dwords (the instruction reads v[a:a+5] of the 8-register operand), so the last two are left undefined:
// materialising zeros there cost a v_mov per dword per read in the loop.
__device__ __forceinline__ v8i lds_operand(const uint8_t* p) {
  typedef int v2i_ __attribute__((ext_vector_type(2)));
  const v2i_ a = *(const v2i_*)(p), b = *(const v2i_*)(p + 8), c = *(const v2i_*)(p + 16);
  const v4i ab = __builtin_shufflevector(a, b, 0, 1, 2, 3);
  const v4i cc = __builtin_shufflevector(c, c, 0, 1, -1, -1);
  return __builtin_shufflevector(ab, cc, 0, 1, 2, 3, 4, 5, -1, -1);
}

// A tile's per-column epilogue constants s2 * second[n] and bias[n]. The raw words are loaded by thread n - n0
// before the first operand copies are issued (branch-free: an absent operand's buffer has no records and reads
// as zero), stay in three registers through the K loop and are first used when the epilogue writes them to
// LDS, so no wait for them precedes the copies.
struct EpiConsts {
  uint32_t s2, sec;
  uint16_t b;
  bool ok;
};
__device__ __forceinline__ EpiConsts epi_consts_load(const float* s2p, const float* second, int second_per_channel,
                                                     const uint16_t* bias, int n0, int tid, int tn, int N) {
  const int n = n0 + tid;
  EpiConsts c;
  c.ok = tid < tn && n < N;
  const uint32_t sec_bytes = second ? (uint32_t)((second_per_channel ? N : 1) * 4) : 0u;
  c.s2 = __builtin_amdgcn_raw_buffer_load_b32(make_rsrc(s2p, s2p ? 4u : 0u), c.ok ? 0u : kOOB, 0, 0);
  c.sec = __builtin_amdgcn_raw_buffer_load_b32(make_rsrc(second, sec_bytes),
                                               c.ok ? (uint32_t)((second_per_channel ? n : 0) * 4) : kOOB, 0, 0);
  c.b = __builtin_amdgcn_raw_buffer_load_b16(make_rsrc(bias, bias ? (uint32_t)(N * 2) : 0u),
                                             c.ok ? (uint32_t)(n * 2) : kOOB, 0, 0);
  return c;
}
// the constants into g_epi[0, tn) (multiplier) and g_epi[tn, 2 tn) (bias); zeros for columns past N
__device__ __forceinline__ void epi_consts_store(const EpiConsts& c, const float* s2p, const float* second,
                                                 const uint16_t* bias, float* g_epi, int tid, int tn) {
  if (tid < tn) {
    float mult = 0.0f, bv = 0.0f;
    if (c.ok) {
      mult = s2p ? __uint_as_float(c.s2) : 1.0f;
      if (second) mult *= __uint_as_float(c.sec);
      if (bias) bv = bf16_to_f32(c.b);
    }
    g_epi[tid] = mult;
    g_epi[tn + tid] = bv;
  }
}

__device__ __forceinline__ v8i buf_operand(rsrc_t r, uint32_t off) {
  typedef unsigned int v2u __attribute__((ext_vector_type(2)));
  const v2u a = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
  const v2u b = __builtin_amdgcn_raw_buffer_load_b64(r, off + 8, 0, 0);
  const v2u c = __builtin_amdgcn_raw_buffer_load_b64(r, off + 16, 0, 0);
  return (v8i){(int)a[0], (int)a[1], (int)b[0], (int)b[1], (int)c[0], (int)c[1], 0, 0};
}

// The next layer's side of the NQ epilogue: smoothing factors (bf16 [N] or
// NULL), proj_down in the fp6 act-quant kernel's operand order (or NULL),
// its rank / 16, the records [N / 128][M][104] and the la partial slots
// [tiles_n][M][r] fp32.
struct NextLayer {
  const uint16_t* smooth;
  const uint16_t* pdo;
  int rb;
  uint8_t* q6;
  float* la_part;
};
constexpr int kNextRbMax = 8;  // next-layer ranks up to 128

// la (bf16 or, with la_f32, fp32) row m, ranks 8 (k0 / 8) .. +8 -> 8 bf16 MFMA operand values
__device__ __forceinline__ v4i la_operand_lds(const uint8_t* lrb, int row, int rowbytes, int k, bool la_f32) {
  if (!la_f32) return *(const v4i*)(lrb + row * rowbytes + k * 2);
  const v4f a = *(const v4f*)(lrb + row * rowbytes + k * 4);
  const v4f b = *(const v4f*)(lrb + row * rowbytes + k * 4 + 16);
  return (v4i){(int)pack_bf16x2_rn(a[0], a[1]), (int)pack_bf16x2_rn(a[2], a[3]), (int)pack_bf16x2_rn(b[0], b[1]),
               (int)pack_bf16x2_rn(b[2], b[3])};
}

}  // namespace
