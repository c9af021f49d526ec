// W4A4 GEMM on gfx950's fp6 MFMA.
//
// Both operands arrive as e3m2 ("bf6") codes in fp6 operand records (one
// 104-byte record per 128-element stage of K and row, stage-major: 96 bytes
// of codes, the stage's two fp16 group scales, 4 unused bytes): the
// activations straight from the act-quant kernel (GWA_QFMT_FP6), the weights
// prepacked once (gwa_svdq_pack_weight_fp6). Every int4 code -8..7 is an exact
// e3m2 value and the MFMA accumulates in fp32, so ONE
// v_mfma_scale_f32_32x32x64_f8f6f4 (unit E8M0 scales) returns the exact
// integer dot product P of a 64-element group for a 32 x 32 block
// (|P| <= 4096), at twice the fp8/int8 MFMA rate.
//
// Dequantization, per group g, 32 x 32 block and element (n, m):
//     acc += P * S,    S = sw[n][g] * sx[m][g]
// S is the outer product of two f16 vectors, formed exactly (fp32 result) by
// one f16 MFMA (32x32x8): lanes 0..31 of the weight-side operand hold the
// stage's 2 group scales of their row in K slots 0..1 and lanes 32..63 hold
// zeros; the activation-side operand holds group g's scale in slot g and zero
// in the other slot. That leaves one VALU fma per output element and group.
//
// Epilogue: acc * s2 * second[n], + la @ up^T (bf16 MFMA), + bias, optional
// GELU (tanh form), four consecutive n per lane packed to bf16 / f16, staged
// in LDS and stored as full rows. With the next-layer variant (NQ) the staged
// bf16 tile is also the next layer's input: it is quantized there into the
// next layer's fp6 operand records (smoothing divide, group-64 scales and
// codes by the same per-lane quantizer as the act-quant kernel, so the
// records equal the act-quant kernel's on this output bit for bit), and its
// product with the next layer's proj_down rows n0 .. n0+TN is stored as the
// column tile's partial (slot tn of an fp32 [tiles_n][M][r] buffer, which
// gwa_svdq_la_reduce sums in a fixed order).
//
// Tiling: a 512-thread workgroup owns a 256 (n) x 256 (m) output tile; its 8
// waves form a 4 x 2 grid of 64 (n) x 128 (m) wave tiles (2 x 4 blocks), two
// waves per SIMD. Operand delivery, not the MFMA, bounds this kernel, so the
// tile is as large as the register file allows (each staged operand byte
// feeds 256 outputs). A tile's stage of operand rows is one contiguous run of
// records, copied linearly into LDS by direct-to-LDS buffer loads
// (buffer_load_dwordx4 ... lds: no staging registers, no ds_write, one address
// register); the 104-byte record stride keeps the 32 rows a block reads on
// distinct LDS bank pairs, and the scales arrive inside the records. Three
// stage buffers rotate: a buffer is refilled (stage st + 3) as soon as every
// wave has read its last operand from it, at stage st's sync point in the
// middle of the stage. Every wave issues the same number of DMA loads per
// stage, so one s_waitcnt vmcnt(N) before that barrier completes exactly the
// stage read next while the newer one stays in flight. Operands live in
// registers across stages (the next group's are read right after their last
// use), so no wave waits on LDS at a stage start. The stage loop is unrolled
// by three so every LDS read names its buffer statically. Within a stage the
// 16 blocks run in a fixed order (a scheduling fence after each), keeping one
// block's P and S live; the other wave on the SIMD fills the matrix pipe
// meanwhile. The fp32 accumulators are scalars so each fma accumulates in
// place (v_fmac_f32, the 4-byte encoding). Tiles are ordered per XCD
// (xcd_tile_of) so operands stay in that XCD's L2.
#include <atomic>

#include "fp6_gemm_common.h"
#include "quant_g64.h"

namespace {


// Tile configurations: TN = 128 (64 x 64 wave tiles, registers for the
// software pipeline, four stage buffers) or TN = 256 (64 x 128 wave tiles,
// each staged byte feeds twice the outputs, three stage buffers, blocks run
// back to back); the 64 x 128 tile has one 32 x 32 block per wave and three
// stage buffers (61 KB), so two workgroups share a CU: small grids (M = 256)
// spread over twice the workgroups of the 128 x 128 tile.
template <int TM, int TN>
struct Cfg {
  static constexpr bool SMALL = TM == 64;
  static constexpr int WBN = SMALL ? 1 : 2;
  static constexpr int WAVES_N = TN / (32 * WBN);
  static constexpr int WAVES_M = NWAVES / WAVES_N;
  static constexpr int WBM = TM / (32 * WAVES_M);
  // the activation rows' region is a whole number of 1 KB copy runs (192 rows: 19.5 KB -> 20 KB; the half
  // run past the tile's rows lands in the padding)
  static constexpr int LDS_X = (TM * REC + 1023) / 1024 * 1024, OFF_W = LDS_X, LDS_W = TN * REC;
  static constexpr int STAGE = LDS_X + LDS_W;
  static constexpr int NB0 = (kLdsBytes - 2 * TN * 4) / STAGE;
  static constexpr int NBUF = SMALL ? 3 : NB0 > 4 ? 4 : NB0;  // stage buffers; DMA runs NBUF - 1 stages ahead
  static constexpr int RUNS = STAGE / 1024;        // 1 KiB DMA runs (64 lanes x 16 B) per stage
  static constexpr int DMA_X = LDS_X / 1024;
  static constexpr int SLOTS = (RUNS + NWAVES - 1) / NWAVES;  // per wave and stage
  static constexpr bool PIPE = WBN * WBM <= 4;
  static_assert(WAVES_N * WAVES_M == NWAVES && WBM * 32 * WAVES_M == TM, "wave grid");
  static_assert(LDS_X % 1024 == 0 && LDS_W % 1024 == 0 && NBUF >= 3, "stage layout");
  static_assert(NBUF * SLOTS < 64, "vmcnt range");
};

template <int TM, int TN, int RB, bool GELU, bool OUT_F16, bool NQ>
__global__ __launch_bounds__(NTHREADS, (TM == 64 ? 4 : 1)) void w4a4_gemm_fp6_kernel(
    const uint8_t* __restrict__ qa, const uint8_t* __restrict__ qw, const float* __restrict__ s2p,
    const float* __restrict__ second, int second_per_channel, const void* __restrict__ la, int la_f32,
    const uint16_t* __restrict__ up, const uint16_t* __restrict__ bias, uint16_t* __restrict__ out, int M, int N,
    int K, NextLayer nx) {
  using C = Cfg<TM, TN>;
  static_assert(!NQ || TM == 256, "the next-layer epilogue's la rows are 32 per wave: 256-row tiles");
  constexpr int WBN = C::WBN, WBM = C::WBM, WAVES_N = C::WAVES_N, NBUF = C::NBUF, SLOTS = C::SLOTS;
  constexpr int OFF_W = C::OFF_W;
  __shared__ __attribute__((aligned(16))) uint8_t g_stage[NBUF][C::STAGE];
  __shared__ __attribute__((aligned(16))) float g_epi[2 * TN];

  const int tid = threadIdx.x;
  const int tiles_n = (N + TN - 1) / TN, tiles_m = (M + TM - 1) / TM;
  int tm, tn;
  if (!xcd_tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn)) return;  // whole workgroup, before any barrier
  const int n0 = tn * TN, m0 = tm * TM;
  const int nst = K >> 7;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int wn = wave % WAVES_N, wm = wave / WAVES_N;
  const int r32 = lane & 31, h = lane >> 5;

  const v4i xbuf = raw_rsrc(qa, (uint32_t)((int64_t)nst * M * REC));
  const v4i wbuf = raw_rsrc(qw, (uint32_t)((int64_t)nst * N * REC));

  // DMA: run q of a stage is LDS bytes [1024 q, +1024) of the stage buffer =
  // bytes [1024 q', +1024) of the tile's contiguous records (q' = q for the
  // activations, q - DMA_X for the weights). Runs are dealt round-robin; a
  // wave left without a last run repeats the final run (same bytes to the
  // same place), so every wave issues SLOTS copies per stage. The offsets
  // are scalar (the hardware does not range-check the SGPR offset): a run
  // that starts past the tile's last real row reads the stage's first run
  // instead, and the one run that straddles it reads up to 1 KB past it,
  // which in the last stage is the 1 KB of slack every record buffer carries.
  const uint32_t dvo = 16u * (uint32_t)lane;
  const uint32_t x_valid = (uint32_t)(M - m0) * REC, w_valid = (uint32_t)(N - n0) * REC;
  [[maybe_unused]] const uint32_t x_bytes = (uint32_t)((int64_t)nst * M * REC);
  [[maybe_unused]] const uint32_t w_bytes = (uint32_t)((int64_t)nst * N * REC);
  auto issue = [&](uint8_t* stage, int st) __attribute__((always_inline)) {
    const uint32_t xs = (uint32_t)(((int64_t)st * M + m0) * REC);
    const uint32_t ws = (uint32_t)(((int64_t)st * N + n0) * REC);
#pragma unroll
    for (int j = 0; j < SLOTS; ++j) {
      int q = wave + NWAVES * j;
      q = q < C::RUNS ? q : C::RUNS - 1;
      const bool isx = q < C::DMA_X;
      // a run that starts past the tile's last real row re-reads the stage's first run (its rows' results are
      // never stored); a run that straddles it reads up to 1 KB past it: the record buffers' slack
      const uint32_t r0 = (uint32_t)((isx ? q : q - C::DMA_X) * 1024);
      uint32_t soff = (isx ? xs : ws) + (r0 < (isx ? x_valid : w_valid) ? r0 : 0u);
      // the run [soff, soff + 1 KB) stays within the records plus their 1 KB slack
      if (!GWA_DCHECK(soff <= (isx ? x_bytes : w_bytes), isx ? kDbgFp6CopyA : kDbgFp6CopyW, soff)) soff = isx ? xs : ws;
      dma16(isx ? xbuf : wbuf, (uint32_t)(uintptr_t)(stage + q * 1024), dvo, soff);
    }
  };

  // The low-rank operands of ranks up to 32 (la rows m0.., up rows n0..: two
  // contiguous runs) are copied into two stage buffers that no stage reads or
  // fills once stage max(nst - 2, 0)'s sync has passed (spare1 / spare2), la
  // into the first, up into the second. The wait after the loop covers them.
  constexpr bool LR_LDS = RB == 1 || RB == 2;
  const int la_row = RB * 32 * (la_f32 ? 2 : 1);  // bytes per la row
  const v4i lbuf4 = raw_rsrc(la, (uint32_t)((int64_t)M * la_row));
  const v4i ubuf4 = raw_rsrc(up, (uint32_t)((int64_t)N * RB * 32));
  auto issue_lowrank = [&](uint8_t* dla, uint8_t* dup) __attribute__((always_inline)) {
    const int la_runs = TM * la_row / 1024;
    constexpr int UP_RUNS = TN * RB * 32 / 1024;
    for (int q = wave; q < la_runs + UP_RUNS; q += NWAVES) {
      const bool isl = q < la_runs;
      const uint32_t in_run = (uint32_t)((isl ? q : q - la_runs) * 1024) + dvo;  // rows past M / N: zeros
      const uint32_t voff = isl ? (in_run < (uint32_t)((M - m0) * la_row) ? (uint32_t)(m0 * la_row) + in_run : kOOB)
                                : (in_run < (uint32_t)((N - n0) * RB * 32) ? (uint32_t)(n0 * RB * 32) + in_run : kOOB);
      dma16(isl ? lbuf4 : ubuf4, (uint32_t)(uintptr_t)(isl ? dla + q * 1024 : dup + (q - la_runs) * 1024), voff,
            0u);
    }
  };

  // NQ: the next layer's proj_down operands for this tile's TN columns (one contiguous run of
  // (TN / 128) * nx.rb * 4 KB in the fp6 act-quant order) are copied into the LDS past the staged output
  // tile at the start of the epilogue, when they fit; else the epilogue loads them from global memory
  constexpr int OSTR = TN * 2 + 8;  // output staging row stride (bytes); 8-byte pad: distinct banks per write
  constexpr int NQ_PDO_OFF = (TM * OSTR + 1023) / 1024 * 1024;
  const int pdo_runs = NQ ? (TN / 128) * nx.rb * 4 : 0;
  const bool pdo_lds = NQ && nx.pdo != nullptr && nx.rb > 0 && NQ_PDO_OFF + pdo_runs * 1024 <= NBUF * C::STAGE;
  const v4i pdo4 = raw_rsrc(nx.pdo, NQ ? (uint32_t)((int64_t)(N >> 7) * nx.rb * 4096) : 0u);
  auto issue_next_pdo = [&](uint8_t* dst) __attribute__((always_inline)) {
    const uint32_t base = (uint32_t)(n0 >> 7) * (uint32_t)nx.rb * 4096u;
    const uint32_t valid = (uint32_t)((N - n0 + 127) >> 7) * (uint32_t)nx.rb * 4096u;  // stages past N: none
    for (int q = wave; q < pdo_runs; q += NWAVES) {
      const uint32_t in_run = (uint32_t)q * 1024u + dvo;
      dma16(pdo4, (uint32_t)(uintptr_t)(dst + q * 1024), in_run < valid ? base + in_run : kOOB, 0u);
    }
  };

  // the main loop's fp32 accumulators, as scalars: each block's fmas then accumulate in place (v_fmac)
  float acc[WBN][WBM][16];
#pragma unroll
  for (int a = 0; a < WBN; ++a)
#pragma unroll
    for (int b = 0; b < WBM; ++b)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[a][b][v] = 0.0f;
  auto pin16 = [](float* a) __attribute__((always_inline)) {
    asm volatile("" : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(a[4]), "+v"(a[5]), "+v"(a[6]), "+v"(a[7]),
                 "+v"(a[8]), "+v"(a[9]), "+v"(a[10]), "+v"(a[11]), "+v"(a[12]), "+v"(a[13]), "+v"(a[14]), "+v"(a[15]));
  };

  // Pending P and S of the previous block (software pipeline, TN = 128): the
  // pipeline starts with zero products "pending" for the last block, so the
  // pending block is a compile-time constant everywhere.
  v16f pp = (v16f){}, ps = (v16f){};
  constexpr int kLast = WBN * WBM - 1;
  auto fma_half = [&](int blk, int half) __attribute__((always_inline)) {
#pragma unroll
    for (int a = 0; a < WBN; ++a)
#pragma unroll
      for (int b = 0; b < WBM; ++b)
        if (blk == a * WBM + b) {
#pragma unroll
          for (int v = 8 * half; v < 8 * half + 8; ++v) acc[a][b][v] = fmaf(pp[v], ps[v], acc[a][b][v]);
        }
  };
  auto pin_acc = [&](int blk) __attribute__((always_inline)) {
#pragma unroll
    for (int a = 0; a < WBN; ++a)
#pragma unroll
      for (int b = 0; b < WBM; ++b)
        if (blk == a * WBM + b) pin16(acc[a][b]);
  };

  // The operands of the group about to run (both operands' 32-code halves and
  // the stage's scales) live in registers across stages; each is refilled
  // with the next group's right after its last use, so LDS reads overlap the
  // MFMAs and fmas. Group 0 refills group 1's operands from this stage's
  // buffer; group 1 refills group 0's (and the scales) from the next stage's
  // buffer, which is complete only after that stage's copies are waited for
  // and the workgroup barrier: `sync` runs inside group 1 before its first
  // read of the next buffer (after the first bn row of blocks, whose
  // operands are already in registers), so no wave starts a stage waiting for
  // LDS. Empty asm statements pin the pure MFMA intrinsics to their place in
  // program order.
  //  * PIPE: one step per block b issues b's two MFMAs between the two halves
  //    of block b-1's 16 fmas (whose P and S completed during step b-1), in
  //    scheduling groups MFMA, 8 VALU, MFMA, 8 VALU; the step's end takes
  //    b-1's accumulator and P_b / S_b, so nothing leaves its step. The
  //    stage's last block hands its P and S to the next stage.
  //  * otherwise: each block's MFMAs, then its 16 fmas (one block's P and S
  //    live); the other wave on the SIMD fills the matrix pipe meanwhile.
  v8i xo[WBM], wo[WBN];
  uint32_t xs[WBM], ws[WBN];
  const int xrow = (32 * WBM * wm + r32) * REC, wrow = OFF_W + (32 * WBN * wn + r32) * REC;
  auto read_x = [&](const uint8_t* base, int bm, int gi) __attribute__((always_inline)) {
    xo[bm] = lds_operand(base + xrow + bm * 32 * REC + 24 * h + gi * GB);
  };
  auto read_w = [&](const uint8_t* base, int bn, int gi) __attribute__((always_inline)) {
    wo[bn] = lds_operand(base + wrow + bn * 32 * REC + 24 * h + gi * GB);
  };
  auto read_xs = [&](const uint8_t* base, int bm) __attribute__((always_inline)) {
    xs[bm] = *(const uint32_t*)(base + xrow + bm * 32 * REC + OFF_SC);
  };
  auto read_ws = [&](const uint8_t* base, int bn) __attribute__((always_inline)) {
    const uint32_t v = *(const uint32_t*)(base + wrow + bn * 32 * REC + OFF_SC);
    ws[bn] = h ? 0u : v;  // K slots 4..7 (lanes 32..63) stay zero
  };

  // the spare buffers for the low-rank operands: neither is read or filled
  // again once stage max(nst - 2, 0)'s sync has passed
  uint8_t* const spare1 = &g_stage[0][0] + (nst % NBUF) * C::STAGE;
  uint8_t* const spare2 = &g_stage[0][0] + ((nst + 1) % NBUF) * C::STAGE;
  // stage st's sync: stage st + 1 complete (this wave's copies, then
  // everyone's; the barrier also retires every wave's reads of this stage's
  // buffer), then this stage's buffer takes stage st + NBUF
  auto sync = [&](int st, uint8_t* buf) __attribute__((always_inline)) {
    if (st + 1 < nst) {
      // copies issued after stage st + 1's: stages st + 2 .. min(st + NBUF - 1, nst - 1)
      wait_stages<SLOTS, NBUF - 2>(min(NBUF - 2, nst - 2 - st));
      barrier_lds();
    }
    if (st + NBUF < nst) issue(buf, st + NBUF);
    if constexpr (LR_LDS) {
      if (st == max(nst - 2, 0)) issue_lowrank(spare1, spare2);
    }
  };

  // One stage's blocks, in (bn, bm) order, on operands already in registers.
  auto stage = [&](int st, uint8_t* cur, const uint8_t* nxt) __attribute__((always_inline)) {
    int prev = kLast;
#pragma unroll
    for (int gi = 0; gi < GS; ++gi) {
      const uint32_t mask = gi ? 0xFFFF0000u : 0x0000FFFFu;
#pragma unroll
      for (int bn = 0; bn < WBN; ++bn) {
        const v4h swop = __builtin_bit_cast(v4h, make_uint2(ws[bn], 0u));
#pragma unroll
        for (int bm = 0; bm < WBM; ++bm) {
          uint32_t s1 = xs[bm] & mask;
          if constexpr (C::PIPE) {
            asm volatile("" : "+v"(s1), "+v"(xo[bm]), "+v"(wo[bn]));  // step start
            const v4h sel = __builtin_bit_cast(v4h, make_uint2(s1, 0u));
            v16f p = group_mfma_fp6(wo[bn], xo[bm]);
            fma_half(prev, 0);
            v16f sv = __builtin_amdgcn_mfma_f32_32x32x8f16(swop, sel, (v16f){}, 0, 0, 0);
            fma_half(prev, 1);
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);
            pin_acc(prev);
            asm volatile("" : "+v"(p), "+v"(sv));  // step end
            pp = p;
            ps = sv;
            prev = bn * WBM + bm;
          } else {
            asm volatile("" : "+v"(s1));  // keeps this S MFMA here (it would otherwise be hoisted to the stage start)
            const v4h sel = __builtin_bit_cast(v4h, make_uint2(s1, 0u));
            const v16f p = group_mfma_fp6(wo[bn], xo[bm]);
            const v16f sv = __builtin_amdgcn_mfma_f32_32x32x8f16(swop, sel, (v16f){}, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[bn][bm][v] = fmaf(p[v], sv[v], acc[bn][bm][v]);
            pin16(acc[bn][bm]);  // this block's fmas complete here, in program order
          }
          if (gi == 0) {
            if (bn == WBN - 1) read_x(cur, bm, 1);
            if (bm == WBM - 1) read_w(cur, bn, 1);
          } else {
            // past the last stage the reads below fetch unused values (in bounds of the LDS)
            if (bn == 0 && bm == WBM - 1) sync(st, cur);
            if (bn == WBN - 1) {
              read_x(nxt, bm, 0);
              read_xs(nxt, bm);
            }
            if (bm == WBM - 1) {
              read_w(nxt, bn, 0);
              read_ws(nxt, bn);
            }
          }
        }
      }
    }
  };

  // the epilogue constants' loads go out first; they are older than every copy, so the stage waits below cover
  // them too
  const EpiConsts epc = epi_consts_load(s2p, second, second_per_channel, bias, n0, tid, TN, N);
  // stages 0 .. NBUF - 1 in flight; stage 0 complete; its first group's operands and scales into registers
#pragma unroll
  for (int u = 0; u < NBUF; ++u)
    if (u < nst) issue(g_stage[u], u);
  wait_stages<SLOTS, NBUF - 1>(min(NBUF - 1, nst - 1));
  barrier_lds();
#pragma unroll
  for (int bn = 0; bn < WBN; ++bn) {
    read_w(g_stage[0], bn, 0);
    read_ws(g_stage[0], bn);
  }
#pragma unroll
  for (int bm = 0; bm < WBM; ++bm) {
    read_x(g_stage[0], bm, 0);
    read_xs(g_stage[0], bm);
  }
  // unrolled by NBUF so every LDS address is static
  for (int st = 0; st < nst; st += NBUF) {
#pragma unroll
    for (int u = 0; u < NBUF; ++u)
      if (st + u < nst) stage(st + u, g_stage[u], g_stage[(u + 1) % NBUF]);
  }
  if constexpr (C::PIPE) {
    fma_half(kLast, 0);
    fma_half(kLast, 1);
  }
  epi_consts_store(epc, s2p, second, bias, g_epi, tid, TN);
  wait_vm_lgkm0<0>();  // the low-rank copies (and the reads past the last stage) complete
  barrier_lds();

  // ---------------- epilogue ----------------
  v16f accv[WBN][WBM];
#pragma unroll
  for (int a = 0; a < WBN; ++a)
#pragma unroll
    for (int b = 0; b < WBM; ++b)
#pragma unroll
      for (int v = 0; v < 16; ++v) accv[a][b][v] = acc[a][b][v];
#pragma unroll
  for (int bn = 0; bn < WBN; ++bn) {
    const int nl = 32 * (WBN * wn + bn);
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) {
      const v4f cm = *(const v4f*)(g_epi + nl + 8 * qd + 4 * h);
#pragma unroll
      for (int bm = 0; bm < WBM; ++bm)
#pragma unroll
        for (int e = 0; e < 4; ++e) accv[bn][bm][4 * qd + e] *= cm[e];
    }
  }
  if constexpr (LR_LDS) {
    // la / up from the two stage buffers after the last stage's
    const uint8_t* lrb = &g_stage[0][0] + (nst % NBUF) * C::STAGE;
    const uint8_t* upb = &g_stage[0][0] + ((nst + 1) % NBUF) * C::STAGE;
#pragma unroll
    for (int k0 = 0; k0 < RB; ++k0) {
      v4i ua[WBN], lb[WBM];
#pragma unroll
      for (int bn = 0; bn < WBN; ++bn)
        ua[bn] = *(const v4i*)(upb + (32 * (WBN * wn + bn) + r32) * (RB * 32) + k0 * 32 + 16 * h);
#pragma unroll
      for (int bm = 0; bm < WBM; ++bm)
        lb[bm] = la_operand_lds(lrb, 32 * (WBM * wm + bm) + r32, la_row, k0 * 16 + 8 * h, la_f32);
#pragma unroll
      for (int bn = 0; bn < WBN; ++bn)
#pragma unroll
        for (int bm = 0; bm < WBM; ++bm)
          accv[bn][bm] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, ua[bn]),
                                                                __builtin_bit_cast(v8bf, lb[bm]), accv[bn][bm], 0, 0, 0);
    }
  } else if constexpr (RB > 0) {
    constexpr int RC = 1;
    const rsrc_t ubuf = make_rsrc(up, (uint32_t)((int64_t)N * RB * 32));
    const rsrc_t lbuf = make_rsrc(la, (uint32_t)((int64_t)M * la_row));
#pragma unroll
    for (int k0 = 0; k0 < RB; k0 += RC) {
      v4i ua[WBN][RC], lb[WBM][RC];
#pragma unroll
      for (int bn = 0; bn < WBN; ++bn)
#pragma unroll
        for (int kk = 0; kk < RC; ++kk)
          ua[bn][kk] = buf_load16(
              ubuf, (uint32_t)((int64_t)(n0 + 32 * (WBN * wn + bn) + r32) * (RB * 32) + (k0 + kk) * 32 + 16 * h));
#pragma unroll
      for (int bm = 0; bm < WBM; ++bm)
#pragma unroll
        for (int kk = 0; kk < RC; ++kk) {
          const uint32_t row_off = (uint32_t)((int64_t)(m0 + 32 * (WBM * wm + bm) + r32) * la_row);
          const int k = (k0 + kk) * 16 + 8 * h;
          if (la_f32) {
            const v4i a = buf_load16(lbuf, row_off + k * 4), b = buf_load16(lbuf, row_off + k * 4 + 16);
            const v4f fa = __builtin_bit_cast(v4f, a), fb = __builtin_bit_cast(v4f, b);
            lb[bm][kk] = (v4i){(int)pack_bf16x2_rn(fa[0], fa[1]), (int)pack_bf16x2_rn(fa[2], fa[3]),
                               (int)pack_bf16x2_rn(fb[0], fb[1]), (int)pack_bf16x2_rn(fb[2], fb[3])};
          } else {
            lb[bm][kk] = buf_load16(lbuf, row_off + k * 2);
          }
        }
#pragma unroll
      for (int bn = 0; bn < WBN; ++bn)
#pragma unroll
        for (int bm = 0; bm < WBM; ++bm)
#pragma unroll
          for (int kk = 0; kk < RC; ++kk)
            accv[bn][bm] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, ua[bn][kk]),
                                                                  __builtin_bit_cast(v8bf, lb[bm][kk]), accv[bn][bm],
                                                                  0, 0, 0);
    }
  }
  // + bias (+ GELU), packed to 16 bits, staged in LDS as [m][n] rows of OSTR
  // bytes (the stage buffers are free; the barrier also retires the la / up
  // reads), then stored as full rows: each lane 16 bytes, 32 lanes per 512
  // bytes of a row, so every wave store covers whole 128-byte lines.
  static_assert(TM * OSTR <= NBUF * C::STAGE, "output staging");
  uint8_t* ob = &g_stage[0][0];
  barrier_lds();
  if constexpr (NQ) {
    if (pdo_lds) issue_next_pdo(ob + NQ_PDO_OFF);  // past the staged tile; completes behind the staging
  }
#pragma unroll
  for (int bn = 0; bn < WBN; ++bn) {
    const int nl = 32 * (WBN * wn + bn);
#pragma unroll
    for (int bm = 0; bm < WBM; ++bm) {
      const int ml = 32 * (WBM * wm + bm) + r32;
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        const int nn = nl + 8 * qd + 4 * h;
        const v4f cb = *(const v4f*)(g_epi + TN + nn);
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float t = accv[bn][bm][4 * qd + e] + cb[e];
          if (GELU) t = gelu_tanh_f32(t);
          o[e] = t;
        }
        uint2 pk;
        if (OUT_F16) {
          pk.x = pack_f16x2(o[0], o[1]);
          pk.y = pack_f16x2(o[2], o[3]);
        } else {
          pk.x = pack_bf16x2_rn(o[0], o[1]);
          pk.y = pack_bf16x2_rn(o[2], o[3]);
        }
        *(uint2*)(ob + ml * OSTR + nn * 2) = pk;
      }
    }
  }
  barrier_lds();
  constexpr int CPR = TN / 8;                 // 16-byte chunks per row
  constexpr int RPP = NTHREADS / CPR;         // rows per pass
  const int crow = tid / CPR, cch = tid % CPR;
  if constexpr (NQ) {
    if (pdo_lds) {  // this wave's copies, then everyone's
      wait_vm_lgkm0<0>();
      barrier_lds();
    }
    // ---- la_next[m0 + rows, :] += tile[rows, :] @ proj_down_next[n0 .. n0 + TN, :]: wave w takes rows
    // 32w .. 32w + 31 (two 16-row MFMA blocks); per 128-column stage, k-step j, lane (r, c) = (lane % 16,
    // lane / 16) supplies columns 32c + 8j .. +8 of row r, the order gwa_svdq_prep_proj_down_fp6 arranges
    // proj_down in
    if (nx.pdo != nullptr && nx.rb > 0) {
      const rsrc_t pb = make_rsrc(nx.pdo, (uint32_t)((int64_t)(N >> 7) * nx.rb * 4096));
      const uint8_t* pl = ob + NQ_PDO_OFF + 16 * lane;
      v4f lacc[2][kNextRbMax];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int rb = 0; rb < kNextRbMax; ++rb) lacc[i][rb] = (v4f){0.f, 0.f, 0.f, 0.f};
      // MFMA block i of wave w: rows 32w + 2r + i (r = lane % 16): a stride of two rows puts the 16 rows of a
      // read on distinct LDS banks
      const uint8_t* arow = ob + (32 * wave + 2 * (lane & 15)) * OSTR + 64 * (lane >> 4);
#pragma unroll
      for (int ts = 0; ts < TN / 128; ++ts) {
        const int sg = (n0 >> 7) + ts;
        if (128 * sg >= N) break;  // the tile's columns past N (N % 128 == 0: whole stages)
#pragma unroll 2
        for (int j = 0; j < 4; ++j) {
          const uint8_t* ar = arow + (128 * ts + 8 * j) * 2;
          const v4i a0 = *(const v4i*)ar;
          const v4i a1 = *(const v4i*)(ar + OSTR);
#pragma unroll
          for (int rb = 0; rb < kNextRbMax; ++rb) {
            if (rb < nx.rb) {
              const v4i b = pdo_lds ? *(const v4i*)(pl + ((ts * 4 + j) * nx.rb + rb) * 1024)
                                    : buf_load16(pb, (uint32_t)(((((int64_t)sg * 4 + j) * nx.rb + rb) * 64 + lane) * 16));
              lacc[0][rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, a0),
                                                                    __builtin_bit_cast(v8bf, b), lacc[0][rb], 0, 0, 0);
              lacc[1][rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, a1),
                                                                    __builtin_bit_cast(v8bf, b), lacc[1][rb], 0, 0, 0);
            }
          }
        }
      }
      const int R = nx.rb * 16;
      float* slot = nx.la_part + (int64_t)tn * M * R;  // this column tile's partial
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int rb = 0; rb < kNextRbMax; ++rb) {
          if (rb < nx.rb) {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              const int m = m0 + 32 * wave + 2 * (4 * (lane >> 4) + t) + i;
              if (m < M) slot[(int64_t)m * R + 16 * rb + (lane & 15)] = lacc[i][rb][t];
            }
          }
        }
    }
  }
  if (!NQ || out != nullptr) {
    const rsrc_t obuf = make_rsrc(out, (uint32_t)((int64_t)M * N * 2));
    const bool col_ok = n0 + 8 * cch < N;
#pragma unroll 4
    for (int r0 = 0; r0 < TM; r0 += RPP) {
      const int row = r0 + crow;
      const uint2 lo = *(const uint2*)(ob + row * OSTR + cch * 16);
      const uint2 hi = *(const uint2*)(ob + row * OSTR + cch * 16 + 8);
      uint32_t off =
          (col_ok && m0 + row < M) ? (uint32_t)(((int64_t)(m0 + row) * N + n0 + 8 * cch) * 2) : kOOB;
      if (!GWA_DCHECK(off == kOOB || (int64_t)off + 16 <= (int64_t)M * N * 2, kDbgFp6Out, off)) off = kOOB;
      buf_store16((v4i){(int)lo.x, (int)lo.y, (int)hi.x, (int)hi.y}, obuf, off);
    }
  }
  if constexpr (NQ) {
    // ---- the next layer's fp6 records (its K = this N; N % 128 == 0, so every column is real).
    // Thread -> 32 fixed consecutive columns (half a group; the other half in lane ^ 1), rows crow, crow +
    // RPP32, ...: the fp6 act-quant kernel's per-lane quantizer, so the records match it bit for bit.
    constexpr int CPR32 = TN / 32, RPP32 = NTHREADS / CPR32;
    const int crow32 = tid / CPR32, cch32 = tid % CPR32;
    const int col = n0 + 32 * cch32;
    float f[32];
    bool divide = false;
    if (nx.smooth) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        // columns past N (the second half of a 256-wide tile when N % 256 == 128): any real factors (those
        // rows' records fall past the buffer and are not stored)
        const v4i sv = *(const v4i*)(nx.smooth + (col < N ? col : 0) + 8 * q);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          f[8 * q + 2 * j] = bf16_lo((uint32_t)sv[j]);
          f[8 * q + 2 * j + 1] = bf16_hi((uint32_t)sv[j]);
        }
      }
#pragma unroll
      for (int t = 0; t < 32; ++t) divide |= !g64::smooth_ok(f[t]);
      divide = __builtin_amdgcn_ballot_w64(divide) != 0;  // wave-uniform: both paths give the same bf16
      if (!divide) {
#pragma unroll
        for (int t = 0; t < 32; ++t) f[t] = 1.0f / f[t];
      }
    }
    const rsrc_t qb = make_rsrc(nx.q6, (uint32_t)((int64_t)(N >> 7) * M * REC));
    const int nstage = col >> 7;
    const uint32_t in_rec = (uint32_t)(48 * ((cch32 >> 1) & 1) + 24 * (cch32 & 1));
    // the scales at 96 + 2 g from the even lanes, zeros into the unused bytes 100..103 from the odd ones
    const uint32_t sc_off = (uint32_t)(96 + 2 * ((cch32 >> 1) & 1) + 4 * (cch32 & 1));
#pragma unroll 1
    for (int r0 = 0; r0 < TM; r0 += RPP32) {
      const int row = r0 + crow32;
      const bool valid = m0 + row < M;
      float v[32];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const v4i c = *(const v4i*)(ob + row * OSTR + cch32 * 64 + 16 * q);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          v[8 * q + 2 * j] = bf16_lo((uint32_t)c[j]);
          v[8 * q + 2 * j + 1] = bf16_hi((uint32_t)c[j]);
        }
      }
      if (nx.smooth) g64::smooth32(v, f, divide);
      uint32_t mu = g64::absmax_bits32(v);
      mu = max(mu, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mu, 0xB1, 0xF, 0xF, false));  // lane ^ 1
      g64::v6u pk;
      uint16_t sh;
      g64::quant32(v, mu, valid, true, 1.0f, pk, sh);
      const uint32_t rec = (uint32_t)(((int64_t)nstage * M + m0 + row) * REC);
      buf_store16((v4i){(int)pk[0], (int)pk[1], (int)pk[2], (int)pk[3]}, qb, valid ? rec + in_rec : kOOB);
      buf_store8(make_uint2(pk[4], pk[5]), qb, valid ? rec + in_rec + 16u : kOOB);
      buf_store2((cch32 & 1) ? (uint16_t)0 : sh, qb, valid ? rec + sc_off : kOOB);
    }
  }
}

// Exact per-group partial sums through the same fp6 MFMA (debug / parity):
// out[m][n][g] = sum_{k in g} qa[m][k] * qw[n][k], one wave per 32 x 32 block.
__global__ __launch_bounds__(64) void w4a4_psums_fp6_kernel(const uint8_t* __restrict__ qa,
                                                            const uint8_t* __restrict__ qw,
                                                            int32_t* __restrict__ out, int M, int N, int K) {
  const int lane = threadIdx.x, r32 = lane & 31, h = lane >> 5;
  const int m0 = blockIdx.x * 32, n0 = blockIdx.y * 32;
  const int G = K >> 6, nst = K >> 7;
  const int m = m0 + r32, nr = n0 + r32;
  const rsrc_t xbuf = make_rsrc(qa, (uint32_t)((int64_t)nst * M * REC));
  const rsrc_t wbuf = make_rsrc(qw, (uint32_t)((int64_t)nst * N * REC));
  const rsrc_t obuf = make_rsrc(out, (uint32_t)((int64_t)M * N * G * 4));
  for (int g = 0; g < G; ++g) {
    const int st = g >> 1, in = (g & 1) * GB + 24 * h;
    // rows past M / N load zeros
    const v8i a = buf_operand(wbuf, nr < N ? (uint32_t)(((int64_t)st * N + nr) * REC + in) : kOOB);
    const v8i b = buf_operand(xbuf, m < M ? (uint32_t)(((int64_t)st * M + m) * REC + in) : kOOB);
    const v16f p = group_mfma_fp6(a, b);
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int n = n0 + 8 * (v >> 2) + 4 * h + (v & 3);
      const uint32_t off = (m < M && n < N) ? (uint32_t)((((int64_t)m * N + n) * G + g) * 4) : kOOB;
      buf_store4((uint32_t)(int32_t)p[v], obuf, off);
    }
  }
}

// int4 weight rows (two's-complement nibbles, element 2j in the low nibble of
// byte j) + fp16 group scales -> fp6 operand records: one thread per (row,
// group, half) turns 16 bytes (32 codes) into 24 bytes with code t at bits
// [6t, 6t + 6); the first half also stores the group's scale and, for the
// stage's first group, zeros the record's unused bytes.
__global__ __launch_bounds__(256) void pack_weight_fp6_kernel(const uint8_t* __restrict__ qw,
                                                              const uint16_t* __restrict__ sw,
                                                              uint8_t* __restrict__ qw6, int N, int K) {
  const int G = K >> 6, GP = 2 * ((K + 127) >> 7);  // groups, and groups of the records (a half stage: G + 1)
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)N * GP * 2) return;
  const int64_t row = i / (2 * GP);
  const int rem = (int)(i - row * 2 * GP), g = rem >> 1, hh = rem & 1;
  const bool pad = g >= G;  // the half stage's second group: zero codes, zero scale
  const uint32_t* src = (const uint32_t*)(qw + row * (K / 2) + (pad ? 0 : g * 32 + hh * 16));
  uint64_t pc[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const uint32_t w = pad ? 0u : src[d];
    const uint32_t ev = w & 0x0F0F0F0Fu, od = (w >> 4) & 0x0F0F0F0Fu;  // codes 8d + 0,2,4,6 / 8d + 1,3,5,7
    const uint32_t c0 = __builtin_amdgcn_perm(od, ev, 0x05010400u);    // codes 8d + 0..3, one per byte
    const uint32_t c1 = __builtin_amdgcn_perm(od, ev, 0x07030602u);    // codes 8d + 4..7
    pc[d] = (uint64_t)pack6_x4(e3m2_x4(c0)) | ((uint64_t)pack6_x4(e3m2_x4(c1)) << 24);
  }
  uint8_t* rec = qw6 + ((int64_t)(g >> 1) * N + row) * REC;
  uint32_t* dst = (uint32_t*)(rec + (g & 1) * GB + hh * 24);
  dst[0] = (uint32_t)pc[0];
  dst[1] = (uint32_t)((pc[0] >> 32) | (pc[1] << 16));
  dst[2] = (uint32_t)(pc[1] >> 16);
  dst[3] = (uint32_t)pc[2];
  dst[4] = (uint32_t)((pc[2] >> 32) | (pc[3] << 16));
  dst[5] = (uint32_t)(pc[3] >> 16);
  if (hh == 0) {
    *(uint16_t*)(rec + OFF_SC + (g & 1) * 2) = pad ? (uint16_t)0 : sw[row * G + g];
    if ((g & 1) == 0) *(uint32_t*)(rec + OFF_SC + 4) = 0u;
  }
}

}  // namespace

extern "C" int gwa_svdq_pack_weight_fp6(const uint8_t* qw, const void* sw, uint8_t* qw6, int64_t N, int64_t K,
                                        void* stream) {
  GWA_REQUIRE(N > 0 && K > 0 && K % 64 == 0, "svdq_pack_weight_fp6: bad shape N=%lld K=%lld (K %% 64 == 0)",
              (long long)N, (long long)K);
  GWA_REQUIRE(N * (K / 64) * 2 < (1ll << 40) && K < (1ll << 30), "svdq_pack_weight_fp6: shape too large");
  GWA_REQUIRE(qw && sw && qw6, "svdq_pack_weight_fp6: null pointer");
  GWA_REQUIRE(GWA_ALIGNED(qw, 4) && GWA_ALIGNED(qw6, 8) && GWA_ALIGNED(sw, 2), "svdq_pack_weight_fp6: misaligned pointer");
  const int64_t threads = N * ((K + 127) / 128) * 2 * 2;  // (row, group of the records, half)
  hipLaunchKernelGGL(pack_weight_fp6_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, qw, (const uint16_t*)sw, qw6, (int)N, (int)K);
  return gwa_check_launch("svdq_pack_weight_fp6");
}

extern "C" int gwa_svdq_group_psums_fp6(const uint8_t* qa6, int64_t qa6_bytes, const uint8_t* qw6,
                                        int64_t qw6_bytes, int32_t* out, int64_t M, int64_t N, int64_t K,
                                        void* stream) {
  GWA_REQUIRE(M >= 0 && N >= 0 && K > 0 && K % 128 == 0, "svdq_group_psums_fp6: bad shape (K %% 128 == 0)");
  GWA_REQUIRE(M < (1ll << 31) && N < (1ll << 30) && K < (1ll << 30) && M * N * (K / 64) * 4 < (1ll << 31) &&
                  M * (K / 128) * REC < (1ll << 31) && N * (K / 128) * REC < (1ll << 31),
              "svdq_group_psums_fp6: shape too large (buffers must stay below 2 GiB)");
  GWA_REQUIRE((N + 31) / 32 < 65536, "svdq_group_psums_fp6: N too large");
  if (M == 0 || N == 0) return GWA_OK;
  // this kernel reads each lane's record bytes through range-checked lane offsets: the records, no slack
  GWA_REQUIRE(qa6_bytes >= (K / 128) * M * REC && qw6_bytes >= (K / 128) * N * REC,
              "svdq_group_psums_fp6: record buffers of %lld / %lld bytes, the shape needs %lld / %lld",
              (long long)qa6_bytes, (long long)qw6_bytes, (long long)((K / 128) * M * REC),
              (long long)((K / 128) * N * REC));
  GWA_REQUIRE(qa6 && qw6 && out, "svdq_group_psums_fp6: null pointer");
  GWA_REQUIRE(GWA_ALIGNED(qa6, 8) && GWA_ALIGNED(qw6, 8) && GWA_ALIGNED(out, 4),
              "svdq_group_psums_fp6: misaligned pointer");
  hipLaunchKernelGGL(w4a4_psums_fp6_kernel, dim3((unsigned)((M + 31) / 32), (unsigned)((N + 31) / 32)), dim3(64), 0,
                     (hipStream_t)stream, qa6, qw6, out, (int)M, (int)N, (int)K);
  return gwa_check_launch("svdq_group_psums_fp6");
}

namespace {

// tile shapes: 256 x 256 and 192 x 256 (128 x 64 and 96 x 64 wave tiles), 256 x 128 and 128 x 128 (64 x 64
// and 32 x 64 wave tiles, with the software pipeline), and the pipelined kernel's 288 x 192 and 256 x 192
// (w4a4_gemm_fp6_pipe.hip)
enum Fp6Tile {
  kTile256x256 = 0, kTile256x128 = 1, kTile128x128 = 2, kTile192x256 = 3, kTile288x192 = 4, kTile256x192 = 5,
  kTile64x128 = 6, kTileCount = 7
};
bool fp6_tile_pipelined(int tile) { return tile == kTile288x192 || tile == kTile256x192; }

template <int TM, int TN, int RB, bool GL, bool F16, bool NQ>
void launch_fp6_tile(dim3 grid, hipStream_t s, const GwaFp6Args& a, const NextLayer& nx) {
  hipLaunchKernelGGL((w4a4_gemm_fp6_kernel<TM, TN, RB, GL, F16, NQ>), grid, dim3(NTHREADS), 0, s, a.qa6, a.qw6, a.s2,
                     a.second, a.per_channel, a.la, a.la_f32, a.up, a.bias, a.out, a.M, a.N, a.K, nx);
}

template <int RB, bool GL, bool F16, bool NQ>
void launch_fp6_rb(int tile, dim3 grid, hipStream_t s, const GwaFp6Args& a, const NextLayer& nx) {
  if (tile == kTile256x256)
    launch_fp6_tile<256, 256, RB, GL, F16, NQ>(grid, s, a, nx);
  else if (!NQ && tile == kTile192x256)
    launch_fp6_tile<192, 256, RB, GL, F16, false>(grid, s, a, nx);
  else if (NQ || tile == kTile256x128)
    launch_fp6_tile<256, 128, RB, GL, F16, NQ>(grid, s, a, nx);
  else if (tile == kTile64x128)
    launch_fp6_tile<64, 128, RB, GL, F16, false>(grid, s, a, nx);
  else
    launch_fp6_tile<128, 128, RB, GL, F16, false>(grid, s, a, nx);
}

template <int RB>
void launch_fp6_flags(int tile, bool gelu, bool f16, bool nq, dim3 grid, hipStream_t s, const GwaFp6Args& a,
                      const NextLayer& nx) {
  if (nq) {  // the next layer's input is bf16: no f16 variant
    if (gelu) launch_fp6_rb<RB, true, false, true>(tile, grid, s, a, nx);
    else launch_fp6_rb<RB, false, false, true>(tile, grid, s, a, nx);
  } else if (gelu) {
    if (f16) launch_fp6_rb<RB, true, true, false>(tile, grid, s, a, nx);
    else launch_fp6_rb<RB, true, false, false>(tile, grid, s, a, nx);
  } else {
    if (f16) launch_fp6_rb<RB, false, true, false>(tile, grid, s, a, nx);
    else launch_fp6_rb<RB, false, false, false>(tile, grid, s, a, nx);
  }
}

// One workgroup per CU (the stage buffers fill the LDS; the 64 x 128 tile fits twice), so a grid runs in
// rounds of kCus tiles. A grid takes the tile shape with the least estimated time: rounds x the tile's MACs x
// its time per MAC relative to the 256 x 256 tile (one round of each at M=256, N=9216, K=3072: 51.4, 31.9,
// 23.0 us for 36 256 x 256, 72 256 x 128 and 144 128 x 128 tiles; at M=1024: 54.3 and 44.0 us for 144
// 256 x 256 and 216 192 x 256 tiles; one round of the 288 x 192 and 256 x 192 tiles at K=3072: 54.3 and
// 43.9 us against 54.9 and 54.6 us for the 256 x 256 tile; 64 x 128: 15.5 us alone on a CU, 23.0 us with two
// to a CU). The next-layer epilogue needs the 256-row, 256- or 128-column tiles.
constexpr int kCus = 256;
struct Fp6Shape {
  int tile, tm, tn;
  double per_mac;         // one workgroup per CU
  double per_mac_shared;  // two workgroups on a CU (0: the tile fills a CU's LDS)
};
constexpr Fp6Shape kFp6Shapes[kTileCount] = {
    {kTile256x256, 256, 256, 1.0, 0},  {kTile256x128, 256, 128, 1.24, 0}, {kTile128x128, 128, 128, 1.80, 0},
    {kTile192x256, 192, 256, 1.08, 0}, {kTile288x192, 288, 192, 1.17, 0}, {kTile256x192, 256, 192, 1.07, 0},
    {kTile64x128, 64, 128, 2.26, 3.35}};
std::atomic<int> g_force_tile{-1};  // test / tuning hook (gwa_svdq_gemm_w4a4_fp6_force_tile)

bool fp6_tile_allowed(int tile, bool nq) { return !nq || tile == kTile256x256 || tile == kTile256x128; }

int fp6_tile(int64_t M, int64_t N, bool nq) {
  const int forced = g_force_tile.load(std::memory_order_relaxed);
  if (forced >= 0 && forced < kTileCount && fp6_tile_allowed(forced, nq)) return forced;
  int best = kTile256x256;
  double best_t = 0.0;
  for (const Fp6Shape& sh : kFp6Shapes) {
    if (!fp6_tile_allowed(sh.tile, nq)) continue;
    const int64_t tiles = ((M + sh.tm - 1) / sh.tm) * ((N + sh.tn - 1) / sh.tn);
    // a tile that fits twice on a CU runs alone while the grid fits the CUs, two to a CU beyond that
    const double t = sh.per_mac_shared == 0.0 || tiles <= kCus
                         ? (double)((tiles + kCus - 1) / kCus) * sh.tm * sh.tn * sh.per_mac
                         : (double)((tiles + 2 * kCus - 1) / (2 * kCus)) * sh.tm * sh.tn * sh.per_mac_shared;
    if (sh.tile == kTile256x256 || t < best_t * 0.999) {
      best = sh.tile;
      best_t = t;
    }
  }
  return best;
}
int fp6_tile_m(int tile) { return kFp6Shapes[tile].tm; }
int fp6_tile_n(int tile) { return kFp6Shapes[tile].tn; }

// shared argument checks and launch of both GEMM entry points (nx.q6 != NULL: the NQ epilogue)
int gemm_fp6(const char* what, const uint8_t* qa6, int64_t qa6_bytes, const uint8_t* qw6, int64_t qw6_bytes,
             const float* s2, const float* second, int64_t second_numel, const void* la, const void* up, int64_t rank,
             const void* bias, void* out, int out_dtype, int epilogue_flags, int64_t M, int64_t N, int64_t K,
             const NextLayer& nx, void* stream) {
  GWA_REQUIRE(M >= 0 && N > 0 && K > 0, "%s: bad shape M=%lld N=%lld K=%lld", what, (long long)M, (long long)N,
              (long long)K);
  GWA_REQUIRE(K % 64 == 0, "%s: K=%lld is not a multiple of 64", what, (long long)K);
  GWA_REQUIRE(N % 16 == 0, "%s: N=%lld is not a multiple of 16", what, (long long)N);
  GWA_REQUIRE(out_dtype == GWA_DT_BF16 || out_dtype == GWA_DT_F16, "%s: out_dtype %d", what, out_dtype);
  GWA_REQUIRE((la == nullptr) == (up == nullptr), "%s: la and up must both be given or both NULL", what);
  const int64_t R = la ? rank : 0;
  GWA_REQUIRE(R == 0 || R == 16 || R == 32 || R == 64 || R == 128, "%s: rank %lld not in {0,16,32,64,128}", what,
              (long long)R);
  GWA_REQUIRE(second == nullptr || second_numel == 1 || second_numel == N, "%s: second has %lld values for N=%lld",
              what, (long long)second_numel, (long long)N);
  GWA_REQUIRE((epilogue_flags & ~(GWA_EPI_GELU_TANH | GWA_EPI_LA_F32)) == 0, "%s: unknown epilogue flags 0x%x",
              what, epilogue_flags);
  const int la_f32 = (epilogue_flags & GWA_EPI_LA_F32) ? 1 : 0;
  // K % 128 == 64: the records' last stage is a half stage whose second group holds zero codes (P = 0), so
  // the kernels run over the padded K
  const int64_t nst = (K + 127) / 128, Kp = nst * 128;
  // the DMA offsets of a tile's last run stay below 2^31 + 2^16
  GWA_REQUIRE(nst * (M + 288) * REC < (1ll << 31) && nst * (N + 256) * REC < (1ll << 31) && M * N * 2 < (1ll << 31) &&
                  M * R * 4 < (1ll << 31) && (N / 128) * M * REC < (1ll << 31),
              "%s: operands must stay below 2 GiB (buffer addressing)", what);
  if (M == 0) return GWA_OK;
  const bool nq = nx.q6 != nullptr;
  GWA_REQUIRE(qa6 && qw6 && (out || nq), "%s: null pointer", what);
  // the copies move records in 1 KB runs with unchecked scalar offsets: the run holding a tile's last real
  // row may read up to GWA_FP6_RECORD_SLACK bytes past the last record
  GWA_REQUIRE(qa6_bytes >= nst * M * REC + GWA_FP6_RECORD_SLACK,
              "%s: qa6 has %lld readable bytes, [%lld, %lld, %d] records need %lld plus %d of slack", what,
              (long long)qa6_bytes, (long long)nst, (long long)M, REC, (long long)(nst * M * REC),
              GWA_FP6_RECORD_SLACK);
  GWA_REQUIRE(qw6_bytes >= nst * N * REC + GWA_FP6_RECORD_SLACK,
              "%s: qw6 has %lld readable bytes, [%lld, %lld, %d] records need %lld plus %d of slack", what,
              (long long)qw6_bytes, (long long)nst, (long long)N, REC, (long long)(nst * N * REC),
              GWA_FP6_RECORD_SLACK);
  GWA_REQUIRE(GWA_ALIGNED(qa6, 16) && GWA_ALIGNED(qw6, 16) && GWA_ALIGNED(la, 16) && GWA_ALIGNED(up, 16) &&
                  GWA_ALIGNED(out, 8) && GWA_ALIGNED(bias, 2) && GWA_ALIGNED(second, 4) && GWA_ALIGNED(s2, 4),
              "%s: misaligned pointer", what);
  const int tile = fp6_tile(M, N, nq);
  const int TMv = fp6_tile_m(tile), TNv = fp6_tile_n(tile);
  const int64_t tiles = ((M + TMv - 1) / TMv) * ((N + TNv - 1) / TNv);
  GWA_REQUIRE(tiles < (1ll << 30), "%s: too many tiles", what);
  const int64_t per_xcd = (tiles + kXcds - 1) / kXcds;
  const dim3 grid((unsigned)(per_xcd * kXcds));
  const GwaFp6Args a{qa6, qw6, s2, second, (int)(second_numel > 1), la, la_f32, (const uint16_t*)up,
                  (const uint16_t*)bias, (uint16_t*)out, (int)M, (int)N, (int)Kp};
  const bool gelu = epilogue_flags & GWA_EPI_GELU_TANH;
  const bool f16 = out_dtype == GWA_DT_F16;
  hipStream_t s = (hipStream_t)stream;
  if (fp6_tile_pipelined(tile)) {
    if (gwa_fp6_pipe_launch(TMv, (int)(R / 16), gelu, f16, grid, s, a) != 0)
      return gwa_set_error(GWA_ERR_INVALID, "%s: rank %lld", what, (long long)R);
    return gwa_check_launch(what);
  }
  switch (R / 16) {
    case 0: launch_fp6_flags<0>(tile, gelu, f16, nq, grid, s, a, nx); break;
    case 1: launch_fp6_flags<1>(tile, gelu, f16, nq, grid, s, a, nx); break;
    case 2: launch_fp6_flags<2>(tile, gelu, f16, nq, grid, s, a, nx); break;
    case 4: launch_fp6_flags<4>(tile, gelu, f16, nq, grid, s, a, nx); break;
    case 8: launch_fp6_flags<8>(tile, gelu, f16, nq, grid, s, a, nx); break;
    default: return gwa_set_error(GWA_ERR_INVALID, "%s: rank %lld", what, (long long)R);
  }
  return gwa_check_launch(what);
}

}  // namespace

extern "C" int gwa_svdq_gemm_w4a4_fp6(const uint8_t* qa6, int64_t qa6_bytes, const uint8_t* qw6,
                                      int64_t qw6_bytes, const float* s2, const float* second, int64_t second_numel,
                                      const void* la, const void* up, int64_t rank, const void* bias, void* out,
                                      int out_dtype, int epilogue_flags, int64_t M, int64_t N, int64_t K,
                                      void* stream) {
  const NextLayer none{nullptr, nullptr, 0, nullptr, nullptr};
  return gemm_fp6("svdq_gemm_w4a4_fp6", qa6, qa6_bytes, qw6, qw6_bytes, s2, second, second_numel, la, up, rank, bias,
                  out, out_dtype, epilogue_flags, M, N, K, none, stream);
}

extern "C" int gwa_svdq_gemm_w4a4_fp6_next(const uint8_t* qa6, int64_t qa6_bytes, const uint8_t* qw6,
                                           int64_t qw6_bytes, const float* s2, const float* second,
                                           int64_t second_numel, const void* la, const void* up,
                                           int64_t rank, const void* bias, void* out, int epilogue_flags,
                                           const void* next_smooth, const void* next_proj_down_op, int64_t next_rank,
                                           uint8_t* next_q6, float* next_la_part, int64_t M, int64_t N, int64_t K,
                                           void* stream) {
  const char* what = "svdq_gemm_w4a4_fp6_next";
  GWA_REQUIRE(N > 0 && N % 128 == 0, "%s: N=%lld is not a multiple of 128 (the next layer's fp6 stages)", what,
              (long long)N);
  GWA_REQUIRE(next_q6 != nullptr, "%s: next_q6 is NULL", what);
  GWA_REQUIRE((next_proj_down_op == nullptr) == (next_la_part == nullptr),
              "%s: next_proj_down_op and next_la_part must both be given or both NULL", what);
  const int64_t NR = next_proj_down_op ? next_rank : 0;
  GWA_REQUIRE(NR == 0 || NR == 16 || NR == 32 || NR == 64 || NR == 128, "%s: next rank %lld not in {0,16,32,64,128}",
              what, (long long)NR);
  GWA_REQUIRE(M * NR * 4 < (1ll << 40), "%s: shape too large", what);
  GWA_REQUIRE(GWA_ALIGNED(next_smooth, 16) && GWA_ALIGNED(next_proj_down_op, 16) && GWA_ALIGNED(next_q6, 8) &&
                  GWA_ALIGNED(next_la_part, 4),
              "%s: next_smooth and next_proj_down_op must be 16-byte, next_q6 8-byte aligned", what);
  const NextLayer nx{(const uint16_t*)next_smooth, (const uint16_t*)next_proj_down_op, (int)(NR / 16), next_q6,
                     next_la_part};
  return gemm_fp6(what, qa6, qa6_bytes, qw6, qw6_bytes, s2, second, second_numel, la, up, rank, bias, out,
                  GWA_DT_BF16, epilogue_flags, M, N, K, nx, stream);
}

extern "C" int gwa_svdq_gemm_w4a4_fp6_tile(int64_t M, int64_t N) {
  if (M <= 0 || N <= 0) return -1;
  return fp6_tile(M, N, false);
}

extern "C" int gwa_svdq_gemm_w4a4_fp6_force_tile(int tile) {
  return g_force_tile.exchange(tile >= 0 && tile < kTileCount ? tile : -1);
}

extern "C" int64_t gwa_svdq_gemm_w4a4_fp6_next_partials(int64_t M, int64_t N) {
  if (M <= 0 || N <= 0) return 0;
  const int tn = fp6_tile_n(fp6_tile(M, N, true));
  return (N + tn - 1) / tn;
}
