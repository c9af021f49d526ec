// W4A4 GEMM on fp6 operand records with a software-pipelined MFMA/VALU chain and tiles that fill every CU
// for token counts that are multiples of 256 or 288.
//
// Arithmetic: the fp6 kernel's (w4a4_gemm_fp6.hip): per 32 x 32 block and 64-element group, one exact fp6 MFMA
// gives the integer dot product P, one f16 MFMA the scale outer product S = sw (x) sx, and 16 fmas per lane
// accumulate acc += P * S (the same operations in the same order per element, so the results are the same).
//
// Chain: an MFMA pair costs ~72 matrix-pipe cycles (32 + 32 and a switch between the two instruction types),
// and one wave issues a VALU op at most every ~4.25 cycles, so the 16 fmas of a block take a wave ~68 cycles.
// With 256-row tiles each step issues block b's P, the first 8 fmas of block b-1, block b's S, then block b-1's
// other 8 fmas: a wave never waits on its own MFMAs (register-only measurement: 86 cycles per block-group and
// SIMD against 103 for the serial P -> S -> fma chain). The 288-row tile has no registers for a second block's
// products in flight and runs the serial chain, the other wave of the SIMD covering the matrix pipe. Inside the
// full kernel (operand copies, LDS reads, the stage barrier) both chains cost about the same per block as the
// 256 x 256 tile of the fp6 kernel (1.07x and 1.17x per MAC); these tiles pay where they fill all CUs.
//
// Tiling: a 512-thread workgroup owns TM (m) x 192 (n) outputs; its 8 waves form a 4 (m) x 2 (n) grid of
// 64 x 96 wave tiles (2 x 3 blocks, registers for the pipeline). TM = 288 adds a ninth block row whose 6
// blocks go to the waves with wm < 3 (each takes the block in its own column wm of its three); the waves with
// wm == 3 compute a repeat of one of them and do not store it, so every wave runs the same 7-block code and
// every SIMD carries 14 blocks. A 4608-token layer then has 16 x (N / 192) tiles (N = 3072: exactly one
// per CU). Operand delivery is the fp6 kernel's: stage-major records copied by direct-to-LDS 1 KB runs, three
// stage buffers, one barrier per stage; operands and scales are read into registers right after their last
// use and consumed one group later.
#include "fp6_gemm_common.h"

namespace {

template <int TM>
struct PipeCfg {
  static constexpr int TN = 192;
  static constexpr bool EXTRA = TM == 288;       // the ninth block row
  static constexpr int NBLK = EXTRA ? 7 : 6;     // blocks per wave
  static constexpr int NA = EXTRA ? 3 : 2;       // activation operands (block rows) per wave
  static constexpr int NB = 3;                   // weight operands (block columns) per wave
  static constexpr bool PIPE = !EXTRA;           // software-pipelined chain (registers permitting)
  // LDS: the three stage buffers' activation regions X_0 X_1 X_2, then their weight regions W_0 W_1 W_2, so a
  // lane's operand address in any buffer is one base register plus an immediate offset (< 64 KB)
  static constexpr int LDS_X = (TM * REC + 1023) / 1024 * 1024;
  static constexpr int LDS_W = (TN * REC + 1023) / 1024 * 1024;
  static constexpr int NBUF = 3;
  static constexpr int OFF_W = NBUF * LDS_X, LDS_TOTAL = NBUF * (LDS_X + LDS_W);
  static constexpr int RUNS = (LDS_X + LDS_W) / 1024, DMA_X = LDS_X / 1024;
  static constexpr int SLOTS = (RUNS + NWAVES - 1) / NWAVES;  // DMA runs per wave and stage
  static_assert(TM == 256 || TM == 288, "tile rows");
  static_assert(LDS_TOTAL + 2 * TN * 4 <= kLdsBytes, "LDS");
  static_assert((NBUF - 1) * LDS_X + OFF_SC + 24 < 65536 && (NBUF - 1) * LDS_W + OFF_SC + 24 < 65536,
                "ds_read immediate offsets");
  static_assert(NBUF * SLOTS < 64, "vmcnt range");
};

// Pipeline order of a wave's blocks within a group: (activation operand, weight operand). With the ninth
// block row the extra block (operand a = 2, its row block 8) comes first and uses weight operand 0: each wave
// takes its three columns rotated by wm (operand b is column (wm + b) % 3 of its three), so the extra block of
// the wave at wm < 3 is column wm.
template <bool EXTRA>
struct PipeOrder {
  static constexpr int N = EXTRA ? 7 : 6;
  static constexpr int A[7] = {EXTRA ? 2 : 0, EXTRA ? 0 : 1, EXTRA ? 1 : 0, EXTRA ? 0 : 1, EXTRA ? 1 : 0,
                               EXTRA ? 0 : 1, 1};
  static constexpr int B[7] = {0, EXTRA ? 0 : 0, EXTRA ? 0 : 1, EXTRA ? 1 : 1, EXTRA ? 1 : 2, EXTRA ? 2 : 2, 2};
  // the position of an operand's last use in the group (its register is refilled right after it)
  static constexpr int last_a(int a) {
    int l = -1;
    for (int p = 0; p < N; ++p)
      if (A[p] == a) l = p;
    return l;
  }
  static constexpr int last_b(int b) {
    int l = -1;
    for (int p = 0; p < N; ++p)
      if (B[p] == b) l = p;
    return l;
  }
  static constexpr int first_refill() {
    int f = N;
    for (int a = 0; a < (EXTRA ? 3 : 2); ++a) f = last_a(a) < f ? last_a(a) : f;
    for (int b = 0; b < 3; ++b) f = last_b(b) < f ? last_b(b) : f;
    return f;
  }
};

template <int TM, int RB, bool GELU, bool OUT_F16>
__global__ __launch_bounds__(NTHREADS, 1) void w4a4_gemm_fp6_pipe_kernel(
    const uint8_t* __restrict__ qa, const uint8_t* __restrict__ qw, const float* __restrict__ s2p,
    const float* __restrict__ second, int second_per_channel, const void* __restrict__ la, int la_f32,
    const uint16_t* __restrict__ up, const uint16_t* __restrict__ bias, uint16_t* __restrict__ out, int M, int N,
    int K) {
  using C = PipeCfg<TM>;
  using O = PipeOrder<C::EXTRA>;
  constexpr int TN = C::TN, NBUF = C::NBUF, SLOTS = C::SLOTS, NBLK = C::NBLK, NA = C::NA, NB = C::NB;
  constexpr int LDS_X = C::LDS_X, LDS_W = C::LDS_W, OFF_W = C::OFF_W;
  __shared__ __attribute__((aligned(16))) uint8_t g_lds[C::LDS_TOTAL];
  __shared__ __attribute__((aligned(16))) float g_epi[2 * TN];

  const int tid = threadIdx.x;
  const int tiles_n = (N + TN - 1) / TN, tiles_m = (M + TM - 1) / TM;
  int tm, tn;
  if (!xcd_tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn)) return;  // whole workgroup, before any barrier
  const int n0 = tn * TN, m0 = tm * TM;
  const int nst = K >> 7;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int wm = wave & 3, wn = wave >> 2;
  const int r32 = lane & 31, h = lane >> 5;
  const int rot = wm % 3;  // the wave's column rotation: operand b is column (rot + b) % 3 of its three

  const v4i xbuf = raw_rsrc(qa, (uint32_t)((int64_t)nst * M * REC));
  const v4i wbuf = raw_rsrc(qw, (uint32_t)((int64_t)nst * N * REC));

  // DMA (the fp6 kernel's scheme): run q of a stage is LDS bytes [1024 q, +1024) of the stage buffer = bytes
  // [1024 q', +1024) of the tile's contiguous records; runs dealt round-robin, a wave without a last run
  // repeats the final one, so every wave issues SLOTS copies per stage. A run that starts past the tile's last
  // real row re-reads the stage's first run; the run that straddles it (and the padding run of a region whose
  // rows do not fill whole KB) reads up to 1 KB past it: the record buffers' slack.
  const uint32_t dvo = 16u * (uint32_t)lane;
  const uint32_t x_valid = (uint32_t)(M - m0) * REC, w_valid = (uint32_t)(N - n0) * REC;
  [[maybe_unused]] const uint32_t x_bytes = (uint32_t)((int64_t)nst * M * REC);
  [[maybe_unused]] const uint32_t w_bytes = (uint32_t)((int64_t)nst * N * REC);
  auto issue = [&](int u, int st) __attribute__((always_inline)) {
    const uint32_t xs_ = (uint32_t)(((int64_t)st * M + m0) * REC);
    const uint32_t ws_ = (uint32_t)(((int64_t)st * N + n0) * REC);
#pragma unroll
    for (int j = 0; j < SLOTS; ++j) {
      int q = wave + NWAVES * j;
      q = q < C::RUNS ? q : C::RUNS - 1;
      const bool isx = q < C::DMA_X;
      const uint32_t r0 = (uint32_t)((isx ? q : q - C::DMA_X) * 1024);
      uint32_t soff = (isx ? xs_ : ws_) + (r0 < (isx ? x_valid : w_valid) ? r0 : 0u);
      // the run [soff, soff + 1 KB) stays within the records plus their 1 KB slack
      if (!GWA_DCHECK(soff <= (isx ? x_bytes : w_bytes), isx ? kDbgFp6CopyA : kDbgFp6CopyW, soff))
        soff = isx ? xs_ : ws_;
      uint8_t* dst = isx ? g_lds + u * LDS_X + q * 1024 : g_lds + OFF_W + u * LDS_W + (q - C::DMA_X) * 1024;
      dma16(isx ? xbuf : wbuf, (uint32_t)(uintptr_t)dst, dvo, soff);
    }
  };

  // low-rank operands of ranks up to 32 with bf16 la (la rows m0.., up rows n0..: two contiguous runs) copied
  // into the activation and weight regions of the stage buffer no stage reads or fills once stage
  // max(nst - 2, 0)'s sync has passed
  const bool lr_lds = (RB == 1 || RB == 2) && !la_f32;
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

  float acc[NBLK][16];
#pragma unroll
  for (int b = 0; b < NBLK; ++b)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[b][v] = 0.0f;
  auto pin16 = [](float* a) __attribute__((always_inline)) {
    asm volatile("" : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(a[4]), "+v"(a[5]), "+v"(a[6]), "+v"(a[7]),
                 "+v"(a[8]), "+v"(a[9]), "+v"(a[10]), "+v"(a[11]), "+v"(a[12]), "+v"(a[13]), "+v"(a[14]), "+v"(a[15]));
  };
  // P and S of the block whose fmas come next (the pipelined chain starts with zero products pending for the
  // last block)
  v16f pp = (v16f){}, ps = (v16f){};
  auto fma_half = [&](int blk, int half) __attribute__((always_inline)) {
#pragma unroll
    for (int b = 0; b < NBLK; ++b)
      if (blk == b) {
#pragma unroll
        for (int v = 8 * half; v < 8 * half + 8; ++v) acc[b][v] = fmaf(pp[v], ps[v], acc[b][v]);
      }
  };
  auto pin_acc = [&](int blk) __attribute__((always_inline)) {
#pragma unroll
    for (int b = 0; b < NBLK; ++b)
      if (blk == b) pin16(acc[b]);
  };

  // operand registers: activation operands (block rows) and their stage scales, weight operands (block columns)
  // and theirs
  v8i xo[NA], wo[NB];
  // The S MFMA's operands. B (activation side, every lane): the row record's eight bytes 96..103 as read,
  // {sx_g0, sx_g1, 0, 0} as f16 K slots (lanes 32..63 read their row's record too: finite scales in slots 4..7).
  // A (weight side): the stage's two weight group scales as read (lanes 32..63 read the record's four zero
  // bytes instead), masked to group g's slot once per run of blocks that share the weight operand (the other
  // group's slot and K slots 2..3 zero; lanes 32..63 zero), so S = sw_g * sx_g exactly.
  uint2 xs8[NA];
  uint32_t wsc[NB];
#pragma unroll
  for (int a = 0; a < NA; ++a) xs8[a] = make_uint2(0u, 0u);
#pragma unroll
  for (int b = 0; b < NB; ++b) wsc[b] = 0u;
  auto row_of = [&](int a) __attribute__((always_inline)) { return a < 2 ? 64 * wm + 32 * a : 256; };
  auto col_of = [&](int b) __attribute__((always_inline)) {
    const int c = rot + b;
    return 96 * wn + 32 * (c < 3 ? c : c - 3);
  };
  // this lane's operand rows (+ its 24-byte half of a group) in buffer 0; buffer u adds u * LDS_X / u * LDS_W
  int xaddr[NA], waddr[NB];
#pragma unroll
  for (int a = 0; a < NA; ++a) xaddr[a] = (row_of(a) + r32) * REC + 24 * h;
#pragma unroll
  for (int b = 0; b < NB; ++b) waddr[b] = OFF_W + (col_of(b) + r32) * REC + 24 * h;
  const uint32_t hmask = h ? 0u : 0xFFFFFFFFu;
  const uint32_t gmask0 = hmask & 0x0000FFFFu, gmask1 = hmask & 0xFFFF0000u;
  auto read_x = [&](int u, int a, int gi) __attribute__((always_inline)) {
    xo[a] = lds_operand(g_lds + xaddr[a] + u * LDS_X + gi * GB);
  };
  auto read_w = [&](int u, int b, int gi) __attribute__((always_inline)) {
    wo[b] = lds_operand(g_lds + waddr[b] + u * LDS_W + gi * GB);
  };
  auto read_xs = [&](int u, int a) __attribute__((always_inline)) {
    xs8[a] = *(const uint2*)(g_lds + xaddr[a] - 24 * h + u * LDS_X + OFF_SC);  // the row's bytes 96..103
  };
  const int wsoff = OFF_SC - 20 * h;  // lanes 32..63: record bytes [100, 104), zero by the record format
  auto read_ws = [&](int u, int b) __attribute__((always_inline)) {
    wsc[b] = *(const uint32_t*)(g_lds + waddr[b] + wsoff + u * LDS_W);
  };

  uint8_t* const spare_x = g_lds + (nst % NBUF) * LDS_X;
  uint8_t* const spare_w = g_lds + OFF_W + (nst % NBUF) * LDS_W;
  // stage st's sync: stage st + 1 complete (this wave's copies, then everyone's; the barrier also retires every
  // wave's reads of this stage's buffer), then this stage's buffer takes stage st + NBUF
  auto sync = [&](int st, int u) __attribute__((always_inline)) {
    if (st + 1 < nst) {
      wait_stages<SLOTS, NBUF - 2>(min(NBUF - 2, nst - 2 - st));
      barrier_lds();
    }
    if (st + NBUF < nst) issue(u, st + NBUF);
    if (lr_lds && st == max(nst - 2, 0)) issue_lowrank(spare_x, spare_w);
  };

  // One step. Pipelined (256-row tiles): block p's P, block p-1's first 8 fmas, block p's S, block p-1's other 8
  // fmas. Serial (288-row tiles, whose seventh block leaves no registers for a second block's P and S in
  // flight): block p's P and S, then its 16 fmas; the other wave of the SIMD fills the matrix pipe meanwhile.
  // The step's MFMA inputs pass through an empty asm, so the (pure) MFMAs cannot be hoisted out of their step;
  // full scheduling fences keep the step's parts in this order (the compiler would otherwise regroup the fmas
  // and MFMAs of neighbouring steps).
  uint2 swp = make_uint2(0u, 0u);  // the S MFMA's A operand for the current run of blocks
  auto step = [&](int p, int gi) __attribute__((always_inline)) {
    const int a = O::A[p], b = O::B[p];
    asm volatile("" : "+v"(xs8[a]), "+v"(xo[a]), "+v"(wo[b]), "+v"(wsc[b]));
    if (p == 0 || O::B[p - 1] != b) swp = make_uint2(wsc[b] & (gi ? gmask1 : gmask0), 0u);
    const v4h swop = __builtin_bit_cast(v4h, swp);
    const v4h sel = __builtin_bit_cast(v4h, xs8[a]);
    if constexpr (C::PIPE) {
      const int prev = p == 0 ? NBLK - 1 : p - 1;
      __builtin_amdgcn_sched_barrier(0);
      v16f p_ = group_mfma_fp6(wo[b], xo[a]);
      __builtin_amdgcn_sched_barrier(0);
      fma_half(prev, 0);
      __builtin_amdgcn_sched_barrier(0);
      v16f s_ = __builtin_amdgcn_mfma_f32_32x32x8f16(swop, sel, (v16f){}, 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
      fma_half(prev, 1);
      __builtin_amdgcn_sched_barrier(0);
      pin_acc(prev);
      pp = p_;
      ps = s_;
    } else {
      __builtin_amdgcn_sched_barrier(0);
      pp = group_mfma_fp6(wo[b], xo[a]);
      ps = __builtin_amdgcn_mfma_f32_32x32x8f16(swop, sel, (v16f){}, 0, 0, 0);
      fma_half(p, 0);
      fma_half(p, 1);
      __builtin_amdgcn_sched_barrier(0);
      pin_acc(p);
    }
  };

  // One stage: each operand register is refilled right after its last use in the group, group 0 from this
  // stage's buffer (group 1's codes), group 1 from the next buffer (the next stage's group 0 codes and the
  // stage's scales) after the stage's sync, which comes right before the first such read.
  auto stage = [&](int st, int cur, int nxt) __attribute__((always_inline)) {
    // fully unrolled (plain unroll pragmas leave the block loop rolled once the masks form in the steps)
#pragma clang loop unroll(full)
    for (int gi = 0; gi < GS; ++gi) {
#pragma clang loop unroll(full)
      for (int p = 0; p < NBLK; ++p) {
        step(p, gi);
        if (gi == 1 && p == O::first_refill()) sync(st, cur);
        const int src = gi ? nxt : cur;  // past the last stage the reads fetch unused LDS bytes
#pragma unroll
        for (int a = 0; a < NA; ++a)
          if (p == O::last_a(a)) {
            read_x(src, a, gi ^ 1);
            if (gi) read_xs(nxt, a);
          }
#pragma unroll
        for (int b = 0; b < NB; ++b)
          if (p == O::last_b(b)) {
            read_w(src, b, gi ^ 1);
            if (gi) read_ws(nxt, b);
          }
      }
    }
  };

  // the epilogue constants' loads go out first; they are older than every copy, so the stage waits below cover
  // them too
  const EpiConsts epc = epi_consts_load(s2p, second, second_per_channel, bias, n0, tid, TN, N);
#pragma unroll
  for (int u = 0; u < NBUF; ++u)
    if (u < nst) issue(u, u);
  wait_stages<SLOTS, NBUF - 1>(min(NBUF - 1, nst - 1));
  barrier_lds();
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    read_w(0, b, 0);
    read_ws(0, b);
  }
#pragma unroll
  for (int a = 0; a < NA; ++a) {
    read_x(0, a, 0);
    read_xs(0, a);
  }
  for (int st = 0; st < nst; st += NBUF) {  // unrolled by NBUF so every LDS address is static
#pragma unroll
    for (int u = 0; u < NBUF; ++u)
      if (st + u < nst) stage(st + u, u, (u + 1) % NBUF);
  }
  if constexpr (C::PIPE) {
    fma_half(NBLK - 1, 0);
    fma_half(NBLK - 1, 1);
  }
  epi_consts_store(epc, s2p, second, bias, g_epi, tid, TN);
  wait_vm_lgkm0<0>();  // the low-rank copies (and the reads past the last stage) complete
  barrier_lds();

  // ---------------- epilogue ----------------
  v16f accv[NBLK];
#pragma unroll
  for (int p = 0; p < NBLK; ++p) {
    const int nl = col_of(O::B[p]);
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) {
      const v4f cm = *(const v4f*)(g_epi + nl + 8 * qd + 4 * h);
#pragma unroll
      for (int e = 0; e < 4; ++e) accv[p][4 * qd + e] = acc[p][4 * qd + e] * cm[e];
    }
  }
  if constexpr (RB > 0) {
    const uint8_t* lrb = spare_x;
    const uint8_t* upb = spare_w;
    const rsrc_t ubuf = make_rsrc(up, (uint32_t)((int64_t)N * RB * 32));
    const rsrc_t lbuf = make_rsrc(la, (uint32_t)((int64_t)M * la_row));
#pragma unroll
    for (int k0 = 0; k0 < RB; ++k0) {
      v4i ua[NB], lb[NA];
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const int n = col_of(b) + r32;
        if (lr_lds) {
          ua[b] = *(const v4i*)(upb + n * (RB * 32) + k0 * 32 + 16 * h);
        } else {
          ua[b] = buf_load16(ubuf, (uint32_t)((int64_t)(n0 + n) * (RB * 32) + k0 * 32 + 16 * h));
        }
      }
#pragma unroll
      for (int a = 0; a < NA; ++a) {
        const int m = row_of(a) + r32, k = k0 * 16 + 8 * h;
        if (lr_lds) {
          lb[a] = la_operand_lds(lrb, m, la_row, k, false);
        } else {
          const uint32_t row_off = (uint32_t)((int64_t)(m0 + m) * la_row);
          if (la_f32) {
            const v4f fa = __builtin_bit_cast(v4f, buf_load16(lbuf, row_off + k * 4));
            const v4f fb = __builtin_bit_cast(v4f, buf_load16(lbuf, row_off + k * 4 + 16));
            lb[a] = (v4i){(int)pack_bf16x2_rn(fa[0], fa[1]), (int)pack_bf16x2_rn(fa[2], fa[3]),
                          (int)pack_bf16x2_rn(fb[0], fb[1]), (int)pack_bf16x2_rn(fb[2], fb[3])};
          } else {
            lb[a] = buf_load16(lbuf, row_off + k * 2);
          }
        }
      }
#pragma unroll
      for (int p = 0; p < NBLK; ++p)
        accv[p] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, ua[O::B[p]]),
                                                         __builtin_bit_cast(v8bf, lb[O::A[p]]), accv[p], 0, 0, 0);
    }
  }
  // + bias (+ GELU), packed to 16 bits, staged in LDS as [m][n] rows of OSTR bytes (the stage buffers are free;
  // the barrier also retires the la / up reads), then stored as full rows. The repeated extra block of the
  // waves with wm == 3 is not staged.
  constexpr int OSTR = TN * 2 + 8;  // 8-byte pad: distinct banks per write
  static_assert(TM * OSTR <= C::LDS_TOTAL, "output staging");
  uint8_t* ob = g_lds;
  barrier_lds();
#pragma unroll
  for (int p = 0; p < NBLK; ++p) {
    if (C::EXTRA && p == 0 && wm == 3) continue;
    const int nl = col_of(O::B[p]);
    const int ml = row_of(O::A[p]) + r32;
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) {
      const int nn = nl + 8 * qd + 4 * h;
      const v4f cb = *(const v4f*)(g_epi + TN + nn);
      float o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float t = accv[p][4 * qd + e] + cb[e];
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
  barrier_lds();
  // rows of 24 16-byte chunks; consecutive threads take consecutive chunks of the tile (row-major)
  constexpr int CPR = TN / 8, CHUNKS = TM * CPR;
  const rsrc_t obuf = make_rsrc(out, (uint32_t)((int64_t)M * N * 2));
#pragma unroll 2
  for (int i = tid; i < CHUNKS; i += NTHREADS) {
    const int row = i / CPR, cch = i - row * CPR;
    const uint2 lo = *(const uint2*)(ob + row * OSTR + cch * 16);
    const uint2 hi = *(const uint2*)(ob + row * OSTR + cch * 16 + 8);
    uint32_t off = (n0 + 8 * cch < N && m0 + row < M) ? (uint32_t)(((int64_t)(m0 + row) * N + n0 + 8 * cch) * 2)
                                                      : kOOB;
    if (!GWA_DCHECK(off == kOOB || (int64_t)off + 16 <= (int64_t)M * N * 2, kDbgFp6Out, off)) off = kOOB;
    buf_store16((v4i){(int)lo.x, (int)lo.y, (int)hi.x, (int)hi.y}, obuf, off);
  }
}

template <int TM, int RB, bool GL, bool F16>
void launch_pipe(dim3 grid, hipStream_t s, const GwaFp6Args& a) {
  hipLaunchKernelGGL((w4a4_gemm_fp6_pipe_kernel<TM, RB, GL, F16>), grid, dim3(NTHREADS), 0, s, a.qa6, a.qw6, a.s2,
                     a.second, a.per_channel, a.la, a.la_f32, a.up, a.bias, a.out, a.M, a.N, a.K);
}

template <int TM, int RB>
void launch_pipe_flags(bool gelu, bool f16, dim3 grid, hipStream_t s, const GwaFp6Args& a) {
  if (gelu) {
    if (f16) launch_pipe<TM, RB, true, true>(grid, s, a);
    else launch_pipe<TM, RB, true, false>(grid, s, a);
  } else {
    if (f16) launch_pipe<TM, RB, false, true>(grid, s, a);
    else launch_pipe<TM, RB, false, false>(grid, s, a);
  }
}

template <int TM>
int launch_pipe_rank(int rb, bool gelu, bool f16, dim3 grid, hipStream_t s, const GwaFp6Args& a) {
  switch (rb) {
    case 0: launch_pipe_flags<TM, 0>(gelu, f16, grid, s, a); return 0;
    case 1: launch_pipe_flags<TM, 1>(gelu, f16, grid, s, a); return 0;
    case 2: launch_pipe_flags<TM, 2>(gelu, f16, grid, s, a); return 0;
    case 4: launch_pipe_flags<TM, 4>(gelu, f16, grid, s, a); return 0;
    case 8: launch_pipe_flags<TM, 8>(gelu, f16, grid, s, a); return 0;
    default: return -1;
  }
}

}  // namespace

// Launch of the pipelined kernel for a tile of tm (256 or 288) x 192; the caller has checked the arguments.
int gwa_fp6_pipe_launch(int tm, int rb, bool gelu, bool f16, dim3 grid, hipStream_t s, const GwaFp6Args& a) {
  if (tm == 288) return launch_pipe_rank<288>(rb, gelu, f16, grid, s, a);
  if (tm == 256) return launch_pipe_rank<256>(rb, gelu, f16, grid, s, a);
  return -1;
}
