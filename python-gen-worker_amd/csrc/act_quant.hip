// Activation-side kernels: int4 group-64 quantization (+ fused x @ proj_down),
// int8 per-token quantization, and the standalone SVDQuant epilogue.
#include "gwa_common.h"
#include "quant_g64.h"

// ---------------------------------------------------------------------------
// Kernel 1: smoothing divide -> group-64 absmax -> fp16 scale -> int4 codes;
// plus la = x @ proj_down on the RAW activations via bf16 MFMA 16x16x32.
//
// Work split: a 512-thread workgroup owns 16 rows and walks K in rounds of
// 256 columns (4 groups). Each round's 16 x 256 bf16 tile is loaded with
// row-contiguous 16-byte loads (512 bytes of a row per 32 lanes: whole cache
// lines) into double-buffered LDS together with the round's smoothing
// factors, PF rounds ahead of use; then
//  * each wave quantizes 2 rows of the tile, a lane holding 8 consecutive
//    elements, the group absmax a max over the group's 8 lanes (three DPP
//    steps), the scale RN(amax / 7) by one fma-corrected multiply (exact for
//    every finite bf16 amax, checked exhaustively with rational arithmetic);
//  * each wave adds one 32-column slice of x @ proj_down with MFMA, the A
//    operand read from the tile in MFMA order and the B operand loaded from
//    proj_down pre-arranged in MFMA operand order (1 KB contiguous per load;
//    gwa_svdq_prep_proj_down), so no transpose touches global memory.
// The eight waves' la partials are summed through LDS at the end.
//
// Output: the reference contract (two's-complement nibbles, element 2j in the
// low nibble of byte j; fp16 scales [M, K/64]; la bf16). The fp6 GEMM lane's
// records come from svdq_quant_fp6_kernel below.
//
// Arithmetic = the reference order (models/svdq_fused.py:88-103,
// models/nvfp4_quant.py:96-102), computed by the per-lane quantizer of
// quant_g64.h (bit-identical fast paths for smoothing, scale and codes).
// ---------------------------------------------------------------------------
namespace {

constexpr int KT = 256;                 // columns per round
constexpr int XT_STR = KT * 2 + 16;     // LDS row stride of the x tile (bytes)
constexpr int XT_BYTES = 16 * XT_STR;   // 8448
constexpr int QBUF = XT_BYTES + KT * 4 * 2 + 16;  // tile + reciprocals + factors + flag word

__device__ __forceinline__ void unpack8_bf16(v4i w, float* v) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t u = (uint32_t)w[j];
    v[2 * j] = bf16_lo(u);
    v[2 * j + 1] = bf16_hi(u);
  }
}

template <int RB, int PF>
__global__ __launch_bounds__(512) void svdq_quant_int4_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const uint16_t* __restrict__ smooth,
    const float* __restrict__ s2p, const uint16_t* __restrict__ pdo, uint8_t* __restrict__ q,
    uint16_t* __restrict__ sc, uint16_t* __restrict__ la, int M, int K) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr int RBX = RB > 0 ? RB : 1;
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int row0 = blockIdx.x * 16;
  const int G = K >> 6;
  const int rounds = (K + KT - 1) / KT;

  // buffers: every access is unconditional; rows >= M, columns >= K read 0 / store nothing
  const rsrc_t xbuf = make_rsrc(x, (uint32_t)(((int64_t)(M - 1) * ldx + K) * 2));
  const int64_t qrow_bytes = (int64_t)K / 2;
  const rsrc_t qbuf = make_rsrc(q, (uint32_t)((int64_t)M * qrow_bytes));
  const rsrc_t sbuf = make_rsrc(sc, (uint32_t)((int64_t)M * G * 2));
  const rsrc_t pbuf = make_rsrc(pdo, (uint32_t)((int64_t)rounds * KT * RB * 32));
  const rsrc_t smbuf = make_rsrc(smooth, smooth ? (uint32_t)(K * 2) : 0u);

  // tile loader: thread t -> row t >> 5, 16 bytes at column 8 (t & 31)
  const int xcol = (tid & 31) * 8;
  const uint32_t xoff = (uint32_t)(((int64_t)(row0 + (tid >> 5)) * ldx + xcol) * 2);
  const bool sm_role = smooth && tid < KT / 2;

  struct Slot {
    v4i xv;
    uint32_t sv;
    v4i lo[RBX];
  };
  auto load_tile = [&](Slot& s, int r) {
    const int kb = r * KT;
    s.xv = buf_load16(xbuf, kb + xcol < K ? xoff + (uint32_t)(kb * 2) : kOOB);
    const int k = kb + 2 * tid;
    s.sv = sm_role ? buf_load4(smbuf, k < K ? (uint32_t)(k * 2) : kOOB) : 0u;
  };
  auto load_lowrank = [&](Slot& s, int r) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
      s.lo[rb] = buf_load16(pbuf, (uint32_t)((((int64_t)(r * (KT / 32) + wave) * RB + rb) * 64 + lane) * 16));
  };
  // round r's tile + factors into LDS buffer b; a factor the multiply path
  // cannot use marks the buffer's flag word with r
  auto store_tile = [&](const Slot& s, int r, int b) {
    uint8_t* base = lds + b * QBUF;
    *(v4i*)(base + (tid >> 5) * XT_STR + (tid & 31) * 16) = s.xv;
    if (sm_role) {
      const float s0 = bf16_lo(s.sv), s1 = bf16_hi(s.sv);
      float* rs = (float*)(base + XT_BYTES);
      float* fs = rs + KT;
      rs[2 * tid] = 1.0f / s0;
      rs[2 * tid + 1] = 1.0f / s1;
      fs[2 * tid] = s0;
      fs[2 * tid + 1] = s1;
      if (r * KT + 2 * tid < K && (!g64::smooth_ok(s0) || !g64::smooth_ok(s1))) *(int*)(fs + KT) = r;
    }
  };

  const float s2 = s2p ? *s2p : 1.0f;
  const bool s2_one = (s2 == 1.0f);

  // quantization roles: wave w rows 2w, 2w+1; lane -> row 2w + (lane >> 5), 8 columns at 8 (lane & 31)
  const int qr = 2 * wave + (lane >> 5), qc = (lane & 31) * 8;
  const int grow = row0 + qr;
  const uint32_t q_row_off = (uint32_t)((int64_t)grow * qrow_bytes);
  const uint32_t s_row_off = (lane & 7) == 0 ? (uint32_t)((int64_t)grow * G * 2) : kOOB;

  if (tid < 2) *(int*)(lds + tid * QBUF + XT_BYTES + KT * 8) = -1;
  Slot slot[PF];
#pragma unroll
  for (int j = 0; j < PF; ++j) {
    load_tile(slot[j], j);
    if (RB > 0) load_lowrank(slot[j], j);
  }
  __syncthreads();

  v4f acc[RBX];
#pragma unroll
  for (int rb = 0; rb < RBX; ++rb) acc[rb] = (v4f){0.f, 0.f, 0.f, 0.f};

  for (int rr = 0; rr < rounds; rr += PF) {
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      const int r = rr + j;
      const int b = r & 1;
      store_tile(slot[j], r, b);
      load_tile(slot[j], r + PF);
      __syncthreads();
      const uint8_t* base = lds + b * QBUF;

      // ---- quantize 8 columns of one row per lane (a group = 8 lanes)
      {
        const int kg = r * KT + qc;       // first column
        const int g = kg >> 6;            // group
        const bool valid = kg < K && grow < M;
        const v4i c0 = *(const v4i*)(base + qr * XT_STR + qc * 2);
        uint32_t w[4];
        if (!smooth) {
#pragma unroll
          for (int t = 0; t < 4; ++t) w[t] = (uint32_t)c0[t];
        } else {
          const bool bad = *(const int*)(base + XT_BYTES + KT * 8) == r;
          float f[8];
          const float* src = (const float*)(base + XT_BYTES) + (bad ? KT : 0) + qc;
          *(v4f*)(f) = *(const v4f*)(src);
          *(v4f*)(f + 4) = *(const v4f*)(src + 4);
          g64::smooth8(c0, f, bad, w);
        }
        uint32_t nb[2];
        uint16_t sh;
        g64::quant8(w, valid, s2_one, s2, nb, sh);
        const uint32_t a = nb[0], bb = nb[1];
        const uint32_t pa = (a & 0xFu) | ((a >> 4) & 0xF0u) | ((a >> 8) & 0xF00u) | ((a >> 12) & 0xF000u);
        const uint32_t pb = (bb & 0xFu) | ((bb >> 4) & 0xF0u) | ((bb >> 8) & 0xF00u) | ((bb >> 12) & 0xF000u);
        buf_store4(pa | (pb << 16), qbuf, valid ? q_row_off + (uint32_t)(kg / 2) : kOOB);
        buf_store2(sh, sbuf, valid ? s_row_off + (uint32_t)(g * 2) : kOOB);
      }

      // ---- la += x[:, slice] @ proj_down[slice, :] for this wave's 32-column slice
      if (RB > 0) {
        const v4i a = *(const v4i*)(base + (lane & 15) * XT_STR + wave * 64 + (lane >> 4) * 16);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
          acc[rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, a),
                                                            __builtin_bit_cast(v8bf, slot[j].lo[rb]), acc[rb], 0, 0, 0);
        load_lowrank(slot[j], r + PF);
      }
    }
  }

  if (RB > 0) {
    // sum the 8 waves' partial la blocks through LDS; wave 0 writes bf16
    __syncthreads();
    float* lap = (float*)lds;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) *(v4f*)(lap + ((wave * RB + rb) * 64 + lane) * 4) = acc[rb];
    __syncthreads();
    if (wave == 0) {
      const int R = RB * 16;
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        v4f s = acc[rb];
#pragma unroll
        for (int w2 = 1; w2 < 8; ++w2) s += *(const v4f*)(lap + ((w2 * RB + rb) * 64 + lane) * 4);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int r = row0 + 4 * (lane >> 4) + t;
          if (r < M) la[(int64_t)r * R + rb * 16 + (lane & 15)] = f32_to_bf16(s[t]);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Kernel 1, fp6 records (the fp6 GEMM lane): smoothing divide -> group-64
// absmax -> fp16 scale -> int4 codes written as e3m2 operand records, plus
// la += x @ proj_down on the RAW activations, in fp32.
//
// Work split: a task is 16 rows x one 128-column stage (one record per row).
// A 256-thread workgroup (4 waves) owns 64 rows x CH consecutive stages; K
// is split over workgroups (grid.y), so la is a sum of per-workgroup
// partials: workgroup (g, y) stores its rows' partial into slot y of
// la_part [P][M][rank] fp32 (plain stores), and gwa_svdq_la_reduce sums the
// slots in a fixed order (deterministic). In a task, lane (r, c) = (lane %
// 16, lane / 16) holds row r, columns 32c .. 32c+31 of the stage: half of
// group c / 2, so a group's absmax is one max over the lane's 32 values and
// one exchange with lane ^ 16.
//  * x goes global -> LDS by direct copies, one task ahead, into a two-task
//    ring per wave: each copy moves four whole 256-byte row segments (16
//    bytes per lane), so every request reads whole cache lines; the
//    quantizer's lane layout (16 bytes of one row per lane and k-step) is
//    then read from LDS, the chunk order of each row XOR-swizzled by the row
//    so those reads are free of bank conflicts. (Loading that layout straight
//    from global memory touches 64 lines per request, a quarter of each: the
//    read ran at 5.5 TB/s against 8.5 for whole lines in a probe of the
//    same shape.)
//  * Each workgroup copies the stages' proj_down operands and smoothing
//    factors to LDS before its first task's x, and waits for those only.
//  * The smoothing reciprocals RN(1/s) of the stages are formed once per
//    workgroup in LDS (a non-normal reciprocal flags the stage for the
//    division path).
//  * Codes: q = RNE(xs / d) by the 2^-12 snap of the multiply path (exact,
//    see quant_g64.h), as floats; the lane's 32 codes are packed to e3m2 by
//    one v_cvt_scalef32_2xpk16_bf6_f32 (unit scale: exact for every integer
//    in [-8, 8]; element 2i from the first source's i, 2i+1 from the
//    second's) straight into the record's bit layout and stored as 24 bytes.
//  * la: the task's x chunks are the A operands of four 16x16x32 bf16 MFMAs
//    per 16 ranks (lane (r, c) supplies columns 32c + 8j .. +8 at k-step j);
//    proj_down is pre-arranged in that order (gwa_svdq_prep_proj_down_fp6)
//    so each B operand is one 16-byte LDS read per lane.
// Arithmetic and exactness = quant_g64.h's: identical codes and scales.
// ---------------------------------------------------------------------------
constexpr int Q6_WAVES = 4, Q6_THREADS = 64 * Q6_WAVES, Q6_ROWS = 16 * Q6_WAVES;

__device__ __forceinline__ void dma16_lds(v4i rsrc, uint32_t lds_addr, uint32_t voff, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(lds_addr), "v"(voff), "s"(rsrc), "s"(soff)
               : "memory", "m0");
}

__device__ __forceinline__ v4i raw_rsrc4(const void* base, uint32_t bytes) {
  const uint64_t a = (uint64_t)base;
  return (v4i){(int)(uint32_t)a, (int)(uint32_t)((a >> 32) & 0xFFFFu), (int)bytes, 0x00020000};
}

template <int n>
__device__ __forceinline__ void wait_vm_lgkm0_q() {
  static_assert(n >= 0 && n < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | (7 << 4));
}

template <int RB, int CH>
__global__ __launch_bounds__(Q6_THREADS) void svdq_quant_fp6_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const uint16_t* __restrict__ smooth, const float* __restrict__ s2p,
    const uint16_t* __restrict__ pdo, uint8_t* __restrict__ q6, float* __restrict__ la_part, int M, int K) {
  constexpr int RBX = RB > 0 ? RB : 1;
  constexpr int PDO_STAGE = RB * 4096;                       // bytes of proj_down operands per stage
  constexpr int RCP_OFF = CH * PDO_STAGE;                    // [CH][128] reciprocals, [CH][128] factors
  constexpr int SMR_OFF = RCP_OFF + CH * 128 * 4 * 2;        // [CH * 128] the factors as copied (bf16)
  constexpr int FLAG_OFF = SMR_OFF + 1024;                   // [CH] division-path flags
  constexpr int X_OFF = (FLAG_OFF + CH * 4 + 1023) / 1024 * 1024;
  constexpr int X_TASK = 4096;                               // a task's x: 16 rows x 256 bytes
  static_assert(CH * 128 * 2 <= 1024, "smoothing factors of a chunk");
  __shared__ __attribute__((aligned(16))) uint8_t lds[X_OFF + Q6_WAVES * 2 * X_TASK];

  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int S = (K + 127) >> 7;  // K % 128 == 64: the last stage's second group lies past K (read as zeros)
  const int st0 = blockIdx.y * CH;
  const int ntask = min(CH, S - st0);  // workgroup-uniform, >= 1
  const int r = lane & 15, c = lane >> 4;
  const int row0 = blockIdx.x * Q6_ROWS + 16 * wave;
  const int grow = row0 + r;
  const bool row_ok = grow < M;

  // x: a task's 16 rows x 256 bytes go global -> LDS by four direct copies per wave (16 bytes per lane, four
  // whole rows per copy: every copy reads whole cache lines), into a two-task ring per wave. Slot s of the
  // task's row q holds the row's 16-byte chunk s ^ q, so the quantizer's reads (row r, chunk 4c + j: sixteen
  // rows at one chunk index per 16 lanes) fall in sixteen distinct bank groups.
  const v4i xr4 = raw_rsrc4(x, (uint32_t)(((int64_t)(M - 1) * ldx + K) * 2));
  uint8_t* const xring = lds + X_OFF + wave * (2 * X_TASK);
  auto issue_x = [&](int t) __attribute__((always_inline)) {
    const int col = (st0 + t) * 128;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int q = 4 * j + (lane >> 4), sl = lane & 15;
      const int cc = col + 8 * (sl ^ q);  // columns past K (a half stage) land as zeros
      const uint32_t off = row0 + q < M && cc < K ? (uint32_t)(((int64_t)(row0 + q) * ldx + cc) * 2) : kOOB;
      dma16_lds(xr4, (uint32_t)(uintptr_t)(xring + (t & 1) * X_TASK + j * 1024), off, 0u);
    }
  };
  // 0. the chunk's smoothing factors (one copy, wave 0), then the stages' proj_down operands, then task 0's x:
  //    everything but task 0's x is waited for before the reciprocals
  if (smooth && wave == 0) {
    const v4i sm4 = raw_rsrc4(smooth, (uint32_t)(K * 2));
    const int col = st0 * 128 + 8 * lane;
    dma16_lds(sm4, (uint32_t)(uintptr_t)(lds + SMR_OFF), lane < CH * 16 && col < K ? (uint32_t)(col * 2) : kOOB,
              0u);
  }
  // 1. the stages' proj_down operands, direct to LDS: CH * RB * 4 runs of 1 KB, dealt round-robin (every
  //    wave issues the same number). The offset goes in the VGPR operand, the one the hardware range-checks:
  //    the runs of stages past K read zeros.
  if constexpr (RB > 0) {
    const v4i pbuf = raw_rsrc4(pdo, (uint32_t)((int64_t)S * PDO_STAGE));
    constexpr int RUNS = CH * RB * 4, PER = RUNS / Q6_WAVES;
    static_assert(RUNS % Q6_WAVES == 0, "proj_down runs");
    const uint32_t valid = (uint32_t)(S - st0) * PDO_STAGE;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int qr = wave + Q6_WAVES * j;
      const uint32_t in_chunk = (uint32_t)(qr * 1024) + 16u * (uint32_t)lane;
      dma16_lds(pbuf, (uint32_t)(uintptr_t)(lds + qr * 1024),
                in_chunk < valid ? (uint32_t)st0 * PDO_STAGE + in_chunk : kOOB, 0u);
    }
  }
  issue_x(0);
  wait_vm_lgkm0_q<4>();  // all but task 0's four copies
  __syncthreads();
  // 2. reciprocals of the factors: thread t holds columns 2t, 2t + 1 of the chunk (CH * 128 columns)
  static_assert(CH * 128 <= 2 * Q6_THREADS, "smoothing columns per thread");
  const int scol = st0 * 128 + 2 * tid;
  const bool s_role = smooth && 2 * tid < CH * 128;
  const uint32_t sv = s_role ? *(const uint32_t*)(lds + SMR_OFF + 4 * tid) : 0u;
  if (s_role) {
    // columns past K (K % 64 == 0: both or neither of the pair) take factor 1: their x is zero
    const float s0 = scol < K ? bf16_lo(sv) : 1.0f, s1 = scol < K ? bf16_hi(sv) : 1.0f;
    float* rcp = (float*)(lds + RCP_OFF);
    const int i = 2 * tid;
    rcp[i] = 1.0f / s0;
    rcp[i + 1] = 1.0f / s1;
    rcp[CH * 128 + i] = s0;
    rcp[CH * 128 + i + 1] = s1;
  }
  if (tid < CH) *(int*)(lds + FLAG_OFF + 4 * tid) = 0;
  __syncthreads();
  if (s_role && scol < K && (!g64::smooth_ok(bf16_lo(sv)) || !g64::smooth_ok(bf16_hi(sv))))
    *(int*)(lds + FLAG_OFF + 4 * (tid / 64)) = 1;   // columns 2t, 2t+1 lie in stage t / 64 of the chunk
  __syncthreads();

  const float s2 = s2p ? *s2p : 1.0f;
  const bool s2_one = s2 == 1.0f;
  const rsrc_t qbuf = make_rsrc(q6, (uint32_t)((int64_t)S * M * GWA_FP6_REC));
  v4f acc[RBX];
#pragma unroll
  for (int rb = 0; rb < RBX; ++rb) acc[rb] = (v4f){0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int t = 0; t < CH; ++t) {
    if (t >= ntask) break;  // workgroup-uniform
    const int st = st0 + t;
    const bool more = t + 1 < ntask;
    if (more) issue_x(t + 1);
    // task t's copies have landed once at most the newer memory operations are in flight: task t - 1's three
    // record stores and task t + 1's four copies (vector memory operations complete in issue order)
    if (t == 0) {
      if (more) wait_vm_lgkm0_q<4>();
      else wait_vm_lgkm0_q<0>();
    } else {
      if (more) wait_vm_lgkm0_q<7>();
      else wait_vm_lgkm0_q<3>();
    }
    asm volatile("" ::: "memory");  // the LDS reads below stay after the wait
    v4i xv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) xv[j] = *(const v4i*)(xring + (t & 1) * X_TASK + r * 256 + 16 * ((4 * c + j) ^ r));
    // ---- xs = RN_bf16(x / smooth) as floats, and the lane's absmax
    float v[32];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[8 * j + 2 * e] = bf16_lo((uint32_t)xv[j][e]);
        v[8 * j + 2 * e + 1] = bf16_hi((uint32_t)xv[j][e]);
      }
    if (smooth) {
      // the stage's flag is workgroup-uniform: one scalar branch, not one per element
      const int divide = __builtin_amdgcn_readfirstlane(*(const int*)(lds + FLAG_OFF + 4 * t));
      const float* f = (const float*)(lds + RCP_OFF) + (divide ? CH * 128 : 0) + t * 128 + 32 * c;
      float fv[32];
#pragma unroll
      for (int i = 0; i < 32; i += 4) *(v4f*)(fv + i) = *(const v4f*)(f + i);
      g64::smooth32(v, fv, divide != 0);
    }
    // group absmax: this lane's half, then the other half in lane ^ 16
    uint32_t mu = g64::absmax_bits32(v);
    mu = max(mu, (uint32_t)__shfl_xor((int)mu, 16));
    g64::v6u pk;
    uint16_t sh;
    g64::quant32(v, mu, row_ok, s2_one, s2, pk, sh);
    // ---- record (stage st, row grow): bytes [24c, 24c + 24) hold this half-group; 96 + 2 g the scale, and
    // the odd lanes zero the record's unused bytes 100..103 (the GEMM reads bytes 96..103 as one operand pair)
    const uint32_t rec = (uint32_t)(((int64_t)st * M + grow) * GWA_FP6_REC);
    // the record lies inside the [S, M, 104] buffer (a row past M stores nothing)
    const bool rec_ok = GWA_DCHECK(!row_ok || (int64_t)rec + GWA_FP6_REC <= (int64_t)S * M * GWA_FP6_REC,
                                   kDbgQuantRec, rec);
    buf_store16((v4i){(int)pk[0], (int)pk[1], (int)pk[2], (int)pk[3]}, qbuf,
                row_ok && rec_ok ? rec + 24u * c : kOOB);
    buf_store8(make_uint2(pk[4], pk[5]), qbuf, row_ok && rec_ok ? rec + 24u * c + 16u : kOOB);
    buf_store2((c & 1) ? (uint16_t)0 : sh, qbuf,
               row_ok && rec_ok ? rec + 96u + (uint32_t)(c & 2) + 4u * (uint32_t)(c & 1) : kOOB);

    // ---- la += x[rows, stage] @ proj_down[stage, :]
    if constexpr (RB > 0) {
      const uint8_t* pb = lds + t * PDO_STAGE + 16 * lane;
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
          acc[rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, xv[j]),
                                                            *(const v8bf*)(pb + (j * RB + rb) * 1024), acc[rb],
                                                            0, 0, 0);
    }
  }
  if constexpr (RB > 0) {
    // lane holds the partial la[row0 + 4c + i][16 rb + r], i = 0..3: slot blockIdx.y of la_part
    const int R = RB * 16;
    float* slot = la_part + (int64_t)blockIdx.y * M * R;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = row0 + 4 * c + i;
        if (m < M) slot[(int64_t)m * R + 16 * rb + r] = acc[rb][i];
      }
  }
}

// la = RN_bf16(sum over p of part[p]) in the order p = 0, 1, ...: one thread per 4 consecutive values, the
// partials loaded 32 at a time (a small-M launch has up to K/128 slots and few threads: the loads of all of
// them go out together, one memory round trip) and added in order.
__global__ __launch_bounds__(256) void la_reduce_kernel(const float* __restrict__ part, int P, int64_t MR,
                                                         uint16_t* __restrict__ la) {
  constexpr int kBatch = 32;
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= MR) return;
  v4f s = (v4f){0.f, 0.f, 0.f, 0.f};
  for (int p0 = 0; p0 < P; p0 += kBatch) {
    v4f v[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
      v[u] = p0 + u < P ? *(const v4f*)(part + (int64_t)(p0 + u) * MR + i) : (v4f){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
      if (p0 + u < P) s = (p0 + u == 0) ? v[u] : s + v[u];
  }
  *(uint2*)(la + i) = make_uint2(pack_bf16x2_rn(s[0], s[1]), pack_bf16x2_rn(s[2], s[3]));
}

// proj_down [K, R] bf16 -> the operand order of svdq_quant_fp6_kernel and of
// the fp6 GEMM's next-layer epilogue: stage-major, per stage 4 k-steps x R/16
// blocks of 64 lanes x 8 values,
// out[(((s * 4 + j) * RB + rb) * 64 + lane) * 8 + e] =
//     proj_down[128 s + 32 (lane / 16) + 8 j + e][16 rb + lane % 16].
__global__ __launch_bounds__(256) void prep_proj_down_fp6_kernel(const uint16_t* __restrict__ pd,
                                                                 uint16_t* __restrict__ out, int K, int R) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int RB = R / 16;
  if (idx >= (int64_t)((K + 127) / 128) * 4 * RB * 64) return;
  const int lane = (int)(idx % 64);
  const int rb = (int)((idx / 64) % RB);
  const int j = (int)((idx / (64 * RB)) % 4);
  const int st = (int)(idx / (64 * RB * 4));
  const int col = rb * 16 + (lane & 15);
  const int k0 = st * 128 + 32 * (lane >> 4) + 8 * j;
  uint16_t v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = k0 + e < K ? pd[(int64_t)(k0 + e) * R + col] : (uint16_t)0;  // a half stage's rows past K: zero
  uint4 o;
  o.x = (uint32_t)v[0] | ((uint32_t)v[1] << 16);
  o.y = (uint32_t)v[2] | ((uint32_t)v[3] << 16);
  o.z = (uint32_t)v[4] | ((uint32_t)v[5] << 16);
  o.w = (uint32_t)v[6] | ((uint32_t)v[7] << 16);
  *(uint4*)(out + idx * 8) = o;
}

// proj_down [K, R] bf16 -> MFMA B-operand order for kernel 1, zero padded to
// a multiple of 256 rows: out[((kc * RB + rb) * 64 + lane) * 8 + e] =
// proj_down[32 kc + 8 (lane / 16) + e][16 rb + lane % 16].
__global__ __launch_bounds__(256) void prep_proj_down_kernel(const uint16_t* __restrict__ pd,
                                                             uint16_t* __restrict__ out, int K, int Kp, int R) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int RB = R / 16;
  if (idx >= (int64_t)(Kp / 32) * RB * 64) return;
  const int lane = (int)(idx % 64);
  const int rb = (int)((idx / 64) % RB);
  const int kc = (int)(idx / (64 * RB));
  const int r = rb * 16 + (lane & 15);
  const int k0 = kc * 32 + (lane >> 4) * 8;
  uint16_t v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = (k0 + e < K) ? pd[(int64_t)(k0 + e) * R + r] : (uint16_t)0;
  uint4 o;
  o.x = (uint32_t)v[0] | ((uint32_t)v[1] << 16);
  o.y = (uint32_t)v[2] | ((uint32_t)v[3] << 16);
  o.z = (uint32_t)v[4] | ((uint32_t)v[5] << 16);
  o.w = (uint32_t)v[6] | ((uint32_t)v[7] << 16);
  *(uint4*)(out + idx * 8) = o;
}

// ---------------------------------------------------------------------------
// int8 activation quantization in the three modes of the reference's W8A8 quantizer: per-token scales from
// each row's |x| maximum, one per-tensor scale from the whole tensor's maximum, or a static scale given by the
// layer. One 256-thread block per row.
// ---------------------------------------------------------------------------
enum { kW8Row = 0, kW8Tensor = 1, kW8Static = 2 };

// |x| maximum of one row (every thread of the block gets it)
__device__ __forceinline__ float w8a8_row_amax(const uint16_t* xr, int nchunk, float* red) {
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
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// Per-tensor maximum: each block folds the maximum of its rows into *amax_bits with an atomic max on the bit
// pattern (non-negative floats order as their bits); w8a8_clear_kernel zeroes the cell first.
__global__ void w8a8_clear_kernel(uint32_t* __restrict__ cell) { *cell = 0u; }

__global__ __launch_bounds__(256) void w8a8_amax_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                        uint32_t* __restrict__ amax_bits, int M, int K) {
  __shared__ float red[4];
  float am = 0.0f;
  for (int row = blockIdx.x; row < M; row += gridDim.x) {
    am = fmaxf(am, w8a8_row_amax(x + (int64_t)row * ldx, K >> 3, red));
    __syncthreads();  // red is reused by the next row
  }
  if (threadIdx.x == 0) atomicMax(amax_bits, __float_as_uint(am));
}

template <int MODE>
__global__ __launch_bounds__(256) void w8a8_quant_int8_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                              int8_t* __restrict__ q, float* __restrict__ sa,
                                                              const float* __restrict__ src, int sa_per_row, int K) {
  __shared__ float red[4];
  const int row = blockIdx.x;
  const uint16_t* xr = x + (int64_t)row * ldx;
  int8_t* qr = q + (int64_t)row * K;
  const int nchunk = K >> 3;
  float s;
  if constexpr (MODE == kW8Row) s = fmaxf(w8a8_row_amax(xr, nchunk, red) / 127.0f, 1e-12f);
  else if constexpr (MODE == kW8Tensor) s = fmaxf(__uint_as_float(*(const uint32_t*)src) / 127.0f, 1e-12f);
  else s = *src;
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
  // one scale per row ([M] output), or the one per-tensor scale ([1] output) from row 0
  if (threadIdx.x == 0 && (sa_per_row || row == 0)) sa[sa_per_row ? row : 0] = s;
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

extern "C" int gwa_svdq_prep_proj_down_fp6(const void* proj_down, void* out, int64_t K, int64_t rank,
                                           void* stream) {
  GWA_REQUIRE(K > 0 && K % 64 == 0 && K < (1ll << 24), "svdq_prep_proj_down_fp6: K=%lld is not a multiple of 64",
              (long long)K);
  GWA_REQUIRE(rank == 16 || rank == 32 || rank == 64 || rank == 128,
              "svdq_prep_proj_down_fp6: rank %lld not in {16,32,64,128}", (long long)rank);
  GWA_REQUIRE(proj_down && out, "svdq_prep_proj_down_fp6: null pointer");
  GWA_REQUIRE(GWA_ALIGNED(proj_down, 2) && GWA_ALIGNED(out, 16), "svdq_prep_proj_down_fp6: out must be 16-byte aligned");
  const int64_t total = ((K + 127) / 128) * 4 * (rank / 16) * 64;
  hipLaunchKernelGGL(prep_proj_down_fp6_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)proj_down, (uint16_t*)out, (int)K, (int)rank);
  return gwa_check_launch("svdq_prep_proj_down_fp6");
}

// stages per workgroup of svdq_quant_fp6_kernel: as many as keep >= 256 workgroups (a workgroup's loads all
// go out at once), with the proj_down operands of a workgroup's stages within 32 KB of LDS
static int quant_fp6_stages_per_group(int64_t M, int64_t K, int64_t R) {
  const int64_t S = (K + 127) / 128, groups = (M + Q6_ROWS - 1) / Q6_ROWS;
  int ch = 4;
  while (ch > 1 && (groups * ((S + ch - 1) / ch) < 256 || ch * (R / 16) > 8)) ch /= 2;
  return ch;
}

extern "C" int64_t gwa_svdq_quant_fp6_partials(int64_t M, int64_t K, int64_t rank) {
  if (M <= 0 || K <= 0 || K % 64 || rank <= 0) return 0;
  const int64_t S = (K + 127) / 128;
  const int ch = quant_fp6_stages_per_group(M, K, rank);
  return (S + ch - 1) / ch;
}

extern "C" int gwa_svdq_la_reduce(const float* part, int64_t P, int64_t M, int64_t rank, void* la, void* stream) {
  GWA_REQUIRE(P >= 1 && M >= 0 && rank % 16 == 0 && rank > 0 && P * M * rank * 4 < (1ll << 40),
              "svdq_la_reduce: bad shape P=%lld M=%lld rank=%lld", (long long)P, (long long)M, (long long)rank);
  if (M == 0) return GWA_OK;
  GWA_REQUIRE(part && la, "svdq_la_reduce: null pointer");
  GWA_REQUIRE(GWA_ALIGNED(part, 16) && GWA_ALIGNED(la, 8), "svdq_la_reduce: part must be 16-byte, la 8-byte aligned");
  const int64_t mr = M * rank, threads = mr / 4;
  hipLaunchKernelGGL(la_reduce_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     part, (int)P, mr, (uint16_t*)la);
  return gwa_check_launch("svdq_la_reduce");
}

extern "C" int64_t gwa_svdq_quant_fp6_la_workspace(int64_t M, int64_t K, int64_t rank) {
  if (M <= 0 || K <= 0 || K % 64 || rank <= 0 || K >= (1ll << 24)) return 0;
  return gwa_svdq_quant_fp6_partials(M, K, rank) * M * rank * 4;
}

extern "C" int gwa_svdq_quant_fp6(const void* x, int64_t ldx, const void* smooth, const float* s2,
                                  const void* proj_down_op6, int64_t rank, uint8_t* q6, float* la_part, int64_t M,
                                  int64_t K, void* stream) {
  const char* what = "svdq_quant_fp6";
  GWA_REQUIRE(M >= 0 && K > 0 && K % 64 == 0, "%s: K=%lld is not a multiple of 64", what, (long long)K);
  GWA_REQUIRE(ldx >= K && ldx % 8 == 0, "%s: row stride %lld must be >= K and a multiple of 8", what,
              (long long)ldx);
  GWA_REQUIRE((proj_down_op6 == nullptr) == (la_part == nullptr),
              "%s: proj_down_op6 and la_part must both be given or both be NULL", what);
  const int64_t R = proj_down_op6 ? rank : 0;
  GWA_REQUIRE(R == 0 || R == 16 || R == 32 || R == 64 || R == 128, "%s: rank %lld not in {0,16,32,64,128}", what,
              (long long)R);
  const int64_t S = (K + 127) / 128;  // K % 128 == 64: a half stage, its second group zero codes
  GWA_REQUIRE(M < (1ll << 31) && K < (1ll << 24) && M * ldx * 2 < (1ll << 31) &&
                  M * S * GWA_FP6_REC < (1ll << 31) && S * R * 256 < (1ll << 31),
              "%s: x and q6 must stay below 2 GiB (buffer addressing)", what);
  if (M == 0) return GWA_OK;
  GWA_REQUIRE(x && q6, "%s: null pointer", what);
  GWA_REQUIRE(GWA_ALIGNED(x, 16) && GWA_ALIGNED(q6, 8) && GWA_ALIGNED(smooth, 4) && GWA_ALIGNED(proj_down_op6, 16) &&
                  GWA_ALIGNED(la_part, 4) && GWA_ALIGNED(s2, 4),
              "%s: x and proj_down_op6 must be 16-byte, q6 8-byte aligned", what);
  const int rb = (int)(R / 16);
  const int64_t groups = (M + Q6_ROWS - 1) / Q6_ROWS;
  const int ch = quant_fp6_stages_per_group(M, K, R);
  const dim3 grid((unsigned)groups, (unsigned)((S + ch - 1) / ch)), block(Q6_THREADS);
  GWA_REQUIRE(groups < (1ll << 31) && grid.y < 65536u, "%s: grid too large", what);
  hipStream_t st = (hipStream_t)stream;
  const uint16_t* xp = (const uint16_t*)x;
  const uint16_t* sm = (const uint16_t*)smooth;
  const uint16_t* pd = (const uint16_t*)proj_down_op6;
  const int m = (int)M, k = (int)K;
#define GWA_Q6_LAUNCH(RBV, CHV) \
  hipLaunchKernelGGL((svdq_quant_fp6_kernel<RBV, CHV>), grid, block, 0, st, xp, ldx, sm, s2, pd, q6, la_part, m, k)
#define GWA_Q6_CH(RBV)                         \
  if (ch == 4) GWA_Q6_LAUNCH(RBV, 4);          \
  else if (ch == 2) GWA_Q6_LAUNCH(RBV, 2);     \
  else GWA_Q6_LAUNCH(RBV, 1);
  switch (rb) {
    case 0: GWA_Q6_CH(0) break;
    case 1: GWA_Q6_CH(1) break;
    case 2: GWA_Q6_CH(2) break;
    case 4:  // ch <= 2 here
      if (ch == 2) GWA_Q6_LAUNCH(4, 2);
      else GWA_Q6_LAUNCH(4, 1);
      break;
    case 8: GWA_Q6_LAUNCH(8, 1); break;  // ch == 1 here
    default: return gwa_set_error(GWA_ERR_INVALID, "%s: rank %lld", what, (long long)R);
  }
#undef GWA_Q6_CH
#undef GWA_Q6_LAUNCH
  return gwa_check_launch(what);
}

extern "C" int gwa_svdq_quant_fp6_la(const void* x, int64_t ldx, const void* smooth, const float* s2,
                                     const void* proj_down_op6, int64_t rank, uint8_t* q6, void* la, float* la_ws,
                                     int64_t la_ws_bytes, int64_t M, int64_t K, void* stream) {
  const char* what = "svdq_quant_fp6_la";
  GWA_REQUIRE(M >= 0 && K > 0 && K % 64 == 0, "%s: K=%lld is not a multiple of 64", what, (long long)K);
  GWA_REQUIRE(rank == 16 || rank == 32 || rank == 64 || rank == 128, "%s: rank %lld not in {16,32,64,128}", what,
              (long long)rank);
  GWA_REQUIRE(M < (1ll << 31) && K < (1ll << 24), "%s: shape too large", what);
  if (M == 0) return GWA_OK;
  GWA_REQUIRE(proj_down_op6 && la, "%s: null pointer", what);
  GWA_REQUIRE(GWA_ALIGNED(la, 8), "%s: la must be 8-byte aligned", what);
  const int64_t slots = gwa_svdq_quant_fp6_partials(M, K, rank);
  GWA_REQUIRE(la_ws && la_ws_bytes >= slots * M * rank * 4, "%s: la workspace of %lld bytes, this shape needs %lld",
              what, (long long)la_ws_bytes, (long long)(slots * M * rank * 4));
  const int rc = gwa_svdq_quant_fp6(x, ldx, smooth, s2, proj_down_op6, rank, q6, la_ws, M, K, stream);
  if (rc != GWA_OK) return rc;
  return gwa_svdq_la_reduce(la_ws, slots, M, rank, la, stream);
}

extern "C" int gwa_svdq_prep_proj_down(const void* proj_down, void* out, int64_t K, int64_t rank, void* stream) {
  GWA_REQUIRE(K > 0 && K % 64 == 0 && K < (1ll << 24), "svdq_prep_proj_down: bad K=%lld", (long long)K);
  GWA_REQUIRE(rank == 16 || rank == 32 || rank == 64 || rank == 128, "svdq_prep_proj_down: rank %lld not in {16,32,64,128}",
              (long long)rank);
  GWA_REQUIRE(proj_down && out, "svdq_prep_proj_down: null pointer");
  GWA_REQUIRE(GWA_ALIGNED(proj_down, 2) && GWA_ALIGNED(out, 16), "svdq_prep_proj_down: out must be 16-byte aligned");
  const int64_t kp = (K + 255) / 256 * 256;
  const int64_t total = (kp / 32) * (rank / 16) * 64;
  hipLaunchKernelGGL(prep_proj_down_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)proj_down, (uint16_t*)out, (int)K, (int)kp, (int)rank);
  return gwa_check_launch("svdq_prep_proj_down");
}

extern "C" int gwa_svdq_quant_int4(const void* x, int64_t ldx, const void* smooth, const float* s2,
                                   const void* proj_down_op, int64_t rank, int out_format, uint8_t* q,
                                   void* scales, void* la, int64_t M, int64_t K, void* stream) {
  GWA_REQUIRE(M >= 0 && K > 0, "svdq_quant_int4: bad shape M=%lld K=%lld", (long long)M, (long long)K);
  GWA_REQUIRE(K % 64 == 0, "svdq_quant_int4: K=%lld is not a multiple of 64", (long long)K);
  GWA_REQUIRE(ldx >= K && ldx % 8 == 0, "svdq_quant_int4: row stride %lld must be >= K and a multiple of 8",
              (long long)ldx);
  GWA_REQUIRE(out_format == GWA_QFMT_INT4,
              "svdq_quant_int4: out_format %d (fp6 operand records come from gwa_svdq_quant_fp6)", out_format);
  GWA_REQUIRE((proj_down_op == nullptr) == (la == nullptr),
              "svdq_quant_int4: proj_down_op and la must both be given or both be NULL");
  const int64_t R = proj_down_op ? rank : 0;
  GWA_REQUIRE(R == 0 || R == 16 || R == 32 || R == 64 || R == 128,
              "svdq_quant_int4: rank %lld not in {0,16,32,64,128}", (long long)R);
  GWA_REQUIRE(M < (1ll << 31) && K < (1ll << 24) && (M * ldx * 2) < (1ll << 31),
              "svdq_quant_int4: x and q must stay below 2 GiB (buffer addressing)");
  if (M == 0) return GWA_OK;
  GWA_REQUIRE(x && q && scales, "svdq_quant_int4: null pointer");
  GWA_REQUIRE(GWA_ALIGNED(x, 16) && GWA_ALIGNED(q, 16) && GWA_ALIGNED(scales, 2) && GWA_ALIGNED(smooth, 4) &&
                  GWA_ALIGNED(proj_down_op, 16) && GWA_ALIGNED(la, 2),
              "svdq_quant_int4: x, q and proj_down_op must be 16-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  const uint16_t* xp = (const uint16_t*)x;
  const uint16_t* sm = (const uint16_t*)smooth;
  const uint16_t* pd = (const uint16_t*)proj_down_op;
  uint16_t* sc = (uint16_t*)scales;
  uint16_t* lp = (uint16_t*)la;
  const int m = (int)M, k = (int)K;
  const int rb = (int)(R / 16);
  const size_t lds = 2 * (size_t)QBUF > (size_t)rb * 8192 ? 2 * (size_t)QBUF : (size_t)rb * 8192;
  const dim3 grid((unsigned)((M + 15) / 16)), block(512);
#define GWA_QUANT_LAUNCH(RBV, PFV)                                                                             \
  hipLaunchKernelGGL((svdq_quant_int4_kernel<RBV, PFV>), grid, block, lds, s, xp, ldx, sm, s2, pd, q, sc, lp, m, k)
  switch (rb) {
    case 0: GWA_QUANT_LAUNCH(0, 4); break;
    case 1: GWA_QUANT_LAUNCH(1, 4); break;
    case 2: GWA_QUANT_LAUNCH(2, 4); break;
    case 4: GWA_QUANT_LAUNCH(4, 3); break;
    case 8: GWA_QUANT_LAUNCH(8, 2); break;
    default: return gwa_set_error(GWA_ERR_INVALID, "svdq_quant_int4: rank %lld not in {0,16,32,64,128}", (long long)R);
  }
#undef GWA_QUANT_LAUNCH
  return gwa_check_launch("svdq_quant_int4");
}

extern "C" int gwa_w8a8_quant(const void* x, int64_t ldx, int8_t* q, float* sa, const float* input_scale,
                              int pertensor, uint32_t* amax_ws, int64_t M, int64_t K, void* stream) {
  const char* what = "w8a8_quant";
  GWA_REQUIRE(M >= 0 && K > 0 && K % 8 == 0, "%s: bad shape M=%lld K=%lld (K %% 8 == 0)", what, (long long)M,
              (long long)K);
  GWA_REQUIRE(ldx >= K && ldx % 8 == 0, "%s: bad row stride %lld", what, (long long)ldx);
  GWA_REQUIRE(M < (1ll << 31) && K < (1ll << 30), "%s: shape too large", what);
  GWA_REQUIRE(pertensor == 0 || pertensor == 1, "%s: pertensor must be 0 or 1", what);
  if (M == 0) return GWA_OK;
  GWA_REQUIRE(x && q && sa, "%s: null pointer", what);
  GWA_REQUIRE(!pertensor || input_scale || amax_ws, "%s: the dynamic per-tensor mode needs amax_ws", what);
  GWA_REQUIRE(GWA_ALIGNED(x, 16) && GWA_ALIGNED(q, 8) && GWA_ALIGNED(sa, 4) && GWA_ALIGNED(input_scale, 4) &&
                  GWA_ALIGNED(amax_ws, 4),
              "%s: x must be 16-byte, q 8-byte and the scales 4-byte aligned", what);
  hipStream_t s = (hipStream_t)stream;
  const uint16_t* xp = (const uint16_t*)x;
  const dim3 grid((unsigned)M), block(256);
  const int per_row = pertensor ? 0 : 1;
  if (input_scale) {
    hipLaunchKernelGGL((w8a8_quant_int8_kernel<kW8Static>), grid, block, 0, s, xp, ldx, q, sa, input_scale, per_row,
                       (int)K);
  } else if (pertensor) {
    hipLaunchKernelGGL(w8a8_clear_kernel, dim3(1), dim3(1), 0, s, amax_ws);
    const unsigned amax_blocks = (unsigned)(M < 2048 ? M : 2048);
    hipLaunchKernelGGL(w8a8_amax_kernel, dim3(amax_blocks), block, 0, s, xp, ldx, amax_ws, (int)M, (int)K);
    hipLaunchKernelGGL((w8a8_quant_int8_kernel<kW8Tensor>), grid, block, 0, s, xp, ldx, q, sa,
                       (const float*)amax_ws, 0, (int)K);
  } else {
    hipLaunchKernelGGL((w8a8_quant_int8_kernel<kW8Row>), grid, block, 0, s, xp, ldx, q, sa, nullptr, 1, (int)K);
  }
  return gwa_check_launch(what);
}

extern "C" int gwa_w8a8_quant_int8(const void* x, int64_t ldx, int8_t* q, float* sa, int64_t M, int64_t K,
                                   void* stream) {
  return gwa_w8a8_quant(x, ldx, q, sa, nullptr, 0, nullptr, M, K, stream);
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
