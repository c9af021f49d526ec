// W8A8 GEMM: int8 MFMA 32x32x32 with int32 accumulation over the whole K and
// the fp32 epilogue acc * sa * sw[n] + bias[n] of torch._scaled_mm: per-token
// activation scales in the rowwise mode (models/w8a8.py:374-378), one scalar in
// the pertensor mode (:366-372, whose weight scale and bias the reference
// applies as two further bf16 ops; here they are fused in fp32).
//
// Same orientation as the W4A4 kernel: A operand = weight rows (n), B operand
// = activation rows (m); accumulator block D[n][m], lane l holds m = l % 32
// and n = 8*(v/4) + 4*(l/32) + (v%4).
#include <atomic>

#include "fp6_gemm_common.h"

namespace {

constexpr int TILE = 128;
constexpr int KT = 128;                 // int8 bytes (= K elements) per row per stage
constexpr int LDS_STRIDE = KT + 16;
constexpr int LDS_TILE = TILE * LDS_STRIDE;
constexpr int LOADS = TILE * KT / 16 / 256;
constexpr int OSTR = TILE * 2 + 8;     // output staging row: 8-byte pad
static_assert(TILE * OSTR <= 2 * LDS_TILE, "output staging fits the weight buffers");

template <int BIAS_DT, bool OUT_F16>  // BIAS_DT: -1 none, else GWA_DT_*
__global__ __launch_bounds__(256) void w8a8_gemm_kernel(const int8_t* __restrict__ qa,
                                                        const int8_t* __restrict__ qw,
                                                        const float* __restrict__ sa,
                                                        const float* __restrict__ sw,
                                                        const void* __restrict__ bias,
                                                        uint16_t* __restrict__ out, int M, int N, int K,
                                                        int sa_row) {
  __shared__ __attribute__((aligned(16))) uint8_t lds_w[2][LDS_TILE];
  __shared__ __attribute__((aligned(16))) uint8_t lds_x[2][LDS_TILE];
  __shared__ __attribute__((aligned(16))) float g_epi[2 * TILE];  // the tile's sw, then its bias as fp32

  const int tiles_n = (N + TILE - 1) / TILE;
  const int tn = blockIdx.x % tiles_n, tm = blockIdx.x / tiles_n;
  const int n0 = tn * TILE, m0 = tm * TILE;
  const int nstages = (K + KT - 1) / KT;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int wn = wave & 1, wm = wave >> 1;
  const int r32 = lane & 31, h = lane >> 5;
  const int t = threadIdx.x;

  v16i acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) acc[a][b] = (v16i){};

  v4i rw[LOADS], rx[LOADS];
  auto load = [&](int stage) {
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
      const int idx = t + j * 256;
      const int row = idx / (KT / 16), c = idx % (KT / 16);
      const int kb = stage * KT + c * 16;
      const bool kin = kb < K;
      rw[j] = (n0 + row < N && kin) ? *(const v4i*)(qw + (int64_t)(n0 + row) * K + kb) : (v4i){0, 0, 0, 0};
      rx[j] = (m0 + row < M && kin) ? *(const v4i*)(qa + (int64_t)(m0 + row) * K + kb) : (v4i){0, 0, 0, 0};
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
      const int idx = t + j * 256;
      const int row = idx / (KT / 16), c = idx % (KT / 16);
      *(v4i*)(lds_w[buf] + row * LDS_STRIDE + c * 16) = rw[j];
      *(v4i*)(lds_x[buf] + row * LDS_STRIDE + c * 16) = rx[j];
    }
  };

  load(0);
  if (t < TILE) {  // the epilogue's per-column constants (published by the next barrier)
    const int n = n0 + t;
    float wv = 0.0f, bv = 0.0f;
    if (n < N) {
      wv = sw[n];
      if (BIAS_DT == GWA_DT_F32) bv = ((const float*)bias)[n];
      if (BIAS_DT == GWA_DT_BF16) bv = bf16_to_f32(((const uint16_t*)bias)[n]);
      if (BIAS_DT == GWA_DT_F16) bv = f16_bits_to_f32(((const uint16_t*)bias)[n]);
    }
    g_epi[t] = wv;
    g_epi[TILE + t] = bv;
  }
  store(0);
  __syncthreads();
  for (int st = 0; st < nstages; ++st) {
    const int buf = st & 1;
    if (st + 1 < nstages) load(st + 1);
    const uint8_t* lw = lds_w[buf];
    const uint8_t* lx = lds_x[buf];
#pragma unroll
    for (int ks = 0; ks < KT / 32; ++ks) {
      v4i a[2], b[2];
#pragma unroll
      for (int bn = 0; bn < 2; ++bn)
        a[bn] = *(const v4i*)(lw + (64 * wn + 32 * bn + r32) * LDS_STRIDE + ks * 32 + 16 * h);
#pragma unroll
      for (int bm = 0; bm < 2; ++bm)
        b[bm] = *(const v4i*)(lx + (64 * wm + 32 * bm + r32) * LDS_STRIDE + ks * 32 + 16 * h);
#pragma unroll
      for (int bn = 0; bn < 2; ++bn)
#pragma unroll
        for (int bm = 0; bm < 2; ++bm)
          acc[bn][bm] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[bn], b[bm], acc[bn][bm], 0, 0, 0);
    }
    if (st + 1 < nstages) store(buf ^ 1);
    __syncthreads();
  }

  // epilogue as in the 256 x 256 kernel: constants from LDS, the packed tile staged in the (free) weight
  // buffers as [m][n] rows, stored as whole row segments
  uint8_t* ob = lds_w[0];
#pragma unroll
  for (int bm = 0; bm < 2; ++bm) {
    const int ml = 64 * wm + 32 * bm + r32, m = m0 + ml;
    const float am = sa[sa_row ? min(m, M - 1) : 0];  // rows past M are computed but never stored
#pragma unroll
    for (int bn = 0; bn < 2; ++bn) {
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        const int nl = 64 * wn + 32 * bn + 8 * qd + 4 * h;
        if (n0 + nl >= N) continue;  // N % 16 == 0: n < N covers n + 3
        const v4f cw = *(const v4f*)(g_epi + nl);
        const v4f cb = *(const v4f*)(g_epi + TILE + nl);
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float y = (float)acc[bn][bm][4 * qd + e] * am * cw[e];
          if (BIAS_DT >= 0) y += cb[e];
          o[e] = y;
        }
        uint2 pk;
        if (OUT_F16) {
          pk.x = pack_f16x2(o[0], o[1]);
          pk.y = pack_f16x2(o[2], o[3]);
        } else {
          pk.x = pack_bf16x2_rn(o[0], o[1]);
          pk.y = pack_bf16x2_rn(o[2], o[3]);
        }
        *(uint2*)(ob + ml * OSTR + nl * 2) = pk;
      }
    }
  }
  __syncthreads();
  // a descriptor over this tile's output span (127 N + 128 elements < 2^28: N < 2^21 is checked on the host)
  const int rows = min(M - m0, TILE), cols = min(N - n0, TILE);
  const rsrc_t obuf = make_rsrc(out + (int64_t)m0 * N + n0, (uint32_t)(((rows - 1) * N + cols) * 2));
  constexpr int CPR = TILE / 8;  // 16-byte chunks per row
#pragma unroll 4
  for (int i = t; i < TILE * CPR; i += 256) {
    const int row = i / CPR, c = i % CPR;
    const uint2 lo = *(const uint2*)(ob + row * OSTR + c * 16);
    const uint2 hi = *(const uint2*)(ob + row * OSTR + c * 16 + 8);
    uint32_t off = row < rows && 8 * c < cols ? (uint32_t)((row * N + 8 * c) * 2) : kOOB;
    if (!GWA_DCHECK(off == kOOB || (int64_t)off + 16 <= (int64_t)((rows - 1) * N + cols) * 2, kDbgW8Out, off))
      off = kOOB;
    buf_store16((v4i){(int)lo.x, (int)lo.y, (int)hi.x, (int)hi.y}, obuf, off);
  }
}

// ---------------------------------------------------------------------------
// 256 x 256 tiles for grids that fill the GPU. Operand delivery is the W4A4 kernels': direct-to-LDS 1 KB
// copies (no staging registers, no ds_write), here into two stage buffers of 128 K-bytes of 256 activation
// rows and 256 weight rows (64 KB each), the next stage's copies in flight while a stage is consumed. A copy
// reads whole 128-byte lines: lane l of a copy takes 16 bytes of row 8 q + l / 8 (eight rows per copy), so
// rows past M or N read zeros through the range-checked per-lane offset and the stage advance rides in the
// scalar offset. In LDS the 16-byte chunk c of row r sits at slot c ^ ((r / 2) % 8) of the row, so the 16
// rows a quarter of a read instruction touches fill all banks. 8 waves form a 2 (n) x 4 (m) grid of
// 128 x 64 wave tiles: per k-step of 32 bytes, 6 operand reads feed 8 int8 MFMAs that accumulate in place.
// The loop is software-pipelined: the reads of k-step s + 1 are issued between the MFMAs of k-step s, and
// at a stage boundary the wave waits for its copies, meets the barrier, issues the copies two stages ahead
// into the buffer just drained and reads the next stage's first k-step under the last k-step's MFMAs.
// ---------------------------------------------------------------------------
constexpr int L_TM = 256, L_TN = 256, L_KS = 128;  // tile rows (m, n); K bytes per stage
constexpr int kCus = 256;                          // MI355X compute units
constexpr int L_REG = 256 * L_KS;                  // one operand region of a stage buffer: 32 KB
constexpr int L_STAGE = 2 * L_REG;                 // activation region, then weight region
constexpr int L_RUNS = L_REG / 1024;               // 1 KB copies per operand and stage: 32
constexpr int L_SLOTS = L_STAGE / 1024 / NWAVES;   // copies per wave and stage: 8 (4 activation, 4 weight)
constexpr int L_OSTR = L_TN * 2 + 8;              // output staging row: 8-byte pad, distinct banks per write
constexpr int L_LDS = 2 * L_STAGE > L_TM * L_OSTR ? 2 * L_STAGE : L_TM * L_OSTR;
static_assert(L_LDS <= kLdsBytes && L_SLOTS * NWAVES * 1024 == L_STAGE, "stage layout");

__device__ __forceinline__ int l_swz(int r) { return (r >> 1) & 7; }

// pins the order of one k-step: MFMA and operand read alternate (6 reads under 8 MFMAs)
__device__ __forceinline__ void pin_kstep() {
#pragma unroll
  for (int i = 0; i < 6; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
  }
  __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
  __builtin_amdgcn_sched_barrier(0);
}

template <int BIAS_DT, bool OUT_F16>
__global__ __launch_bounds__(NTHREADS, 1) void w8a8_gemm_lds_kernel(const int8_t* __restrict__ qa,
                                                                    const int8_t* __restrict__ qw,
                                                                    const float* __restrict__ sa,
                                                                    const float* __restrict__ sw,
                                                                    const void* __restrict__ bias,
                                                                    uint16_t* __restrict__ out, int M, int N, int K,
                                                                    int sa_row) {
  __shared__ __attribute__((aligned(16))) uint8_t g_lds[L_LDS];
  __shared__ __attribute__((aligned(16))) float g_epi[2 * L_TN];  // the tile's sw, then its bias as fp32
  const int tid = threadIdx.x;
  const int tiles_n = (N + L_TN - 1) / L_TN, tiles_m = (M + L_TM - 1) / L_TM;
  int tm, tn;
  if (!xcd_tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn)) return;  // whole workgroup, before any barrier
  const int m0 = tm * L_TM, n0 = tn * L_TN;
  const int nst = K / L_KS;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int wn = wave & 1, wm = wave >> 1;
  const int r32 = lane & 31, h = lane >> 5;

  // descriptors over this tile's rows only (256 K < 2^31 bytes, checked on the host, so kOOB lies past them)
  const v4i xbuf = raw_rsrc(qa + (int64_t)m0 * K, (uint32_t)(min(M - m0, L_TM) * K));
  const v4i wbuf = raw_rsrc(qw + (int64_t)n0 * K, (uint32_t)(min(N - n0, L_TN) * K));
  // copy j of this wave is run q = wave + 8 j of a stage: runs 0..31 carry activation rows, 32..63 weight
  // rows (j < 4: activations); lane -> row 8 (q % 32) + lane / 8 of the region, LDS slot lane % 8
  uint32_t voff[L_SLOTS];
  uint32_t ldst[L_SLOTS];
#pragma unroll
  for (int j = 0; j < L_SLOTS; ++j) {
    const int q = wave + NWAVES * j;
    const bool isx = j < L_SLOTS / 2;
    const int row = 8 * (q % L_RUNS) + (lane >> 3);
    const int chunk = (lane & 7) ^ l_swz(row);
    const bool live = (isx ? m0 : n0) + row < (isx ? M : N);
    voff[j] = live ? (uint32_t)(row * K + 16 * chunk) : kOOB;
    ldst[j] = (uint32_t)(uintptr_t)(g_lds + (isx ? 0 : L_REG) + (q % L_RUNS) * 1024);
  }
  auto issue = [&](int u, int st) __attribute__((always_inline)) {
    // the stage's K bytes lie inside every operand row (the lane offsets are range-checked by the hardware,
    // the stage's scalar offset is not)
    const uint32_t soff = GWA_DCHECK((st + 1) * L_KS <= K, kDbgW8Copy, st * L_KS) ? (uint32_t)(st * L_KS) : 0u;
#pragma unroll
    for (int j = 0; j < L_SLOTS; ++j)
      dma16(j < L_SLOTS / 2 ? xbuf : wbuf, ldst[j] + (uint32_t)(u * L_STAGE), voff[j], soff);
  };

  v16i acc[4][2];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) acc[a][b] = (v16i){};
  // operand rows of this lane: weight block bn row 128 wn + 32 bn + r32, activation block bm row 64 wm + 32 bm + r32
  int wrow[4], xrow[2];
#pragma unroll
  for (int bn = 0; bn < 4; ++bn) wrow[bn] = 128 * wn + 32 * bn + r32;
#pragma unroll
  for (int bm = 0; bm < 2; ++bm) xrow[bm] = 64 * wm + 32 * bm + r32;
  // k-step ks (32 bytes) of a stage buffer: this lane's half h of each operand row
  auto read_ops = [&](const uint8_t* buf, int ks, v4i (&a)[4], v4i (&b)[2]) __attribute__((always_inline)) {
    const int c = 2 * ks + h;
#pragma unroll
    for (int bn = 0; bn < 4; ++bn) a[bn] = *(const v4i*)(buf + L_REG + wrow[bn] * L_KS + 16 * (c ^ l_swz(wrow[bn])));
#pragma unroll
    for (int bm = 0; bm < 2; ++bm) b[bm] = *(const v4i*)(buf + xrow[bm] * L_KS + 16 * (c ^ l_swz(xrow[bm])));
  };
  auto mma = [&](const v4i (&a)[4], const v4i (&b)[2]) __attribute__((always_inline)) {
#pragma unroll
    for (int bn = 0; bn < 4; ++bn)
#pragma unroll
      for (int bm = 0; bm < 2; ++bm)
        acc[bn][bm] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[bn], b[bm], acc[bn][bm], 0, 0, 0);
  };
  // k-steps 1..3 of a stage, each read under the previous k-step's MFMAs; leaves k-step 3 in (a1, b1)
  v4i a0[4], b0[2], a1[4], b1[2];
  auto stage_body = [&](const uint8_t* buf) __attribute__((always_inline)) {
    read_ops(buf, 1, a1, b1);
    mma(a0, b0);
    pin_kstep();
    read_ops(buf, 2, a0, b0);
    mma(a1, b1);
    pin_kstep();
    read_ops(buf, 3, a1, b1);
    mma(a0, b0);
    pin_kstep();
  };

  issue(0, 0);
  // the epilogue's per-column constants, once per tile (the first barrier publishes them)
  if (tid < L_TN) {
    const int n = n0 + tid;
    float wv = 0.0f, bv = 0.0f;
    if (n < N) {
      wv = sw[n];
      if (BIAS_DT == GWA_DT_F32) bv = ((const float*)bias)[n];
      if (BIAS_DT == GWA_DT_BF16) bv = bf16_to_f32(((const uint16_t*)bias)[n]);
      if (BIAS_DT == GWA_DT_F16) bv = f16_bits_to_f32(((const uint16_t*)bias)[n]);
    }
    g_epi[tid] = wv;
    g_epi[L_TN + tid] = bv;
  }
  wait_vm_lgkm0<0>();
  barrier_lds();
  if (1 < nst) issue(1, 1);
  read_ops(g_lds, 0, a0, b0);
  for (int st = 0; st < nst - 1; ++st) {
    stage_body(g_lds + (st & 1) * L_STAGE);
    // stage st + 1's copies (this wave's: the only ones in flight) and this wave's reads of stage st are
    // complete; after the barrier everyone's are, so buffer st & 1 takes the copies of stage st + 2
    wait_vm_lgkm0<0>();
    barrier_lds();
    if (st + 2 < nst) issue(st & 1, st + 2);
    __builtin_amdgcn_sched_barrier(0);
    read_ops(g_lds + ((st + 1) & 1) * L_STAGE, 0, a0, b0);
    mma(a1, b1);
    pin_kstep();
  }
  stage_body(g_lds + ((nst - 1) & 1) * L_STAGE);
  mma(a1, b1);

  // epilogue: y = acc * sa[m] * sw[n] + bias[n] (sw and bias from the tile's LDS copy: per-element global
  // loads of them would cost the texture path two 64-lane instructions per output pair), packed to 16 bits and
  // staged in LDS as [m][n] rows of OSTR
  // bytes (the stage buffers are free once every wave has passed the barrier), then stored as whole row
  // segments, consecutive threads on consecutive 16-byte chunks of a row (a 32-row column of 8-byte pieces
  // per store instruction, as the accumulator layout gives, spreads every store over 32 rows of the output)
  uint8_t* ob = g_lds;
  barrier_lds();
#pragma unroll
  for (int bm = 0; bm < 2; ++bm) {
    const int ml = 64 * wm + 32 * bm + r32, m = m0 + ml;
    const float am = sa[sa_row ? min(m, M - 1) : 0];  // rows past M are computed but never stored
#pragma unroll
    for (int bn = 0; bn < 4; ++bn) {
#pragma unroll
      for (int qd = 0; qd < 4; ++qd) {
        const int nl = 128 * wn + 32 * bn + 8 * qd + 4 * h, n = n0 + nl;
        if (n >= N) continue;  // N % 16 == 0: n < N covers n + 3
        const v4f cw = *(const v4f*)(g_epi + nl);
        const v4f cb = *(const v4f*)(g_epi + L_TN + nl);
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float y = (float)acc[bn][bm][4 * qd + e] * am * cw[e];
          if (BIAS_DT >= 0) y += cb[e];
          o[e] = y;
        }
        uint2 pk;
        if (OUT_F16) {
          pk.x = pack_f16x2(o[0], o[1]);
          pk.y = pack_f16x2(o[2], o[3]);
        } else {
          pk.x = pack_bf16x2_rn(o[0], o[1]);
          pk.y = pack_bf16x2_rn(o[2], o[3]);
        }
        *(uint2*)(ob + ml * L_OSTR + nl * 2) = pk;
      }
    }
  }
  barrier_lds();
  // a descriptor over this tile's output span (255 N + 256 elements < 2^29: N < 2^21 is checked on the host)
  const int rows = min(M - m0, L_TM), cols = min(N - n0, L_TN);
  const rsrc_t obuf = make_rsrc(out + (int64_t)m0 * N + n0, (uint32_t)(((rows - 1) * N + cols) * 2));
  constexpr int CPR = L_TN / 8;  // 16-byte chunks per row
#pragma unroll 4
  for (int i = tid; i < L_TM * CPR; i += NTHREADS) {
    const int row = i / CPR, c = i % CPR;
    const uint2 lo = *(const uint2*)(ob + row * L_OSTR + c * 16);
    const uint2 hi = *(const uint2*)(ob + row * L_OSTR + c * 16 + 8);
    uint32_t off = row < rows && 8 * c < cols ? (uint32_t)((row * N + 8 * c) * 2) : kOOB;
    if (!GWA_DCHECK(off == kOOB || (int64_t)off + 16 <= (int64_t)((rows - 1) * N + cols) * 2, kDbgW8Out, off))
      off = kOOB;
    buf_store16((v4i){(int)lo.x, (int)lo.y, (int)hi.x, (int)hi.y}, obuf, off);
  }
}

std::atomic<int> g_w8a8_force_tile{-1};  // test / tuning hook (gwa_w8a8_gemm_force_tile)

using W8Kernel = void (*)(const int8_t*, const int8_t*, const float*, const float*, const void*, uint16_t*, int, int,
                          int, int);

template <int BD>
W8Kernel pick_kernel(int tile, bool f16) {
  if (tile == GWA_W8A8_TILE_256x256) return f16 ? w8a8_gemm_lds_kernel<BD, true> : w8a8_gemm_lds_kernel<BD, false>;
  return f16 ? w8a8_gemm_kernel<BD, true> : w8a8_gemm_kernel<BD, false>;
}

// 256 x 256 tiles when their rounds over the CUs finish first: a 256 x 256 tile takes about 2.7 times as
// long as a 128 x 128 one (four times the work at a higher rate: 50 us against 18.3 us at K = 3072), so the
// choice compares ceil(tiles / CUs) rounds of each; 128-byte stages need K % 128 == 0, and the per-tile
// descriptors 256 K < 2^31
int w8a8_tile(int64_t M, int64_t N, int64_t K) {
  if (K % L_KS || K >= (1ll << 23)) return GWA_W8A8_TILE_128x128;
  const int forced = g_w8a8_force_tile.load(std::memory_order_relaxed);
  if (forced >= 0) return forced;
  const int64_t big = ((M + L_TM - 1) / L_TM) * ((N + L_TN - 1) / L_TN);
  const int64_t small = ((M + TILE - 1) / TILE) * ((N + TILE - 1) / TILE);
  const int64_t rounds_big = (big + kCus - 1) / kCus, rounds_small = (small + kCus - 1) / kCus;
  return 27 * rounds_big < 10 * rounds_small ? GWA_W8A8_TILE_256x256 : GWA_W8A8_TILE_128x128;
}

}  // namespace

extern "C" int gwa_w8a8_gemm_tile(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return -1;
  return w8a8_tile(M, N, K);
}

extern "C" int gwa_w8a8_gemm_force_tile(int tile) {
  return g_w8a8_force_tile.exchange(tile == GWA_W8A8_TILE_128x128 || tile == GWA_W8A8_TILE_256x256 ? tile : -1);
}

extern "C" int gwa_w8a8_gemm(const int8_t* qa, const int8_t* qw, const float* sa, int64_t sa_numel,
                             const float* sw, const void* bias, int bias_dtype, void* out, int out_dtype, int64_t M,
                             int64_t N, int64_t K, void* stream) {
  GWA_REQUIRE(M >= 0 && N > 0 && K > 0, "w8a8_gemm: bad shape M=%lld N=%lld K=%lld", (long long)M, (long long)N,
              (long long)K);
  GWA_REQUIRE(K % 64 == 0, "w8a8_gemm: K=%lld is not a multiple of 64", (long long)K);
  GWA_REQUIRE(N % 16 == 0, "w8a8_gemm: N=%lld is not a multiple of 16", (long long)N);
  GWA_REQUIRE(out_dtype == GWA_DT_BF16 || out_dtype == GWA_DT_F16, "w8a8_gemm: out_dtype %d not bf16/f16",
              out_dtype);
  GWA_REQUIRE(bias == nullptr || bias_dtype == GWA_DT_BF16 || bias_dtype == GWA_DT_F16 || bias_dtype == GWA_DT_F32,
              "w8a8_gemm: bias_dtype %d", bias_dtype);
  GWA_REQUIRE(M < (1ll << 31) && N < (1ll << 21) && K < (1ll << 30), "w8a8_gemm: shape too large");
  if (M == 0) return GWA_OK;
  GWA_REQUIRE(sa_numel == 1 || sa_numel == M, "w8a8_gemm: sa has %lld values for M=%lld (1 or M)",
              (long long)sa_numel, (long long)M);
  GWA_REQUIRE(qa && qw && sa && sw && out, "w8a8_gemm: null pointer");
  GWA_REQUIRE(GWA_ALIGNED(qa, 16) && GWA_ALIGNED(qw, 16) && GWA_ALIGNED(out, 8) && GWA_ALIGNED(sa, 4) &&
                  GWA_ALIGNED(sw, 4) && GWA_ALIGNED(bias, 2),
              "w8a8_gemm: qa/qw must be 16-byte and out 8-byte aligned");
  const int64_t tiles = ((M + TILE - 1) / TILE) * ((N + TILE - 1) / TILE);
  GWA_REQUIRE(tiles < (1ll << 31), "w8a8_gemm: too many tiles");
  hipStream_t s = (hipStream_t)stream;
  const bool f16 = out_dtype == GWA_DT_F16;
  uint16_t* op = (uint16_t*)out;
  const int m = (int)M, n = (int)N, k = (int)K, sr = sa_numel == M && M > 1 ? 1 : 0;
  const int tile = w8a8_tile(M, N, K);
  const bool lds = tile != GWA_W8A8_TILE_128x128;
  const int64_t big = ((M + L_TM - 1) / L_TM) * ((N + L_TN - 1) / L_TN);
  const int64_t per_xcd = (big + kXcds - 1) / kXcds;
  const dim3 grid(lds ? (unsigned)(per_xcd * kXcds) : (unsigned)tiles), block(lds ? NTHREADS : 256);
  const int bd = bias ? bias_dtype : -1;
  W8Kernel kern = nullptr;
  if (bd == -1) kern = pick_kernel<-1>(tile, f16);
  else if (bd == GWA_DT_F32) kern = pick_kernel<GWA_DT_F32>(tile, f16);
  else if (bd == GWA_DT_BF16) kern = pick_kernel<GWA_DT_BF16>(tile, f16);
  else kern = pick_kernel<GWA_DT_F16>(tile, f16);
  hipLaunchKernelGGL(kern, grid, block, 0, s, qa, qw, sa, sw, bias, op, m, n, k, sr);
  return gwa_check_launch("w8a8_gemm");
}
